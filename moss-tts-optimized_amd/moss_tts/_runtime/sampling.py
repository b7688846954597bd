"""Decode-step sampling on the gfx950 library.

``sample_topk(logits, temperature=1.7, top_k=25, top_p=0.8)`` keeps the reference's signature and
meaning (``src/moss_tts/_runtime/llm.py:10-19``); the random draw comes from a counter-based
Philox4x32-10 keyed by ``seed`` and indexed by the device-side ``position`` and the row, so a
captured decode graph samples fresh values at every position.  The key is read from a device
buffer when the kernel runs (``seed_buffer``), so each request can set its own seed without
recapturing.  ``compose_next_ids`` is the token logic of the reference's ``_decode``
(``llm.py:280-287``).  ``advance_step`` is the host loop's per-step update
(``src/moss_tts/_runtime/streaming.py:107-112``) on the device, so several decode steps can be
captured in one graph (``src/moss_tts/_runtime/first_audio_graph.py:14-29``).
"""
from __future__ import annotations

import torch

from . import native
from .w4g32 import _cuda_contig, _require

MAX_TOP_K = 64
MAX_VOCAB = 2048
_U64 = 0xFFFFFFFFFFFFFFFF


def seed_value(seed: int) -> int:
    """A 64-bit seed as the signed int64 whose bits the sampler reads as its Philox key."""
    _require(isinstance(seed, int), "seed must be an int")
    u = int(seed) & _U64
    return u - (1 << 64) if u >= 1 << 63 else u


def seed_buffer(seed: int, device) -> torch.Tensor:
    """A device int64 ``[1]`` holding ``seed``'s 64 bits: the sampler's key buffer."""
    return torch.full((1,), seed_value(seed), dtype=torch.int64, device=device)


def sample_topk(logits: torch.Tensor, temperature: float = 1.7, top_k: int = 25, top_p: float = 0.8, *,
                seed: int | torch.Tensor = 0, position: torch.Tensor | None = None, salt: int = 0,
                vocab: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 logits ``[rows, stride]`` (or ``[stride]``) -> int64 indices ``[rows]`` into the first
    ``vocab`` entries of each row.  ``seed``: an int, or a device int64 ``[1]`` buffer read when the
    kernel runs (what a captured graph uses)."""
    _cuda_contig("logits", logits, torch.bfloat16)
    rows = 1 if logits.dim() == 1 else logits.shape[0]
    stride = logits.shape[-1]
    vocab = stride if vocab is None else int(vocab)
    _require(0 < vocab <= min(stride, MAX_VOCAB), f"vocab must be in [1, min(stride, {MAX_VOCAB})]")
    if temperature > 0:
        _require(1 <= top_k <= min(MAX_TOP_K, vocab), f"top_k must be in [1, min({MAX_TOP_K}, vocab)]")
    if position is None:
        position = torch.zeros(1, dtype=torch.int64, device=logits.device)
    _cuda_contig("position", position, torch.int64, logits.device)
    _require(position.numel() == 1, "position holds one value")
    if not isinstance(seed, torch.Tensor):
        seed = seed_buffer(seed, logits.device)
    _cuda_contig("seed", seed, torch.int64, logits.device)
    _require(seed.numel() == 1, "seed holds one value")
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    else:
        _cuda_contig("out", out, torch.int64, logits.device)
        _require(out.numel() == rows, f"out must hold {rows} indices")
    native.call("moss_sample_topk", native.ptr(logits), rows, stride, vocab, float(temperature), int(top_k),
                float(top_p), native.ptr(seed), native.ptr(position), int(salt), native.ptr(out),
                native.stream_of(logits))
    return out


def _sample_set(logits, temperature, top_k, top_p, vocab, out):
    _cuda_contig("logits", logits, torch.bfloat16)
    rows = 1 if logits.dim() == 1 else logits.shape[0]
    stride = logits.shape[-1]
    vocab = stride if vocab is None else int(vocab)
    _require(0 < vocab <= min(stride, MAX_VOCAB), f"vocab must be in [1, min(stride, {MAX_VOCAB})]")
    if temperature > 0:
        _require(1 <= top_k <= min(MAX_TOP_K, vocab), f"top_k must be in [1, min({MAX_TOP_K}, vocab)]")
    _cuda_contig("out", out, torch.int64, logits.device)
    _require(out.numel() == rows, f"out must hold {rows} indices")
    return (native.ptr(logits), rows, stride, vocab, float(temperature), int(top_k), float(top_p))


def sample_topk_pair(a: dict, b: dict, *, seed: torch.Tensor, position: torch.Tensor) -> None:
    """Two :func:`sample_topk` calls sharing ``seed`` and ``position`` in one launch (the decode
    step's text row and audio rows, ``llm.py:280,284``); each of ``a`` and ``b`` holds ``logits``,
    ``temperature``, ``top_k``, ``top_p``, ``salt``, ``out`` and optionally ``vocab``.  The outputs
    equal the two separate calls'."""
    sets = []
    for d in (a, b):
        head = _sample_set(d["logits"], d["temperature"], d["top_k"], d["top_p"], d.get("vocab"), d["out"])
        _require(d["logits"].device == a["logits"].device, "both sets on one device")
        sets.append(head + (int(d["salt"]), native.ptr(d["out"])))
    dev = a["logits"].device
    for name, t in (("seed", seed), ("position", position)):
        _cuda_contig(name, t, torch.int64, dev)
        _require(t.numel() == 1, f"{name} holds one value")
    native.call("moss_sample_topk_pair", *sets[0], *sets[1], native.ptr(seed), native.ptr(position),
                native.stream_of(a["logits"]))


def compose_next_ids(text_index: torch.Tensor, audio_index: torch.Tensor, text_ids: torch.Tensor,
                     audio_length: torch.Tensor, delay_length: torch.Tensor, *, delay_slot_id: int,
                     audio_end_id: int, pad_code: int = 1024, out: torch.Tensor | None = None) -> torch.Tensor:
    """int64 ``[1 + channels]``: the next text token and audio codes (``llm.py:280-287``)."""
    dev = audio_index.device
    for name, t in (("text_index", text_index), ("audio_index", audio_index), ("text_ids", text_ids),
                    ("audio_length", audio_length), ("delay_length", delay_length)):
        _cuda_contig(name, t, torch.int64, dev)
    _require(text_ids.numel() == 2, "text_ids holds the gen-slot and delay-slot ids")
    channels = audio_index.numel()
    _require(0 < channels <= 64, "at most 64 channels")
    if out is None:
        out = torch.empty(1 + channels, dtype=torch.int64, device=dev)
    native.call("moss_compose_next_ids", native.ptr(text_index), native.ptr(audio_index), native.ptr(text_ids),
                native.ptr(audio_length), native.ptr(delay_length), int(delay_slot_id), int(audio_end_id),
                channels, int(pad_code), native.ptr(out), native.stream_of(audio_index))
    return out


def advance_step(next_ids: torch.Tensor, ids: torch.Tensor, position: torch.Tensor, audio_length: torch.Tensor,
                 delay_length: torch.Tensor, *, step: int = 0, history: torch.Tensor | None = None,
                 status: torch.Tensor | None = None, audio_start_id: int, gen_slot_id: int,
                 delay_slot_id: int) -> None:
    """In place: ``ids <- next_ids`` (and ``history[step]``), position + 1, the audio length and delay
    counter advanced by the text token ``next_ids[0]``; ``status = (text, length, delay, position)``."""
    dev = next_ids.device
    for name, t in (("next_ids", next_ids), ("ids", ids), ("position", position), ("audio_length", audio_length),
                    ("delay_length", delay_length)):
        _cuda_contig(name, t, torch.int64, dev)
    width = next_ids.numel()
    _require(0 < width <= 64 and ids.numel() == width, "ids and next_ids must hold the same 1..64 ids")
    _require(next_ids.data_ptr() != ids.data_ptr(), "next_ids and ids must be distinct buffers")
    for name, t in (("position", position), ("audio_length", audio_length), ("delay_length", delay_length)):
        _require(t.numel() == 1, f"{name} holds one value")
    if history is not None:
        _cuda_contig("history", history, torch.int64, dev)
        _require(history.dim() == 2 and history.shape[1] == width and 0 <= step < history.shape[0],
                 "history must be [steps, width] with 0 <= step < steps")
    else:
        _require(step >= 0, "step must be non-negative")
    if status is not None:
        _cuda_contig("status", status, torch.int64, dev)
        _require(status.numel() == 4, "status holds 4 values")
    native.call("moss_advance_step", native.ptr(next_ids), native.ptr(ids), native.ptr(position),
                native.ptr(audio_length), native.ptr(delay_length), native.ptr(history) if history is not None else None,
                native.ptr(status) if status is not None else None, int(step), width, int(audio_start_id),
                int(gen_slot_id), int(delay_slot_id), native.stream_of(next_ids))
