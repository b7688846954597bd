"""Decode and prefill attention over the static bf16 KV cache, and the embedding sum.

``decode_attention`` mirrors the reference's decode path after q/k-norm + RoPE
(``src/moss_tts/_runtime/kernels.py:211-251``, native launcher
``src/moss_tts/_runtime/attention_native.py:31-44``): validation raises ``ValueError``,
the split workspaces are caller-owned or allocated with ``torch.empty``, launches go to the
current stream.  ``prefill_attention`` replaces the causal ``scaled_dot_product_attention`` of the
prompt pass (``src/moss_tts/_runtime/llm.py:116-128``).  ``embedding_sum`` mirrors
``src/moss_tts/_runtime/kernels.py:21-26``.
"""
from __future__ import annotations

import functools

import torch

from . import native, w4a8
from .w4g32 import _aligned, _cuda_contig, _require

QH, KH, HD = 32, 8, 128


@functools.lru_cache(maxsize=None)
def splits(L: int) -> int:
    return int(native.lib().moss_decode_attention_splits(int(L)))


def workspace(L: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """(partial fp32 [32, S, 128], lse fp32 [32, S]) for a cache of ``L`` rows; calls that
    share a workspace must not overlap (one stream, or one graph)."""
    s = splits(L)
    return (torch.empty((QH, s, HD), device=device, dtype=torch.float32),
            torch.empty((QH, s), device=device, dtype=torch.float32))


def decode_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, position: torch.Tensor,
                     *, out: torch.Tensor | None = None, ws=None) -> torch.Tensor:
    """One decode token: ``q`` bf16 (32*128 values), ``keys``/``values`` bf16 ``[1, 8, L, 128]``
    (one layer, L a multiple of 64), ``position`` int64 ``[1]`` on the device.  Returns bf16
    ``[1, 1, 4096]``."""
    _cuda_contig("q", q, torch.bfloat16)
    dev = q.device
    _require(q.numel() == QH * HD, f"q must hold {QH}x{HD} values")
    for name, t in (("keys", keys), ("values", values)):
        _cuda_contig(name, t, torch.bfloat16, dev)
    _require(keys.shape == values.shape and keys.ndim == 4 and tuple(keys.shape[:2]) == (1, KH)
             and keys.shape[3] == HD, "matching [1, 8, L, 128] KV buffers required")
    _cuda_contig("position", position, torch.int64, dev)
    _require(position.numel() == 1, "one int64 position required")
    _require(_aligned(keys, 16) and _aligned(values, 16), "KV buffers must be 16-byte aligned")
    L = keys.shape[2]
    _require(L % 64 == 0 and L <= 32768, "the cache length must be a multiple of 64, at most 32768")
    partial, lse = ws if ws is not None else workspace(L, dev)
    _require(partial.numel() >= QH * splits(L) * HD and lse.numel() >= QH * splits(L), "workspace too small")
    if out is None:
        out = torch.empty((1, 1, QH * HD), device=dev, dtype=torch.bfloat16)
    native.call("moss_decode_attention", native.ptr(q), native.ptr(keys), native.ptr(values), native.ptr(position),
                native.ptr(partial), native.ptr(lse), native.ptr(out), L, native.stream_of(q))
    return out


def decode_attention_qkv(qkv: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, position: torch.Tensor,
                         eps: float, *, out: torch.Tensor | None = None, ws=None, quantize: bool = False,
                         out_activation=None):
    """q/k head-norm + RoPE + KV-cache write + decode attention in one pass
    (``src/moss_tts/_runtime/kernels.py:211-251``): ``qkv`` bf16 (6144 values: q | k | v),
    head-norm weights bf16 [128], cos/sin bf16 ``[L, 128]`` tables indexed by the device
    position; K/V row ``position`` of the cache is written.  Returns bf16 ``[1, 1, 4096]``,
    bit-identical to ``qk_rope`` followed by ``decode_attention``.  ``quantize``: the merge also
    forms the int8 groups of 32 of that output for a W4A8 projection and ``(out, activation)`` is
    returned (``src/moss_tts/_runtime/attention_quant.py:8-32``)."""
    _cuda_contig("qkv", qkv, torch.bfloat16)
    dev = qkv.device
    _require(qkv.numel() == (QH + 2 * KH) * HD, "one q||k||v row of 6144 values required")
    for name, t in (("keys", keys), ("values", values)):
        _cuda_contig(name, t, torch.bfloat16, dev)
    _require(keys.shape == values.shape and keys.ndim == 4 and tuple(keys.shape[:2]) == (1, KH)
             and keys.shape[3] == HD, "matching [1, 8, L, 128] KV buffers required")
    L = keys.shape[2]
    _require(L % 64 == 0 and L <= 32768, "the cache length must be a multiple of 64, at most 32768")
    for name, t in (("q_norm", q_norm), ("k_norm", k_norm)):
        _cuda_contig(name, t, torch.bfloat16, dev)
        _require(t.numel() == HD, f"{name} must hold {HD} values")
    for name, t in (("cos", cos), ("sin", sin)):
        _cuda_contig(name, t, torch.bfloat16, dev)
        _require(t.numel() == L * HD, f"{name} must be an [L, {HD}] table")
    _cuda_contig("position", position, torch.int64, dev)
    _require(position.numel() == 1, "one int64 position required")
    _require(_aligned(keys, 16) and _aligned(values, 16), "KV buffers must be 16-byte aligned")
    partial, lse = ws if ws is not None else workspace(L, dev)
    _require(partial.numel() >= QH * splits(L) * HD and lse.numel() >= QH * splits(L), "workspace too small")
    if out is None:
        out = torch.empty((1, 1, QH * HD), device=dev, dtype=torch.bfloat16)
    else:
        _cuda_contig("out", out, torch.bfloat16, dev)
        _require(out.numel() == QH * HD, f"out must hold {QH * HD} values")
    if not quantize:
        _require(out_activation is None, "out_activation needs quantize=True")
        native.call("moss_decode_attention_qkv", native.ptr(qkv), native.ptr(q_norm), native.ptr(k_norm),
                    native.ptr(cos), native.ptr(sin), native.ptr(keys), native.ptr(values), native.ptr(position),
                    native.ptr(partial), native.ptr(lse), native.ptr(out), L, float(eps), native.stream_of(qkv))
        return out
    act = out_activation if out_activation is not None else w4a8.empty_activation(QH * HD, dev)
    w4a8._check_activation(act, QH * HD, dev)
    native.call("moss_decode_attention_qkv_quant", native.ptr(qkv), native.ptr(q_norm), native.ptr(k_norm),
                native.ptr(cos), native.ptr(sin), native.ptr(keys), native.ptr(values), native.ptr(position),
                native.ptr(partial), native.ptr(lse), native.ptr(out), native.ptr(act.qx), native.ptr(act.scales),
                native.ptr(act.sums), L, float(eps), native.stream_of(qkv))
    return out, act


def prefill_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, start: torch.Tensor, *,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal attention of ``n`` prompt tokens: ``q`` bf16 ``[n, 32, 128]`` (``[1, n, 32, 128]`` as
    ``qk_rope`` writes it), the tokens at positions ``start .. start + n - 1`` (``start`` int64 ``[1]``
    on the device) with their K/V rows already in ``keys``/``values`` ``[1, 8, L, 128]``.  Returns bf16
    ``[n, 4096]``."""
    _cuda_contig("q", q, torch.bfloat16)
    dev = q.device
    _require(q.numel() % (QH * HD) == 0 and q.numel() > 0, f"q must hold n x {QH} x {HD} values")
    n = q.numel() // (QH * HD)
    for name, t in (("keys", keys), ("values", values)):
        _cuda_contig(name, t, torch.bfloat16, dev)
    _require(keys.shape == values.shape and keys.ndim == 4 and tuple(keys.shape[:2]) == (1, KH)
             and keys.shape[3] == HD, "matching [1, 8, L, 128] KV buffers required")
    L = keys.shape[2]
    _require(L % 64 == 0 and L <= 32768, "the cache length must be a multiple of 64, at most 32768")
    _require(n <= L, "more prompt tokens than KV rows")
    _require(_aligned(q, 16) and _aligned(keys, 16) and _aligned(values, 16), "q and KV buffers must be 16-byte aligned")
    _cuda_contig("start", start, torch.int64, dev)
    _require(start.numel() == 1, "one int64 start position required")
    if out is None:
        out = torch.empty((n, QH * HD), device=dev, dtype=torch.bfloat16)
    else:
        _cuda_contig("out", out, torch.bfloat16, dev)
        _require(out.numel() == n * QH * HD, f"out must hold {n * QH * HD} values")
    native.call("moss_prefill_attention", native.ptr(q), native.ptr(keys), native.ptr(values), native.ptr(start),
                native.ptr(out), n, L, native.stream_of(q))
    return out


def embedding_sum(ids: torch.Tensor, text_weight: torch.Tensor, audio_weight: torch.Tensor) -> torch.Tensor:
    """``ids`` int64 ``[..., Q+1]`` -> bf16 ``[..., H]``: text row plus the Q codebook rows,
    rounded to bf16 after every addition."""
    _cuda_contig("ids", ids, torch.int64)
    dev = ids.device
    _cuda_contig("text_weight", text_weight, torch.bfloat16, dev)
    _cuda_contig("audio_weight", audio_weight, torch.bfloat16, dev)
    _require(text_weight.ndim == 2 and audio_weight.ndim == 3, "text [V, H] and audio [Q, V, H] tables required")
    q = audio_weight.shape[0]
    _require(ids.shape[-1] == q + 1, f"ids must end in a dimension of {q + 1}")
    h = text_weight.shape[1]
    _require(audio_weight.shape[2] == h, "text and audio widths differ")
    t = ids.numel() // (q + 1)
    out = torch.empty((*ids.shape[:-1], h), device=dev, dtype=torch.bfloat16)
    native.call("moss_embedding_sum", native.ptr(ids), native.ptr(text_weight), native.ptr(audio_weight),
                native.ptr(out), t, h, text_weight.shape[0], audio_weight.shape[1], q, native.stream_of(ids))
    return out
