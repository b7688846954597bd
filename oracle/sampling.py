"""CPU oracle: decode-step sampling and next-id composition.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference anchors
-----------------
* ``sample_topk`` -- ``src/moss_tts/_runtime/llm.py:10-19``: temperature <= 0 gives
  ``logits.argmax(-1)`` (first maximal index); otherwise ``torch.topk(logits.float() / T, k)``
  (values descending), ``softmax``, entries with ``cumsum - p > top_p`` set to 0, then
  ``torch.multinomial``.  Here the draw is made explicit: with a uniform ``u`` in [0, 1), the first
  kept index whose cumulative probability exceeds ``u * sum(kept)``; ties in value keep the lower
  index first.
* The next-id composition -- ``src/moss_tts/_runtime/llm.py:280-287``.
* The per-step state update of the in-audio loop -- ``src/moss_tts/_runtime/streaming.py:107-112``
  (inside the first 32 steps after the audio start: ``first_audio_graph.py:14-29``).
* Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy as 1, 2, 3",
  SC 2011): the counter-based generator the kernels draw ``u`` from, with counter
  ``(position low, position high, row, salt)`` and key ``(seed low, seed high)``.

Pinning (tests/test_oracle_sampling.py): Philox against the published known-answer vectors of the
Random123 distribution; the top-k set and order against ``torch.topk`` on distinct values and the
argmax against ``torch.argmax``; the probabilities against ``torch.softmax``; the u-inversion against
``torch.multinomial`` frequencies and against the exact probabilities (chi-square bound); the
composition against a direct loop restating the reference's two ``torch.where`` lines; the state
update by its closed forms over token sequences (the delay counter equals the steps since the first
delay-slot token, inclusive; the audio length counts the start / gen-slot / delay-slot tokens) and,
composed with the composition, by the audio end appearing exactly 32 steps after the first delay
slot.
"""
from __future__ import annotations

import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK = 0xFFFFFFFF


def philox4x32_10(counter, key):
    """counter: 4 uint32, key: 2 uint32 -> 4 uint32 (Python ints)."""
    c = [int(v) & MASK for v in counter]
    k = [int(v) & MASK for v in key]
    for r in range(10):
        if r:
            k = [(k[0] + W0) & MASK, (k[1] + W1) & MASK]
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        c = [((p1 >> 32) ^ c[1] ^ k[0]) & MASK, p1 & MASK, ((p0 >> 32) ^ c[3] ^ k[1]) & MASK, p0 & MASK]
    return c


def uniform(seed: int, position: int, row: int, salt: int = 0) -> np.float32:
    """The kernels' u for one (position, row): the top 24 bits of Philox word 0, times 2^-24."""
    out = philox4x32_10([position & MASK, (position >> 32) & MASK, row, salt], [seed & MASK, (seed >> 32) & MASK])
    return np.float32((out[0] >> 8) * (1.0 / 16777216.0))


def topk(values: np.ndarray, k: int):
    """Indices and values of the k largest, descending; equal values keep the lower index first."""
    order = np.lexsort((np.arange(values.size), -values.astype(np.float64)))
    idx = order[:k]
    return idx, values[idx]


def sample_row(logits_bf16_as_f32: np.ndarray, temperature: float, top_k: int, top_p: float, u):
    """One row of ``sample_topk`` with an explicit uniform ``u``.  Returns (index, kept probabilities,
    their index order) -- the last two for boundary checks."""
    x = np.asarray(logits_bf16_as_f32, dtype=np.float32)
    if not temperature > 0:
        return int(np.argmax(x)), None, None
    v = (x / np.float32(temperature)).astype(np.float32)
    idx, vals = topk(v, top_k)
    e = np.exp((vals - vals[0]).astype(np.float32)).astype(np.float32)
    s = np.float32(0)
    for t in e:
        s = np.float32(s + t)
    probs = np.empty_like(e)
    cum = np.float32(0)
    total = np.float32(0)
    for i, t in enumerate(e):
        q = np.float32(t / s)
        cum = np.float32(cum + q)
        if np.float32(cum - q) > np.float32(top_p):
            q = np.float32(0)
        probs[i] = q
        total = np.float32(total + q)
    target = np.float32(np.float32(u) * total)
    acc = np.float32(0)
    pick = 0
    for i, q in enumerate(probs):
        if q > 0:
            pick = i
        acc = np.float32(acc + q)
        if q > 0 and acc > target:
            break
    return int(idx[pick]), probs, idx


def sample_topk(logits: np.ndarray, temperature: float, top_k: int, top_p: float, *, seed: int, position: int,
                salt: int = 0, vocab: int | None = None) -> np.ndarray:
    """Rows of bf16 logits (as float32 values) -> int64 indices, as ``moss_sample_topk``."""
    logits = np.atleast_2d(np.asarray(logits, dtype=np.float32))
    vocab = logits.shape[1] if vocab is None else vocab
    out = np.empty(logits.shape[0], dtype=np.int64)
    for r in range(logits.shape[0]):
        u = uniform(seed, position, r, salt)
        out[r] = sample_row(logits[r, :vocab], temperature, top_k, top_p, u)[0]
    return out


def compose_next_ids(text_index: int, audio_index, text_ids, audio_length: int, delay_length: int,
                     delay_slot_id: int, audio_end_id: int, pad_code: int = 1024) -> np.ndarray:
    """``llm.py:281-287``: the text token with the delay overrides, the audio codes masked by channel."""
    tok = int(text_ids[text_index])
    if delay_length >= 0:
        tok = delay_slot_id
    if delay_length == 32:
        tok = audio_end_id
    audio = np.asarray(audio_index, dtype=np.int64)
    c = np.arange(audio.size)
    valid = (c < audio_length) & ((delay_length < 0) | (c >= delay_length))
    return np.concatenate([[tok], np.where(valid, audio, pad_code)]).astype(np.int64)


def advance_state(next_ids, position: int, audio_length: int, delay_length: int, *, audio_start_id: int,
                  gen_slot_id: int, delay_slot_id: int):
    """``streaming.py:107-112`` for one in-audio step: the next ids become the input ids, the
    position advances, the audio length grows on the start / gen-slot / delay-slot tokens, the delay
    counter starts at the first delay-slot token and then counts every step.  Returns
    (ids, position, audio_length, delay_length, status)."""
    ids = np.asarray(next_ids, dtype=np.int64).copy()
    text = int(ids[0])
    if text in (audio_start_id, gen_slot_id, delay_slot_id):
        audio_length += 1
    if delay_length < 0 and text == delay_slot_id:
        delay_length = 0
    if delay_length >= 0:
        delay_length += 1
    position += 1
    return ids, position, audio_length, delay_length, np.array([text, audio_length, delay_length, position],
                                                               dtype=np.int64)
