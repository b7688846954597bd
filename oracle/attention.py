"""CPU oracle: GQA decode attention over a static KV cache, and the embedding sum.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import math

import torch

SCALE = 1.0 / math.sqrt(128.0)


def decode_attention(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, position: int) -> torch.Tensor:
    """One query token against cache rows ``[0, position]`` in fp32, exact softmax.

    ``q [32, 128]`` bf16, caches ``[1, 8, L, 128]`` bf16 (query head h reads KV head h // 4),
    scale ``1/sqrt(128)``.  Returns fp32 ``[32, 128]``.  The reference splits this into
    32-token blocks with a log-sum-exp merge (``src/moss_tts/_runtime/kernels.py:173-208``);
    a split softmax equals the whole one up to fp32 rounding.
    """
    k = kc[0, :, : position + 1].float()                       # [8, T, 128]
    v = vc[0, :, : position + 1].float()
    qh = q.float().view(8, 4, 128)                              # KV head, its 4 query heads
    s = torch.einsum("gjd,gtd->gjt", qh, k) * SCALE
    p = torch.softmax(s, dim=-1)
    return torch.einsum("gjt,gtd->gjd", p, v).reshape(32, 128)


def prefill_attention(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, start: int) -> torch.Tensor:
    """Causal attention of the prompt pass: ``q [n, 32, 128]`` bf16 for the tokens at absolute positions
    ``start .. start + n - 1``; token t attends cache rows ``0 .. start + t`` of ``[1, 8, L, 128]``
    caches (query head h reads KV head h // 4), fp32 scores scaled by ``1/sqrt(128)``, exact softmax.
    Returns fp32 ``[n, 32, 128]``.  The reference runs ``F.scaled_dot_product_attention(...,
    is_causal=True, enable_gqa=True)`` on the cache rows its prefill wrote
    (``src/moss_tts/_runtime/llm.py:116-128``)."""
    n = q.shape[0]
    end = int(start) + n
    k = kc[0, :, :end].float()                                  # [8, T, 128]
    v = vc[0, :, :end].float()
    qh = q.float().view(n, 8, 4, 128).permute(1, 2, 0, 3)      # [8, 4, n, 128]
    s = torch.matmul(qh, k[:, None].transpose(-1, -2)) * SCALE  # [8, 4, n, T]
    visible = torch.arange(end)[None, :] <= (int(start) + torch.arange(n))[:, None]
    s = s.masked_fill(~visible, float("-inf"))
    out = torch.matmul(torch.softmax(s, dim=-1), v[:, None])     # [8, 4, n, 128]
    return out.permute(2, 0, 1, 3).reshape(n, 32, 128).contiguous()


def embedding_sum(ids: torch.Tensor, text: torch.Tensor, audio: torch.Tensor) -> torch.Tensor:
    """``ids [33]`` = text token, 32 audio codes; ``x = text[ids[0]]`` then
    ``x = bf16(x + audio[q, ids[q+1]])`` for q = 0..31 in order (bf16 after every add,
    ``src/moss_tts/_runtime/kernels.py:7-18``).  Returns bf16 ``[4096]``; ``ids [T, 33]`` gives
    ``[T, 4096]``."""
    if ids.dim() == 2:
        return torch.stack([embedding_sum(row, text, audio) for row in ids])
    x = text[int(ids[0])].float()
    for qi in range(audio.shape[0]):
        x = (x + audio[qi, int(ids[qi + 1])].float()).bfloat16().float()
    return x.bfloat16()
