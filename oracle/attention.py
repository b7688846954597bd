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


def embedding_sum(ids: torch.Tensor, text: torch.Tensor, audio: torch.Tensor) -> torch.Tensor:
    """``ids [33]`` = text token, 32 audio codes; ``x = text[ids[0]]`` then
    ``x = bf16(x + audio[q, ids[q+1]])`` for q = 0..31 in order (bf16 after every add,
    ``src/moss_tts/_runtime/kernels.py:7-18``).  Returns bf16 ``[4096]``."""
    x = text[int(ids[0])].float()
    for qi in range(audio.shape[0]):
        x = (x + audio[qi, int(ids[qi + 1])].float()).bfloat16().float()
    return x.bfloat16()
