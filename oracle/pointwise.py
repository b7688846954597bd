"""CPU oracle: RMSNorm, add-RMSNorm, q/k head-norm + RoPE + KV write, SiLU*mul, RoPE tables.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  All arithmetic is float32 on the
CPU with the reference's bf16 rounding points made explicit.
"""
from __future__ import annotations

import torch


def _r(t: torch.Tensor) -> torch.Tensor:
    """Round float32 through bf16 (the reference's ``.to(bf16).to(f32)``)."""
    return t.bfloat16().float()


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """``bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)`` -- ``src/moss_tts/_runtime/kernels.py:50-59``
    (Qwen3RMSNorm, transformers ``modeling_qwen3.py:59-64``)."""
    f = x.float()
    r = torch.rsqrt(f.pow(2).mean(-1, keepdim=True) + eps)
    return (_r(f * r) * w.float()).bfloat16()


def add_rmsnorm(x: torch.Tensor, res: torch.Tensor, w: torch.Tensor, eps: float):
    """``s = bf16(x + res)``, ``y = rmsnorm(s)`` -- ``src/moss_tts/_runtime/kernels.py:69-82``."""
    s = (x.float() + res.float()).bfloat16()
    return s, rmsnorm(s, w, eps)


def silu_mul(x: torch.Tensor) -> torch.Tensor:
    """``[.., 2n] -> [.., n]``: ``bf16(bf16(g / (1 + exp(-g))) * u)`` --
    ``src/moss_tts/_runtime/prefill_pointwise.py:120-130`` (mode 0) and ``kernels.py:124-129``."""
    n = x.shape[-1] // 2
    g = x[..., :n].float()
    u = x[..., n:].float()
    return (_r(g / (1.0 + torch.exp(-g))) * u).bfloat16()


def rope_tables(positions: torch.Tensor, theta: float = 1e6, dim: int = 128):
    """cos/sin bf16 ``[n, dim]`` as Qwen3RotaryEmbedding computes them
    (transformers ``modeling_qwen3.py:106-138``): ``inv_freq = 1/theta^(2i/dim)`` in fp32,
    ``freqs = pos * inv_freq``, ``emb = cat(freqs, freqs)``, cos/sin in fp32 then bf16."""
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float) / dim))
    freqs = positions.float()[:, None] @ inv[None, :]
    emb = torch.cat([freqs, freqs], -1)
    return emb.cos().bfloat16(), emb.sin().bfloat16()


def qk_norm_rope_kv(qkv: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, positions: torch.Tensor,
                    eps: float) -> torch.Tensor:
    """Per head of 128: ``r = rsqrt(sum x^2 / 128 + eps)``, ``xn = bf16(bf16(x r) w[d])``,
    ``out = bf16(bf16(xn cos) + bf16(+-xn[(d+64)%128] sin))`` (minus for d < 64, float
    negation); K rows go to ``kc[:, :, pos]``, V rows are copied to ``vc[:, :, pos]``
    (in place).  Returns q ``[n, 32, 128]`` bf16.
    ``src/moss_tts/_runtime/kernels.py:142-170``, ``src/moss_tts/_runtime/prefill_qkv.py:7-28``.
    """
    n = qkv.shape[0]
    x = qkv.float().view(n, 48, 128)
    heads = x[:, :40]
    w = torch.cat([qw.float().expand(32, 128), kw.float().expand(8, 128)])[None]
    r = torch.rsqrt(heads.pow(2).sum(-1, keepdim=True) / 128 + eps)
    xn = _r(_r(heads * r) * w)
    xs = torch.cat([-xn[..., 64:], xn[..., :64]], -1)
    c = cos.float().view(n, 1, 128)
    s = sin.float().view(n, 1, 128)
    out = (_r(xn * c) + _r(xs * s)).bfloat16()
    for t in range(n):
        p = int(positions[t])
        kc[0, :, p] = out[t, 32:40]
        vc[0, :, p] = qkv[t].view(48, 128)[40:48]
    return out[:, :32].contiguous()
