"""RMSNorm, q/k head-norm + RoPE + KV write, and SiLU*mul on the gfx950 library.

Interfaces mirror the reference's Python operators: ``rmsnorm(x, weight, eps)`` and
``add_rmsnorm(x, residual, weight, eps) -> (summed, normalized)``
(``src/moss_tts/_runtime/kernels.py:62-90``), ``qk_rope(qkv, q_weight, k_weight, cos, sin,
keys, values, positions, eps) -> q`` (``src/moss_tts/_runtime/prefill_qkv.py:61-83``), and
``silu_mul(x)`` (``src/moss_tts/_runtime/kernels.py:132-139``).
"""
from __future__ import annotations

import torch

from . import native
from .w4g32 import _aligned, _cuda_contig, _require


def _norm_common(x: torch.Tensor, weight: torch.Tensor):
    _cuda_contig("x", x, torch.bfloat16)
    _cuda_contig("weight", weight, torch.bfloat16, x.device)
    n = x.shape[-1]
    _require(weight.numel() == n, f"weight must have {n} values")
    _require(n % 8 == 0 and n <= 8192, "hidden size must be a multiple of 8 and <= 8192")
    _require(_aligned(x, 16) and _aligned(weight, 16), "x and weight must be 16-byte aligned")
    return n, x.numel() // n


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    n, rows = _norm_common(x, weight)
    y = torch.empty_like(x)
    native.call("moss_rmsnorm", native.ptr(x), None, native.ptr(weight), None, native.ptr(y), rows, n,
                float(eps), native.stream_of(x))
    return y


def add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """Returns ``(summed, normalized)`` with ``summed = bf16(x + residual)``."""
    n, rows = _norm_common(x, weight)
    _cuda_contig("residual", residual, torch.bfloat16, x.device)
    _require(residual.shape == x.shape, "residual must match x")
    _require(_aligned(residual, 16), "residual must be 16-byte aligned")
    summed = torch.empty_like(x)
    y = torch.empty_like(x)
    native.call("moss_rmsnorm", native.ptr(x), native.ptr(residual), native.ptr(weight), native.ptr(summed),
                native.ptr(y), rows, n, float(eps), native.stream_of(x))
    return summed, y


QH, KH, HD = 32, 8, 128
QKV = (QH + 2 * KH) * HD


def qk_rope(qkv: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor, cos: torch.Tensor,
            sin: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, positions: torch.Tensor,
            eps: float, *, cos_by_position: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """q/k head RMSNorm + RoPE for ``n`` tokens; writes K/V rows ``positions`` of the cache
    in place and returns ``q`` as ``[1, 32, n, 128]`` (a transposed view, like the reference).

    ``cos``/``sin`` hold one row per token, or with ``cos_by_position`` a whole ``[L, 128]``
    table indexed by each token's (device-side) position.  Positions are device values and are not
    checked here: the kernel clamps one outside ``[0, L)`` to the nearest row, so it overwrites
    that row rather than memory beyond the cache.  ``out``: a contiguous bf16 buffer of
    ``n * 32 * 128`` values to write ``q`` into (``[1, n, 32, 128]`` order)."""
    _cuda_contig("qkv", qkv, torch.bfloat16)
    dev = qkv.device
    _require(qkv.shape[-1] == QKV, f"Qwen3-8B QKV rows of {QKV} required")
    n = qkv.numel() // QKV
    L = keys.shape[2] if keys.ndim == 4 else 0
    for name, t in (("cos", cos), ("sin", sin)):
        _cuda_contig(name, t, torch.bfloat16, dev)
        rows = L if cos_by_position else n
        _require(t.numel() == rows * HD, f"{name} must hold {rows} rows of {HD}")
    for name, t in (("q_weight", q_weight), ("k_weight", k_weight)):
        _cuda_contig(name, t, torch.bfloat16, dev)
        _require(t.numel() == HD, f"{name} must hold {HD} values")
    for name, t in (("keys", keys), ("values", values)):
        _cuda_contig(name, t, torch.bfloat16, dev)
    _require(keys.shape == values.shape and keys.ndim == 4 and tuple(keys.shape[:2]) == (1, KH)
             and keys.shape[3] == HD, "matching [1, 8, L, 128] KV buffers required")
    _cuda_contig("positions", positions, torch.int64, dev)
    _require(positions.numel() == n, "one int64 position per token required")
    _require(n <= L, "more tokens than KV rows")
    if out is not None:
        _cuda_contig("out", out, torch.bfloat16, dev)
        _require(out.numel() == n * QH * HD, f"out must hold {n * QH * HD} values")
        q = out.view(1, n, QH, HD)
    else:
        q = torch.empty((1, n, QH, HD), device=dev, dtype=torch.bfloat16)
    native.call("moss_qk_norm_rope_kv", native.ptr(qkv), native.ptr(q_weight), native.ptr(k_weight),
                native.ptr(cos), native.ptr(sin), native.ptr(q), native.ptr(keys), native.ptr(values),
                native.ptr(positions), L, n, float(eps), int(bool(cos_by_position)), native.stream_of(qkv))
    return q.transpose(1, 2)


def silu_mul(x: torch.Tensor) -> torch.Tensor:
    """``[..., 2n]`` (gate | up) -> ``[..., n]`` with ``bf16(bf16(silu(g)) * u)``."""
    _cuda_contig("x", x, torch.bfloat16)
    _require(x.shape[-1] % 4 == 0, "gate/up width must be a multiple of 4")
    n = x.shape[-1] // 2
    rows = x.numel() // x.shape[-1]
    y = torch.empty((*x.shape[:-1], n), device=x.device, dtype=torch.bfloat16)
    native.call("moss_silu_mul", native.ptr(x), native.ptr(y), rows, n, native.stream_of(x))
    return y
