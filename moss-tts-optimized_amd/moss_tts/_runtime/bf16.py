"""bf16-weight decode GEMV on the gfx950 library: the output heads.

The reference keeps the 32 audio-codebook heads and the two text-head rows in bf16 and applies them
with ``F.linear`` (``src/moss_tts/_runtime/llm.py:188-191,270-279``; its Triton GEMV
``linear_decode``, ``src/moss_tts/_runtime/kernels.py:93-108``): ``y = bf16(sum f32(w) f32(x))``.
Validation, allocation and error conventions follow ``w4g32``.
"""
from __future__ import annotations

import torch

from . import native
from .w4g32 import _aligned, _cuda_contig, _require

_KC = (1, 2, 3, 4, 5, 6, 7, 8, 12, 16)       # K / 512 values the kernel is built for


def _check(x: torch.Tensor, w: torch.Tensor, rows_per_wave: int) -> tuple[int, int]:
    _cuda_contig("w", w, torch.bfloat16)
    _require(w.ndim == 2, "w must be [N, K]")
    n, k = w.shape
    _require(k % 512 == 0 and k // 512 in _KC, f"K must be 512 * one of {_KC}, got {k}")
    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.numel() == k, f"one contiguous bf16 row of {k} values required, got shape {tuple(x.shape)}")
    _require(_aligned(x, 16) and _aligned(w, 16), "x and w must be 16-byte aligned")
    _require(rows_per_wave in (0, 1, 2, 4), "rows_per_wave must be 0 (auto), 1, 2 or 4")
    return n, k


def _out(x, n, out):
    if out is None:
        return torch.empty((*x.shape[:-1], n), dtype=torch.bfloat16, device=x.device)
    _cuda_contig("out", out, torch.bfloat16, x.device)
    _require(out.numel() == n, f"out must hold {n} values")
    return out


def gemv(x: torch.Tensor, w: torch.Tensor, *, rows_per_wave: int = 0, out: torch.Tensor | None = None):
    """``F.linear(x, w)`` for one bf16 row ``[..., K]`` and bf16 ``w [N, K]`` -> ``[..., N]``."""
    n, k = _check(x, w, rows_per_wave)
    y = _out(x, n, out)
    native.call("moss_bf16_gemv", native.ptr(x), native.ptr(w), native.ptr(y), k, n, rows_per_wave,
                native.stream_of(x))
    return y


def norm_gemv(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, w: torch.Tensor, *,
              residual: torch.Tensor | None = None, rows_per_wave: int = 0, out: torch.Tensor | None = None):
    """``gemv(rmsnorm(x))`` in one kernel; with ``residual``: ``s = bf16(x + residual)``, returns
    ``(s, gemv(rmsnorm(s)))`` -- the decode step's final norm and heads."""
    n, k = _check(x, w, rows_per_wave)
    _require(k % 2048 == 0 and k <= 8192, "the fused norm needs K % 2048 == 0 and K <= 8192")
    _cuda_contig("norm_weight", norm_weight, torch.bfloat16, w.device)
    _require(norm_weight.numel() == k and _aligned(norm_weight, 16), f"norm_weight must be an aligned row of {k}")
    summed = None
    if residual is not None:
        _cuda_contig("residual", residual, torch.bfloat16, w.device)
        _require(residual.numel() == k and _aligned(residual, 16), f"residual must be an aligned row of {k}")
        summed = torch.empty_like(x)
    y = _out(x, n, out)
    native.call("moss_bf16_norm_gemv", native.ptr(x), native.ptr(residual) if residual is not None else None,
                native.ptr(norm_weight), native.ptr(summed) if summed is not None else None, float(eps),
                native.ptr(w), native.ptr(y), k, n, rows_per_wave, native.stream_of(x))
    return y if summed is None else (summed, y)
