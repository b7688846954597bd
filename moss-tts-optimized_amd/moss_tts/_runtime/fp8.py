"""FP8 E4M3 (OCP) weight-only linear on the gfx950 library.

``fp8_silu_decode(x, weight, scale=None)`` keeps the reference's signature and meaning
(``src/moss_tts/_runtime/fused_mlp.py:26-30``): ``weight`` is e4m3 ``[2n, K]`` (gate rows
first), ``scale`` an optional fp32 ``[2n]``, output bf16 ``[..., n]`` from the first row of
``x`` (the reference reads only its first row; here exactly one row is required).  ``linear(x, weight, scale)`` is the plain
projection for any number of rows (GEMV for one row, MFMA GEMM for more).  Weights may be
passed as ``torch.float8_e4m3fn`` or as their ``uint8`` bit patterns.
"""
from __future__ import annotations

import torch

from . import native
from .w4g32 import _aligned, _cuda_contig, _require

_MAX_GEMV_K = 16384


def _weight_bytes(weight: torch.Tensor) -> torch.Tensor:
    _require(isinstance(weight, torch.Tensor), "weight must be a tensor")
    _require(weight.dtype in (torch.float8_e4m3fn, torch.uint8), "weight must be float8_e4m3fn (or its uint8 bits)")
    w = weight.view(torch.uint8)
    _cuda_contig("weight", w, torch.uint8)
    _require(w.ndim == 2, "weight must be 2-D [out, in]")
    _require(_aligned(w, 16), "weight must be 16-byte aligned")
    return w


def _scale_arg(scale, rows: int, device):
    if scale is None:
        return None
    _cuda_contig("scale", scale, torch.float32, device)
    _require(scale.numel() == rows, f"scale must hold {rows} fp32 values")
    return native.ptr(scale)


def linear(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor | None = None, *,
           rows_per_wave: int = 0) -> torch.Tensor:
    """``bf16(s[n] * sum_k f32(w[n, k]) x[.., k])``: bf16 ``[..., K]`` -> bf16 ``[..., N]``."""
    w = _weight_bytes(weight)
    n, k = w.shape
    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.shape[-1] == k, f"x must end in a dimension of {k}")
    _require(_aligned(x, 16), "x must be 16-byte aligned")
    _require(rows_per_wave in (0, 1, 2, 4), "rows_per_wave must be 0 (auto), 1, 2 or 4")
    m = x.numel() // k
    _require(m > 0, "empty input")
    if m == 1:
        _require(k % 16 == 0 and k <= _MAX_GEMV_K, f"decode GEMV needs K % 16 == 0 and K <= {_MAX_GEMV_K}")
    else:
        _require(k % 64 == 0, "the prefill GEMM needs K % 64 == 0")
    s = _scale_arg(scale, n, w.device)
    y = torch.empty((*x.shape[:-1], n), dtype=torch.bfloat16, device=x.device)
    wp, wb, _keep = native.gemm_workspace(m, k, n, x.device) if m > 1 else (None, 0, None)
    native.call("moss_fp8_linear", native.ptr(x), native.ptr(w), s, native.ptr(y), m, k, n, rows_per_wave, wp, wb,
                native.stream_of(x))
    return y


def fp8_silu_decode(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor | None = None, *,
                    rows_per_wave: int = 0) -> torch.Tensor:
    """Fused gate||up decode GEMV with ``bf16(silu(bf16(gate))) * bf16(up)`` stored as bf16."""
    w = _weight_bytes(weight)
    n2, k = w.shape
    _require(n2 % 2 == 0, "gate||up weight needs an even number of rows")
    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.shape[-1] == k and x.numel() == k, f"one contiguous bf16 row of {k} values required")
    _require(k % 16 == 0 and k <= _MAX_GEMV_K, f"decode GEMV needs K % 16 == 0 and K <= {_MAX_GEMV_K}")
    _require(_aligned(x, 16), "x must be 16-byte aligned")
    _require(rows_per_wave in (0, 1, 2, 4), "rows_per_wave must be 0 (auto), 1, 2 or 4")
    s = _scale_arg(scale, n2, w.device)
    y = torch.empty((*x.shape[:-1], n2 // 2), dtype=torch.bfloat16, device=x.device)
    native.call("moss_fp8_gateup_silu", native.ptr(x), native.ptr(w), s, native.ptr(y), 1, k, n2 // 2,
                rows_per_wave, native.stream_of(x))
    return y


def to_bf16(weight: torch.Tensor) -> torch.Tensor:
    """Exact e4m3 -> bf16 conversion of a whole weight (the conversion the kernels use)."""
    w = _weight_bytes(weight)
    _require(w.numel() % 4 == 0, "element count must be a multiple of 4")
    out = torch.empty(w.shape, dtype=torch.bfloat16, device=w.device)
    native.call("moss_fp8_to_bf16", native.ptr(w), native.ptr(out), w.numel(), native.stream_of(w))
    return out
