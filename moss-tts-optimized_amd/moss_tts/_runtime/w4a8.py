"""W4A8 G32 decode mode on the gfx950 library: bf16 activations quantized to int8 per group of
32, integer dot products against the row-packed INT4 codes, fp32 group combine -- the
reference's serving arithmetic.

``linear`` mirrors ``src/moss_tts/_runtime/dp4a_scaled.py:80-95`` (``linear(x, packed, scales,
*, paired, fused, prequantized)``): ``x`` is quantized on the device unless ``prequantized``
is given; ``paired`` selects the gate||up SiLU*mul epilogue; ``fused`` also quantizes that
output for the next projection and returns ``(out, activation)``.  ``norm_quant`` mirrors
``src/moss_tts/_runtime/dp4a_fusions.py:53-62``.  Errors follow the other operators: caller
mistakes raise ``ValueError`` before any launch, launches go to the current stream.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import native
from .w4g32 import GROUP, PackedW4G32, _aligned, _cuda_contig, _require

_MAX_K = 16384
_DOT4_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)


@dataclass(frozen=True)
class QuantizedActivation:
    """int8 activations of one row: ``qx int8 [K]`` in dot4 order (bytes ``8b..8b+7`` hold
    ``x[8b + (0, 4, 1, 5, 2, 6, 3, 7)]``), ``scales fp32 [K/32]``, ``sums int32 [K/32]``."""

    qx: torch.Tensor
    scales: torch.Tensor
    sums: torch.Tensor

    @property
    def K(self) -> int:
        return self.qx.numel()

    def natural(self) -> torch.Tensor:
        """The codes in natural order, int8 ``[K]`` (the reference's ``Q`` tensor)."""
        out = torch.empty_like(self.qx).view(-1, 8)
        out[:, list(_DOT4_ORDER)] = self.qx.view(-1, 8)
        return out.view(-1)


def empty_activation(k: int, device) -> QuantizedActivation:
    _require(k % GROUP == 0, f"K must be a multiple of {GROUP}")
    return QuantizedActivation(torch.empty(k, dtype=torch.int8, device=device),
                               torch.empty(k // GROUP, dtype=torch.float32, device=device),
                               torch.empty(k // GROUP, dtype=torch.int32, device=device))


def _check_activation(a: QuantizedActivation, k: int, device) -> None:
    _require(isinstance(a, QuantizedActivation), "prequantized must be a QuantizedActivation")
    _cuda_contig("qx", a.qx, torch.int8, device)
    _cuda_contig("scales", a.scales, torch.float32, device)
    _cuda_contig("sums", a.sums, torch.int32, device)
    _require(a.qx.numel() == k and a.scales.numel() == k // GROUP and a.sums.numel() == k // GROUP,
             f"prequantized activation must cover K = {k}")
    _require(_aligned(a.qx, 16), "qx must be 16-byte aligned")


def quantize(x: torch.Tensor, *, out: QuantizedActivation | None = None) -> QuantizedActivation:
    """bf16 row ``[K]`` -> int8 groups of 32 (``src/moss_tts/_runtime/int4_dp4a.py:21-30``)."""
    _cuda_contig("x", x, torch.bfloat16)
    k = x.numel()
    _require(k % GROUP == 0 and _aligned(x, 16), "x must be a 16-byte aligned row with K % 32 == 0")
    a = out if out is not None else empty_activation(k, x.device)
    _check_activation(a, k, x.device)
    native.call("moss_int8_quantize_g32", native.ptr(x), native.ptr(a.qx), native.ptr(a.scales),
                native.ptr(a.sums), k, native.stream_of(x))
    return a


def norm_quant(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float, *,
               normalized: bool = True, out: QuantizedActivation | None = None):
    """(add+)RMSNorm with the moss_rmsnorm rounding points, then the int8 group quantizer.

    Returns ``(summed, y, activation)`` like the reference (``summed`` is ``x`` without a
    residual; ``y`` is ``None`` when ``normalized`` is false)."""
    _cuda_contig("x", x, torch.bfloat16)
    _cuda_contig("weight", weight, torch.bfloat16, x.device)
    n = x.shape[-1]
    rows = x.numel() // n
    _require(weight.numel() == n, f"weight must have {n} values")
    _require(n % GROUP == 0 and n <= 8192, "hidden size must be a multiple of 32 and <= 8192")
    _require(_aligned(x, 16) and _aligned(weight, 16), "x and weight must be 16-byte aligned")
    _require(rows == 1 or out is None, "out is for one row")
    summed = x
    if residual is not None:
        _cuda_contig("residual", residual, torch.bfloat16, x.device)
        _require(residual.shape == x.shape and _aligned(residual, 16), "residual must match x")
        summed = torch.empty_like(x)
    y = torch.empty_like(x) if normalized else None
    if out is None:
        a = QuantizedActivation(torch.empty(x.shape, dtype=torch.int8, device=x.device),
                                torch.empty(rows * n // GROUP, dtype=torch.float32, device=x.device),
                                torch.empty(rows * n // GROUP, dtype=torch.int32, device=x.device))
    else:
        a = out
        _check_activation(a, n, x.device)
    native.call("moss_rmsnorm_quant_g32", native.ptr(x), native.ptr(residual) if residual is not None else None,
                native.ptr(weight), native.ptr(summed) if residual is not None else None,
                native.ptr(y) if y is not None else None, native.ptr(a.qx), native.ptr(a.scales), native.ptr(a.sums),
                rows, n, float(eps), native.stream_of(x))
    return summed, y, a


def norm_linear(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, w: PackedW4G32, *,
                residual: torch.Tensor | None = None, paired: bool = False, rows_per_wave: int = 0):
    """(add+)RMSNorm, the int8 group quantizer and the W4A8 projection in one kernel
    (``src/moss_tts/_runtime/dp4a_norm_projection.py:48-166``): ``y``, or ``(summed, y)`` with
    ``residual``; bit-identical to ``norm_quant`` followed by ``linear(prequantized=...)``."""
    _require(isinstance(w, PackedW4G32), "w must be a PackedW4G32")
    k = w.K
    _require(k in (2048, 4096, 8192), "the fused norm needs K in {2048, 4096, 8192}")
    _require(rows_per_wave in (0, 1, 2, 4), "rows_per_wave must be 0 (auto), 1, 2 or 4")
    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.numel() == k and _aligned(x, 16), f"one aligned bf16 row of {k} values required")
    _cuda_contig("norm_weight", norm_weight, torch.bfloat16, w.device)
    _require(norm_weight.numel() == k and _aligned(norm_weight, 16), f"norm_weight must be an aligned row of {k}")
    summed = None
    if residual is not None:
        _cuda_contig("residual", residual, torch.bfloat16, w.device)
        _require(residual.numel() == k and _aligned(residual, 16), f"residual must be an aligned row of {k}")
        summed = torch.empty_like(x)
    _require(not paired or w.N % 2 == 0, "gate||up weight needs an even number of rows")
    n_out = w.N // 2 if paired else w.N
    y = torch.empty((*x.shape[:-1], n_out), dtype=torch.bfloat16, device=w.device)
    native.call("moss_w4a8_norm_gateup_silu" if paired else "moss_w4a8_norm_gemv", native.ptr(x),
                native.ptr(residual) if residual is not None else None, native.ptr(norm_weight),
                native.ptr(summed) if summed is not None else None, float(eps), native.ptr(w.qw), native.ptr(w.scales),
                native.ptr(w.zeros), native.ptr(y), k, n_out, rows_per_wave, native.stream_of(x))
    return y if summed is None else (summed, y)


def linear(x: torch.Tensor | None, w: PackedW4G32, *, paired: bool = False, fused: bool = False,
           prequantized: QuantizedActivation | None = None, rows_per_wave: int = 0,
           out: torch.Tensor | None = None, out_activation: QuantizedActivation | None = None):
    """W4A8 decode projection of one row: ``y[n] = bf16(sum_g f32(isum[n,g]) * (s[n,g] * sx[g]))``
    with ``isum`` the exact integer dot of the group's codes (minus zero point) and int8 ``x``.

    A bf16 ``x`` without ``prequantized`` is quantized inside the projection's kernel (the
    paired form quantizes it first), bit-identical to ``quantize`` then the prequantized call.

    ``paired``: ``w`` holds gate rows then up rows; returns ``bf16(bf16(silu(gate)) * up)``.
    ``fused`` (paired only, N/2 % 32 == 0): also returns that output quantized,
    ``(y, activation)`` (``src/moss_tts/_runtime/dp4a_scaled.py:70-78``)."""
    _require(isinstance(w, PackedW4G32), "w must be a PackedW4G32")
    k = w.K
    _require(k % 64 == 0 and k <= _MAX_K, f"W4A8 GEMV supports K % 64 == 0 and K <= {_MAX_K}")
    _require(rows_per_wave in (0, 1, 2, 4), "rows_per_wave must be 0 (auto), 1, 2 or 4")
    _require(not fused or paired, "fused output quantization requires the paired gate/up form")
    # the plain projection of a bf16 row quantizes inside its own kernel (one launch)
    quant_inside = prequantized is None and not paired
    if prequantized is None:
        _require(x is not None, "x or prequantized is required")
        _require(x.numel() == k, f"one contiguous bf16 row of {k} values required, got shape {tuple(x.shape)}")
        _cuda_contig("x", x, torch.bfloat16, w.device)
        _require(_aligned(x, 16), "x must be 16-byte aligned")
        a = None if quant_inside else quantize(x)
    else:
        a = prequantized
        _check_activation(a, k, w.device)
    n_out = w.N // 2 if paired else w.N
    _require(not paired or w.N % 2 == 0, "gate||up weight needs an even number of rows")
    _require(not fused or (n_out % GROUP == 0 and rows_per_wave in (0, 2, 4)),
             "fused output quantization needs N/2 % 32 == 0 and rows_per_wave 0, 2 or 4")
    if out is None:
        shape = (*x.shape[:-1], n_out) if x is not None else (n_out,)
        out = torch.empty(shape, dtype=torch.bfloat16, device=w.device)
    else:
        _cuda_contig("out", out, torch.bfloat16, w.device)
        _require(out.numel() == n_out, f"out must hold {n_out} values")
    stream = native.stream_of(out)
    if quant_inside:
        native.call("moss_w4a8_quant_gemv", native.ptr(x), native.ptr(w.qw), native.ptr(w.scales),
                    native.ptr(w.zeros), native.ptr(out), k, n_out, rows_per_wave, stream)
        return out
    if not paired:
        native.call("moss_w4a8_gemv", native.ptr(a.qx), native.ptr(a.scales), native.ptr(a.sums), native.ptr(w.qw),
                    native.ptr(w.scales), native.ptr(w.zeros), native.ptr(out), k, n_out, rows_per_wave, stream)
        return out
    o = None
    if fused:
        o = out_activation if out_activation is not None else empty_activation(n_out, w.device)
        _check_activation(o, n_out, w.device)
    native.call("moss_w4a8_gateup_silu", native.ptr(a.qx), native.ptr(a.scales), native.ptr(a.sums),
                native.ptr(w.qw), native.ptr(w.scales), native.ptr(w.zeros), native.ptr(out),
                native.ptr(o.qx) if o else None, native.ptr(o.scales) if o else None,
                native.ptr(o.sums) if o else None, k, n_out, rows_per_wave, stream)
    return (out, o) if fused else out
