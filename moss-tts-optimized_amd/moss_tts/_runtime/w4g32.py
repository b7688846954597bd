"""INT4 group-32 operators on the gfx950 library: weight formats, dequant, decode GEMV.

Operator conventions follow the reference's projection functions
(``src/moss_tts/_runtime/dp4a_scaled.py:81-95``, ``dp4a_layout.py:75-84``): caller mistakes
(dtype, contiguity, device, shapes) raise ``ValueError`` before any launch; outputs are
allocated with ``torch.empty`` on the input's device; launches go to the current stream and
are graph-capturable; a failed launch raises ``RuntimeError``.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import native

GROUP = 32


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _cuda_contig(name: str, t: torch.Tensor, dtype: torch.dtype, device=None) -> None:
    _require(isinstance(t, torch.Tensor), f"{name} must be a tensor")
    _require(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _require(t.is_cuda, f"{name} must be a CUDA (HIP) tensor")
    _require(t.is_contiguous(), f"{name} must be contiguous")
    if device is not None:
        _require(t.device == device, f"{name} must be on {device}, got {t.device}")


def _aligned(t: torch.Tensor, a: int) -> bool:
    return t.data_ptr() % a == 0


#: Scales must lie below this bound: the decode GEMV's exact mode and the prefill GEMM form the
#: bit-exact dequant from (128 + q) * s and (128 + z) * s in fp32, which stay finite only for
#: s < 2^120.8 (``moss_w4g32_dequant_bf16`` is exact for every finite scale).  Real group scales
#: are many orders of magnitude smaller (absmax / 7 of bf16 weights).
MAX_SCALE = 2.0 ** 120


def _check_scales(scales: torch.Tensor) -> None:
    """Raise unless every scale is finite and below :data:`MAX_SCALE` in magnitude (one reduction
    and one host sync, at load time)."""
    _require(bool((scales.float().abs() < MAX_SCALE).all()),
             "scales must be finite and below 2^120 in magnitude for the exact in-register dequant")


@dataclass(frozen=True)
class PackedW4G32:
    """One INT4-G32 weight in the row-packed layout (see ``include/moss_hip.h``).

    ``qw int32 [N, K/8]``, ``scales bf16 [N, K/32]``, ``zeros uint8 [N, K/64]``.
    """

    qw: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor

    def __post_init__(self):
        qw, sc, zp = self.qw, self.scales, self.zeros
        _cuda_contig("qw", qw, torch.int32)
        _cuda_contig("scales", sc, torch.bfloat16, qw.device)
        _cuda_contig("zeros", zp, torch.uint8, qw.device)
        _require(qw.ndim == 2 and sc.ndim == 2 and zp.ndim == 2, "packed tensors must be 2-D")
        n, k8 = qw.shape
        k = 8 * k8
        _require(k % 64 == 0, "K must be a multiple of 64")
        _require(tuple(sc.shape) == (n, k // GROUP), f"scales must be [{n}, {k // GROUP}], got {tuple(sc.shape)}")
        _require(tuple(zp.shape) == (n, k // 64), f"zeros must be [{n}, {k // 64}], got {tuple(zp.shape)}")
        _require(_aligned(qw, 16), "qw must be 16-byte aligned")

    @property
    def N(self) -> int:
        return self.qw.shape[0]

    @property
    def K(self) -> int:
        return self.qw.shape[1] * 8

    @property
    def device(self) -> torch.device:
        return self.qw.device

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.qw, self.scales, self.zeros))

    def rows(self, start: int, stop: int) -> "PackedW4G32":
        """Row slice (output channels ``[start, stop)``) as a view."""
        return PackedW4G32(self.qw[start:stop], self.scales[start:stop], self.zeros[start:stop])

    @staticmethod
    def cat(parts: list["PackedW4G32"]) -> "PackedW4G32":
        """Concatenate along output rows (the fused q||k||v and gate||up weights)."""
        return PackedW4G32(torch.cat([p.qw for p in parts]), torch.cat([p.scales for p in parts]),
                           torch.cat([p.zeros for p in parts]))

    @staticmethod
    def empty(N: int, K: int, device) -> "PackedW4G32":
        _require(K % 64 == 0 and K > 0 and N > 0, "K must be a positive multiple of 64")
        return PackedW4G32(torch.empty((N, K // 8), dtype=torch.int32, device=device),
                           torch.empty((N, K // GROUP), dtype=torch.bfloat16, device=device),
                           torch.empty((N, K // 64), dtype=torch.uint8, device=device))


# ------------------------------------------------------------------------ formats
def repack_gptq(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor) -> PackedW4G32:
    """AutoGPTQ-style ``qweight int32 [K/8,N]``, ``scales bf16 [K/32,N]``, ``qzeros int32
    [K/32,N/8]`` (zeros stored literally, no act-order) -> :class:`PackedW4G32`."""
    _cuda_contig("qweight", qweight, torch.int32)
    dev = qweight.device
    _cuda_contig("scales", scales, torch.bfloat16, dev)
    _cuda_contig("qzeros", qzeros, torch.int32, dev)
    _require(qweight.ndim == 2, "qweight must be [K/8, N]")
    k8, n = qweight.shape
    k = 8 * k8
    _require(k % 64 == 0 and n % 8 == 0, "K must be a multiple of 64 and N of 8")
    _require(tuple(scales.shape) == (k // GROUP, n), f"scales must be [{k // GROUP}, {n}]")
    _require(tuple(qzeros.shape) == (k // GROUP, n // 8), f"qzeros must be [{k // GROUP}, {n // 8}]")
    _check_scales(scales)
    out = PackedW4G32.empty(n, k, dev)
    native.call("moss_w4g32_repack_gptq", native.ptr(qweight), native.ptr(scales), native.ptr(qzeros),
                native.ptr(out.qw), native.ptr(out.scales), native.ptr(out.zeros), k, n, native.stream_of(qweight))
    return out


def import_signed(packed: torch.Tensor, scales: torch.Tensor) -> PackedW4G32:
    """The reference's export record ``packed u8 [N,K/2]`` + ``scales [N,K/32]`` (bf16, or
    fp32 that is exactly representable in bf16) -> :class:`PackedW4G32` with ``q = u ^ 8``,
    ``z = 8`` (``src/moss_tts/calibration.py:190-203``, ``_runtime/calibrated_backend.py:46-51``)."""
    _cuda_contig("packed", packed, torch.uint8)
    dev = packed.device
    _require(scales.is_cuda and scales.device == dev, "scales must be on the packed tensor's device")
    _require(scales.dtype in (torch.bfloat16, torch.float32), "scales must be bf16 or fp32")
    _require(packed.ndim == 2, "packed must be [N, K/2]")
    n, k2 = packed.shape
    k = 2 * k2
    _require(k % 64 == 0, "K must be a multiple of 64")
    _require(tuple(scales.shape) == (n, k // GROUP), f"scales must be [{n}, {k // GROUP}]")
    sc = scales.to(torch.bfloat16).contiguous()
    if scales.dtype != torch.bfloat16:
        # the reference's own exactness rule before narrowing scale storage
        # (src/moss_tts/_runtime/dp4a_packing.py:149-152, short_scales.py:37-40)
        _require(torch.equal(sc.float(), scales), "scales are not exactly representable as bf16")
    _check_scales(sc)
    _require(_aligned(packed, 4), "packed must be 4-byte aligned")
    qw = torch.empty((n, k // 8), dtype=torch.int32, device=dev)
    zp = torch.empty((n, k // 64), dtype=torch.uint8, device=dev)
    native.call("moss_w4g32_import_signed", native.ptr(packed), native.ptr(qw), native.ptr(zp), k, n,
                native.stream_of(packed))
    return PackedW4G32(qw, sc, zp)


def quantize_minmax(w: torch.Tensor) -> PackedW4G32:
    """fp32 ``[N, K]`` -> :class:`PackedW4G32` (asymmetric min-max RTN per (row, 32-group))."""
    _cuda_contig("w", w, torch.float32)
    _require(w.ndim == 2 and w.shape[1] % 64 == 0, "w must be [N, K] with K % 64 == 0")
    _require(_aligned(w, 16), "w must be 16-byte aligned")
    n, k = w.shape
    out = PackedW4G32.empty(n, k, w.device)
    native.call("moss_w4g32_quantize_minmax", native.ptr(w), native.ptr(out.qw), native.ptr(out.scales),
                native.ptr(out.zeros), k, n, native.stream_of(w))
    _check_scales(out.scales)
    return out


def quantize_symmetric(w: torch.Tensor) -> PackedW4G32:
    """fp32 ``[N, K]`` -> :class:`PackedW4G32` with the reference's static symmetric scales
    (``bf16(max|w_g| / 7)``) and round-to-nearest codes in [-7, 7], stored with zero point 8
    (``src/moss_tts/_runtime/calibrated_quant.py:36-38,74-77``)."""
    _cuda_contig("w", w, torch.float32)
    _require(w.ndim == 2 and w.shape[1] % 64 == 0, "w must be [N, K] with K % 64 == 0")
    _require(_aligned(w, 16), "w must be 16-byte aligned")
    n, k = w.shape
    out = PackedW4G32.empty(n, k, w.device)
    native.call("moss_w4g32_quantize_symmetric", native.ptr(w), native.ptr(out.qw), native.ptr(out.scales),
                native.ptr(out.zeros), k, n, native.stream_of(w))
    _check_scales(out.scales)
    return out


def unpack_codes(w: PackedW4G32) -> torch.Tensor:
    """Unsigned 4-bit codes ``uint8 [N, K]``."""
    codes = torch.empty((w.N, w.K), dtype=torch.uint8, device=w.device)
    native.call("moss_w4g32_unpack_codes", native.ptr(w.qw), native.ptr(codes), w.K, w.N, native.stream_of(w.qw))
    return codes


def dequantize(w: PackedW4G32) -> torch.Tensor:
    """Bit-exact ``bf16 [N, K]``: ``bf16_rne(float(q - z) * float(s))``
    (``src/moss_tts/_runtime/calibrated_quant.py:41-42``)."""
    out = torch.empty((w.N, w.K), dtype=torch.bfloat16, device=w.device)
    native.call("moss_w4g32_dequant_bf16", native.ptr(w.qw), native.ptr(w.scales), native.ptr(w.zeros),
                native.ptr(out), w.K, w.N, native.stream_of(w.qw))
    return out


# --------------------------------------------------------------------- projections
_MAX_GEMV_K = 8 * 64 * 32


def _check_row(x: torch.Tensor, w: PackedW4G32) -> None:
    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.numel() == w.K, f"one contiguous bf16 row of {w.K} values required, got shape {tuple(x.shape)}")
    _require(w.K <= _MAX_GEMV_K, f"decode GEMV supports K <= {_MAX_GEMV_K}")
    _require(_aligned(x, 16), "x must be 16-byte aligned")


def _rows_arg(rows_per_wave: int) -> int:
    _require(rows_per_wave in (0, 1, 2, 4), "rows_per_wave must be 0 (auto), 1, 2 or 4")
    return rows_per_wave


#: every weight is the bit-exact bf16 dequant before it meets x (default)
EXACT = 0
#: sum_g s * sum (q - z) x, without rounding each weight to bf16
UNROUNDED = 1


def _mode_arg(dequant: int) -> int:
    _require(dequant in (EXACT, UNROUNDED), "dequant must be EXACT (0) or UNROUNDED (1)")
    return dequant


#: tokens the GEMV takes in one pass over the weights
MAX_GEMV_TOKENS = 4


def gemv(x: torch.Tensor, w: PackedW4G32, *, rows_per_wave: int = 0, dequant: int = EXACT) -> torch.Tensor:
    """Decode projection: bf16 ``[..., K]`` -> bf16 ``[..., N]``.  One row, or up to
    ``MAX_GEMV_TOKENS`` rows (exact mode; ``K <= 4096`` or ``K`` in 8192 / 12288 / 16384) read the
    weights once, each output row bit-identical to the one-row GEMV of its input row."""
    _cuda_contig("x", x, torch.bfloat16, w.device)
    m = x.numel() // w.K if w.K else 0
    _require(x.shape[-1] == w.K and m * w.K == x.numel() and 1 <= m <= MAX_GEMV_TOKENS,
             f"1 to {MAX_GEMV_TOKENS} contiguous bf16 rows of {w.K} values required, got shape {tuple(x.shape)}")
    _require(w.K <= _MAX_GEMV_K, f"decode GEMV supports K <= {_MAX_GEMV_K}")
    _require(_aligned(x, 16), "x must be 16-byte aligned")
    rows = _rows_arg(rows_per_wave)
    mode = _mode_arg(dequant)
    if m > 1:
        g = w.K // 32
        _require(mode == EXACT, "several rows take the exact dequant only")
        _require(g <= 128 or (g % 128 == 0 and g <= 512), "several rows need K <= 4096 or K in 8192, 12288, 16384")
    y = torch.empty((*x.shape[:-1], w.N), dtype=torch.bfloat16, device=x.device)
    native.call("moss_w4g32_gemv", native.ptr(x), native.ptr(w.qw), native.ptr(w.scales), native.ptr(w.zeros),
                native.ptr(y), m, w.K, w.N, rows, mode, native.stream_of(x))
    return y


def gateup_silu(x: torch.Tensor, w: PackedW4G32, *, rows_per_wave: int = 0, dequant: int = EXACT) -> torch.Tensor:
    """Fused gate||up decode projection with the SiLU*mul epilogue: ``[..., K]`` ->
    ``[..., N/2]`` (gate rows ``[0, N/2)``, up rows ``[N/2, N)``)."""
    _check_row(x, w)
    _require(w.N % 2 == 0, "gate||up weight needs an even number of rows")
    rows = _rows_arg(rows_per_wave)
    mode = _mode_arg(dequant)
    half = w.N // 2
    y = torch.empty((*x.shape[:-1], half), dtype=torch.bfloat16, device=x.device)
    native.call("moss_w4g32_gateup_silu", native.ptr(x), native.ptr(w.qw), native.ptr(w.scales),
                native.ptr(w.zeros), native.ptr(y), 1, w.K, half, rows, mode, native.stream_of(x))
    return y


def _norm_call(name, x, norm_weight, eps, w, n_out, residual, rows_per_wave, dequant, out=None):
    _check_row(x, w)
    _require(w.K % 2048 == 0 and w.K <= 8192, "the fused norm needs K % 2048 == 0 and K <= 8192")
    _cuda_contig("norm_weight", norm_weight, torch.bfloat16, w.device)
    _require(norm_weight.numel() == w.K, f"norm_weight must hold {w.K} values")
    _require(_aligned(norm_weight, 16), "norm_weight must be 16-byte aligned")
    rows = _rows_arg(rows_per_wave)
    mode = _mode_arg(dequant)
    summed = None
    if residual is not None:
        _cuda_contig("residual", residual, torch.bfloat16, w.device)
        _require(residual.numel() == w.K and _aligned(residual, 16), f"residual must be an aligned row of {w.K}")
        summed = torch.empty_like(x)
    if out is None:
        y = torch.empty((*x.shape[:-1], n_out), dtype=torch.bfloat16, device=x.device)
    else:
        _cuda_contig("out", out, torch.bfloat16, w.device)
        _require(out.numel() == n_out, f"out must hold {n_out} values")
        y = out
    native.call(name, native.ptr(x), native.ptr(residual) if residual is not None else None, native.ptr(norm_weight),
                native.ptr(summed) if summed is not None else None, float(eps), native.ptr(w.qw),
                native.ptr(w.scales), native.ptr(w.zeros), native.ptr(y), w.K, n_out, rows, mode,
                native.stream_of(x))
    return y if summed is None else (summed, y)


def norm_gemv(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, w: PackedW4G32, *,
              residual: torch.Tensor | None = None, rows_per_wave: int = 0, dequant: int = EXACT,
              out: torch.Tensor | None = None):
    """``gemv(rmsnorm(x))`` in one kernel; with ``residual``: ``s = bf16(x + residual)``,
    returns ``(s, gemv(rmsnorm(s)))`` (``src/moss_tts/_runtime/dp4a_norm_projection.py:132-166``).
    ``out``: a contiguous bf16 buffer of N values to write instead of a new tensor."""
    return _norm_call("moss_w4g32_norm_gemv", x, norm_weight, eps, w, w.N, residual, rows_per_wave, dequant, out)


def norm_gateup_silu(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, w: PackedW4G32, *,
                     residual: torch.Tensor | None = None, rows_per_wave: int = 0, dequant: int = EXACT):
    """``gateup_silu(rmsnorm(x))`` in one kernel (optionally after the residual add)."""
    _require(w.N % 2 == 0, "gate||up weight needs an even number of rows")
    return _norm_call("moss_w4g32_norm_gateup_silu", x, norm_weight, eps, w, w.N // 2, residual, rows_per_wave,
                      dequant)


def gemm(x: torch.Tensor, w: PackedW4G32) -> torch.Tensor:
    """Prefill projection: bf16 ``[..., M, K]`` -> bf16 ``[..., M, N]`` on the matrix cores, with
    bit-exact bf16 dequantized weights and fp32 accumulation."""
    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.shape[-1] == w.K, f"x must end in a dimension of {w.K}")
    _require(_aligned(x, 16), "x must be 16-byte aligned")
    m = x.numel() // w.K
    _require(m > 0, "empty input")
    y = torch.empty((*x.shape[:-1], w.N), dtype=torch.bfloat16, device=x.device)
    wp, wb, _keep = native.gemm_workspace(m, w.K, w.N, x.device)
    native.call("moss_w4g32_gemm", native.ptr(x), native.ptr(w.qw), native.ptr(w.scales), native.ptr(w.zeros),
                native.ptr(y), m, w.K, w.N, wp, wb, native.stream_of(x))
    return y


def gemm_silu(x: torch.Tensor, w: PackedW4G32) -> torch.Tensor:
    """Prefill gate||up with the SiLU*mul epilogue: ``w`` holds gate rows then up rows (2 N rows),
    bf16 ``[..., M, K]`` -> bf16 ``[..., M, N]``, equal bit for bit to ``silu_mul(gemm(x, w))``
    (``src/moss_tts/_runtime/llm.py:27-29``, ``prefill_pointwise.py:18-31``)."""
    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.shape[-1] == w.K, f"x must end in a dimension of {w.K}")
    _require(_aligned(x, 16), "x must be 16-byte aligned")
    _require(w.N % 8 == 0, "gate||up weight needs 2 N rows with N % 4 == 0")
    m, n = x.numel() // w.K, w.N // 2
    _require(m > 0, "empty input")
    y = torch.empty((*x.shape[:-1], n), dtype=torch.bfloat16, device=x.device)
    wp, wb, _keep = native.workspace(int(native.lib().moss_gemm_silu_workspace_bytes(m, w.K, n)), x.device)
    native.call("moss_w4g32_gemm_silu", native.ptr(x), native.ptr(w.qw), native.ptr(w.scales), native.ptr(w.zeros),
                native.ptr(y), m, w.K, n, wp, wb, native.stream_of(x))
    return y


def gemm_qk_rope(x: torch.Tensor, w: PackedW4G32, q_weight: torch.Tensor, k_weight: torch.Tensor, cos: torch.Tensor,
                 sin: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, positions: torch.Tensor, eps: float, *,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill QKV projection with the q/k head RMSNorm + RoPE and the K/V cache write as its
    epilogue: equal bit for bit to ``pointwise.qk_rope(gemm(x, w), q_weight, k_weight, cos, sin, keys,
    values, positions, eps, cos_by_position=True, out=out)`` (``src/moss_tts/_runtime/prefill_qkv.py:31-53``).
    ``w`` holds the 6144 QKV rows; ``cos``/``sin`` are ``[L, 128]`` tables indexed by each token's
    device-side position (clamped into the cache).  Returns ``q`` as ``[1, 32, n, 128]`` (a
    transposed view of ``[1, n, 32, 128]``), like ``qk_rope``."""
    from . import pointwise

    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.shape[-1] == w.K, f"x must end in a dimension of {w.K}")
    _require(_aligned(x, 16), "x must be 16-byte aligned")
    _require(w.N == pointwise.QKV, f"the QKV weight must hold {pointwise.QKV} rows")
    n = x.numel() // w.K
    _require(n > 0, "empty input")
    dev = x.device
    _require(keys.ndim == 4 and keys.shape == values.shape and tuple(keys.shape[:2]) == (1, pointwise.KH)
             and keys.shape[3] == pointwise.HD, "matching [1, 8, L, 128] KV buffers required")
    L = keys.shape[2]
    for name, t in (("keys", keys), ("values", values), ("cos", cos), ("sin", sin), ("q_weight", q_weight),
                    ("k_weight", k_weight)):
        _cuda_contig(name, t, torch.bfloat16, dev)
        _require(_aligned(t, 8), f"{name} must be 8-byte aligned")
    for name, t in (("cos", cos), ("sin", sin)):
        _require(t.numel() == L * pointwise.HD, f"{name} must hold {L} rows of {pointwise.HD}")
    for name, t in (("q_weight", q_weight), ("k_weight", k_weight)):
        _require(t.numel() == pointwise.HD, f"{name} must hold {pointwise.HD} values")
    _cuda_contig("positions", positions, torch.int64, dev)
    _require(positions.numel() == n, "one int64 position per token required")
    _require(n <= L, "more tokens than KV rows")
    if out is not None:
        _cuda_contig("out", out, torch.bfloat16, dev)
        _require(out.numel() == n * pointwise.QH * pointwise.HD, f"out must hold {n * pointwise.QH * pointwise.HD} values")
        q = out.view(1, n, pointwise.QH, pointwise.HD)
    else:
        q = torch.empty((1, n, pointwise.QH, pointwise.HD), device=dev, dtype=torch.bfloat16)
    _require(_aligned(q, 8), "out must be 8-byte aligned")
    wp, wb, _keep = native.workspace(int(native.lib().moss_gemm_qk_rope_workspace_bytes(n, w.K)), dev)
    native.call("moss_w4g32_gemm_qk_rope", native.ptr(x), native.ptr(w.qw), native.ptr(w.scales), native.ptr(w.zeros),
                native.ptr(q_weight), native.ptr(k_weight), native.ptr(cos), native.ptr(sin), native.ptr(q),
                native.ptr(keys), native.ptr(values), native.ptr(positions), n, w.K, L, float(eps), wp, wb,
                native.stream_of(x))
    return q.transpose(1, 2)


def gemm_add_rmsnorm(x: torch.Tensor, w: PackedW4G32, residual: torch.Tensor, norm_weight: torch.Tensor,
                     eps: float) -> tuple:
    """Prefill projection followed by the residual add and RMSNorm: ``(summed, y)`` with
    ``summed = bf16(gemm(x, w) + residual)`` and ``y = rmsnorm(summed)``, equal bit for bit to
    ``pointwise.add_rmsnorm(gemm(x, w), residual, norm_weight, eps)``; a K-split GEMM's partial sums
    are reduced inside the norm kernel (``src/moss_tts/_runtime/prefill_pointwise.py:46-57``)."""
    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.shape[-1] == w.K, f"x must end in a dimension of {w.K}")
    m = x.numel() // w.K
    _require(m > 0, "empty input")
    _require(w.N % 8 == 0 and w.N <= 8192, "the norm needs N % 8 == 0 and N <= 8192")
    _cuda_contig("residual", residual, torch.bfloat16, w.device)
    _require(residual.numel() == m * w.N, f"residual must hold {m} x {w.N} values")
    _cuda_contig("norm_weight", norm_weight, torch.bfloat16, w.device)
    _require(norm_weight.numel() == w.N, f"norm_weight must hold {w.N} values")
    for name, t in (("x", x), ("residual", residual), ("norm_weight", norm_weight)):
        _require(_aligned(t, 16), f"{name} must be 16-byte aligned")
    summed = torch.empty((*x.shape[:-1], w.N), dtype=torch.bfloat16, device=x.device)
    y = torch.empty_like(summed)
    wp, wb, _keep = native.gemm_workspace(m, w.K, w.N, x.device)
    native.call("moss_w4g32_gemm_add_rmsnorm", native.ptr(x), native.ptr(w.qw), native.ptr(w.scales),
                native.ptr(w.zeros), native.ptr(residual), native.ptr(norm_weight), float(eps), native.ptr(summed),
                native.ptr(y), m, w.K, w.N, wp, wb, native.stream_of(x))
    return summed, y


#: bytes of the library's scratch array behind :func:`gemm_noalloc` (every GEMM plan's partials fit)
NOALLOC_SCRATCH_BYTES = 32 << 20


def gemm_noalloc(x: torch.Tensor, w: PackedW4G32, out: torch.Tensor) -> torch.Tensor:
    """:func:`gemm` into a caller-provided ``out`` (bf16 ``[..., M, N]``) through the allocation-free
    entry point: the K-split partials live in the library's own device array, so the call allocates
    nothing.  Calls that overlap on one device race on that array."""
    _cuda_contig("x", x, torch.bfloat16, w.device)
    _require(x.shape[-1] == w.K, f"x must end in a dimension of {w.K}")
    _require(_aligned(x, 16), "x must be 16-byte aligned")
    m = x.numel() // w.K
    _require(m > 0, "empty input")
    _cuda_contig("out", out, torch.bfloat16, w.device)
    _require(out.numel() == m * w.N, f"out must hold {m} x {w.N} values")
    need = int(native.lib().moss_gemm_workspace_bytes(m, w.K, w.N))
    _require(need <= NOALLOC_SCRATCH_BYTES, f"this GEMM's partial sums ({need} B) exceed the "
             f"{NOALLOC_SCRATCH_BYTES} B scratch of the allocation-free entry point")
    native.call("moss_w4g32_gemm_noalloc", native.ptr(x), native.ptr(w.qw), native.ptr(w.scales),
                native.ptr(w.zeros), native.ptr(out), m, w.K, w.N, native.stream_of(x))
    return out
