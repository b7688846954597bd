"""CPU oracle: INT4 group-32 formats, quantizers, bf16 dequant and dequant-then-matmul.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Conventions
-----------
* Weights are in torch orientation ``[N, K]`` (out_features, in_features), grouped along
  K in groups of 32 consecutive input channels (``G = K // 32``).
* ``q`` are unsigned 4-bit codes in [0, 15], ``z`` the per-(row, group) zero point in
  [0, 15] (stored literally, no "-1" offset), ``s`` bf16 scales.  The dequantized weight is
  ``w = bf16_rne(float32(q - z) * float32(s))``.
* bf16 values are carried as ``torch.bfloat16`` tensors; bit-level work uses numpy.

Reference anchors
-----------------
* dequant: ``src/moss_tts/_runtime/calibrated_quant.py:41-42`` -- ``bf16(float(q) * float(s))``
  on signed codes, one RNE rounding.  With ``q_u = q_signed XOR 8`` (two's-complement
  nibble reinterpreted) and ``z = 8``, ``(q_u - 8) == q_signed`` so the zero-point form
  below reduces to it bit for bit.
* static scales: ``src/moss_tts/_runtime/calibrated_quant.py:36-38``.
* export nibble packing: ``src/moss_tts/calibration.py:190-191``; unpack:
  ``src/moss_tts/_runtime/calibrated_backend.py:8-13``.
* interleaved dp4a packing: ``src/moss_tts/_runtime/dp4a_packing.py:15-27``.
* dequant-then-matmul contract: ``src/moss_tts/calibration.py:185-188``.
"""
from __future__ import annotations

import numpy as np
import torch

GROUP = 32


# ----------------------------------------------------------------------------- bf16 bits
def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 with round-to-nearest-even; returns uint16 bit patterns.

    Published method: add ``0x7FFF + lsb`` to the fp32 bit pattern and keep the high 16
    bits; NaN maps to the canonical quiet NaN ``0x7FC0`` (sign kept).
    """
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r = np.where(nan, ((u >> 16) & 0x8000).astype(np.uint16) | np.uint16(0x7FC0), r)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bits_to_bf16(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def bf16_to_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _np(t) -> np.ndarray:
    return t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)


# ------------------------------------------------------------------------- quantizers
def quantize_minmax_g32(w: torch.Tensor):
    """Asymmetric min-max RTN quantizer per (row, 32-group), the synthetic weight recipe.

    ``s = bf16((max - min) / 15)`` (clamped to >= 1e-8 before rounding),
    ``z = clamp(rint(-min / s), 0, 15)``, ``q = clamp(rint(w / s) + z, 0, 15)``, all in
    float32 with IEEE division and round-half-even ``rint``.
    Returns ``q uint8 [N,K]``, ``z uint8 [N,G]``, ``s bf16 [N,G]``.
    """
    a = _np(w).astype(np.float32)
    n, k = a.shape
    if k % GROUP:
        raise ValueError("K must be a multiple of 32")
    g = a.reshape(n, k // GROUP, GROUP)
    lo = g.min(-1)
    hi = g.max(-1)
    s32 = np.maximum((hi - lo) / np.float32(15), np.float32(1e-8)).astype(np.float32)
    sb = f32_to_bf16_bits(s32)
    sf = bf16_bits_to_f32(sb)
    z = np.clip(np.rint(-lo / sf), 0, 15).astype(np.float32)
    q = np.clip(np.rint(g / sf[..., None]) + z[..., None], 0, 15)
    return (torch.from_numpy(q.reshape(n, k).astype(np.uint8)),
            torch.from_numpy(z.astype(np.uint8)),
            bits_to_bf16(sb))


def static_scales(w: torch.Tensor, group: int = GROUP) -> torch.Tensor:
    """``bf16(clamp_min(max|w_g|, 1e-8) / 7)`` -- ``calibrated_quant.py:36-38``."""
    a = np.abs(_np(w).astype(np.float32))
    n, k = a.shape
    m = np.maximum(a.reshape(n, k // group, group).max(-1), np.float32(1e-8))
    return bits_to_bf16(f32_to_bf16_bits((m / np.float32(7)).astype(np.float32)))


def quantize_symmetric(w: torch.Tensor, scales: torch.Tensor, group: int = GROUP) -> torch.Tensor:
    """Round-to-nearest signed codes in [-7, 7] against static scales.

    The no-Hessian special case of ``calibrated_quant.py:74-77`` (torch backend):
    ``code = clamp(round(w / s), -7, 7)``.
    """
    a = _np(w).astype(np.float32)
    n, k = a.shape
    s = bf16_bits_to_f32(bf16_to_bits(scales)).reshape(n, k // group, 1)
    c = np.clip(np.rint(a.reshape(n, k // group, group) / s), -7, 7)
    return torch.from_numpy(c.reshape(n, k).astype(np.int8))


# -------------------------------------------------------------------------- dequant
def dequantize(q: torch.Tensor, z: torch.Tensor, s: torch.Tensor, group: int = GROUP) -> torch.Tensor:
    """``w = bf16_rne(f32(q - z) * f32(s))`` per (row, group) -> bf16 ``[N,K]``.

    The fp32 product is exact ((q-z) has <= 5 significant bits, s has 8), so the single
    RNE to bf16 is the only rounding -- as in ``calibrated_quant.py:42``.
    """
    qn = _np(q).astype(np.int32)
    zn = _np(z).astype(np.int32)
    n, k = qn.shape
    sf = bf16_bits_to_f32(bf16_to_bits(s))
    d = (qn.reshape(n, k // group, group) - zn[..., None]).astype(np.float32)
    prod = (d * sf[..., None]).astype(np.float32).reshape(n, k)
    return bits_to_bf16(f32_to_bf16_bits(prod))


def dequantize_signed(codes: torch.Tensor, scales: torch.Tensor, group: int = GROUP) -> torch.Tensor:
    """The reference's own ``dequantize(signed, scales, group)`` (``calibrated_quant.py:41-42``)."""
    c = _np(codes).astype(np.float32)
    n, k = c.shape
    sf = bf16_bits_to_f32(bf16_to_bits(scales)) if scales.dtype == torch.bfloat16 \
        else _np(scales).astype(np.float32)
    prod = (c.reshape(n, k // group, group) * sf[..., None]).astype(np.float32).reshape(n, k)
    return bits_to_bf16(f32_to_bf16_bits(prod))


# ------------------------------------------------------------ AutoGPTQ-style G32 layout
def pack_gptq(q: torch.Tensor, z: torch.Tensor, s: torch.Tensor):
    """Torch-orientation codes -> ``qweight int32 [K/8,N]``, ``scales bf16 [G,N]``,
    ``qzeros int32 [G,N/8]``.  Nibble j of ``qweight[i,n]`` is ``q[n, 8i+j]``; nibble j of
    ``qzeros[g,c]`` is ``z[8c+j, g]`` (zero points stored literally)."""
    qn = _np(q).astype(np.uint32)
    zn = _np(z).astype(np.uint32)
    n, k = qn.shape
    if k % 8 or n % 8:
        raise ValueError("K and N must be multiples of 8")
    t = qn.T.reshape(k // 8, 8, n)
    qw = np.zeros((k // 8, n), dtype=np.uint32)
    for j in range(8):
        qw |= (t[:, j, :] & 15) << (4 * j)
    zt = zn.T.reshape(zn.shape[1], n // 8, 8)
    qz = np.zeros((zn.shape[1], n // 8), dtype=np.uint32)
    for j in range(8):
        qz |= (zt[:, :, j] & 15) << (4 * j)
    return (torch.from_numpy(qw.view(np.int32)),
            s.t().contiguous(),
            torch.from_numpy(qz.view(np.int32)))


def unpack_gptq(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor):
    """Inverse of :func:`pack_gptq` -> ``q [N,K]``, ``z [N,G]``, ``s bf16 [N,G]``."""
    qw = _np(qweight).view(np.uint32)
    qz = _np(qzeros).view(np.uint32)
    k8, n = qw.shape
    q = np.stack([(qw >> (4 * j)) & 15 for j in range(8)], axis=1).reshape(k8 * 8, n)
    z = np.stack([(qz >> (4 * j)) & 15 for j in range(8)], axis=2).reshape(qz.shape[0], n)
    return (torch.from_numpy(q.T.astype(np.uint8).copy()),
            torch.from_numpy(z.T.astype(np.uint8).copy()),
            scales.t().contiguous())


# ------------------------------------------------ the reference's signed-nibble export
def pack_signed(codes: torch.Tensor) -> torch.Tensor:
    """``packed[n,j] = (c[n,2j] & 15) | (c[n,2j+1] & 15) << 4`` -- ``calibration.py:190-191``."""
    u = _np(codes).astype(np.int16).astype(np.uint8) & 15
    return torch.from_numpy((u[:, ::2] | (u[:, 1::2] << 4)).astype(np.uint8))


def unpack_signed(packed: torch.Tensor) -> torch.Tensor:
    """Two's-complement nibbles -> int8 codes -- ``calibrated_backend.py:8-13``."""
    p = _np(packed).astype(np.uint8)
    lo = (p & 15).astype(np.int8)
    hi = (p >> 4).astype(np.int8)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    return torch.from_numpy(np.stack([lo, hi], -1).reshape(p.shape[0], -1).astype(np.int8))


def signed_export_to_codes(packed: torch.Tensor, scales: torch.Tensor):
    """Reference export ``(packed u8 [N,K/2], scales [N,G])`` -> ``(q, z, s)``.

    The exact bijection: ``q = u XOR 8`` (u = stored nibble), ``z = 8``, scales kept
    (fp32 scales must be bf16-exact).  Then ``(q - 8) * s == signed * s`` bit for bit.
    """
    p = _np(packed).astype(np.uint8)
    u = np.stack([p & 15, p >> 4], -1).reshape(p.shape[0], -1)
    q = (u ^ 8).astype(np.uint8)
    z = np.full((p.shape[0], scales.shape[1]), 8, dtype=np.uint8)
    s = scales if scales.dtype == torch.bfloat16 else scales.bfloat16()
    if scales.dtype != torch.bfloat16 and not torch.equal(s.float(), scales.float()):
        raise ValueError("scales are not exactly representable as bf16")
    return torch.from_numpy(q), torch.from_numpy(z), s.contiguous()


def pack_interleaved(packed: torch.Tensor) -> torch.Tensor:
    """``dp4a_packing.py:15-19``: per 8-code block, byte i = u[8t+i] | u[8t+i+4] << 4."""
    p = _np(packed).astype(np.uint8)
    n, k2 = p.shape
    u = np.stack([p & 15, p >> 4], -1).reshape(n, -1, 8)
    return torch.from_numpy((u[:, :, :4] | (u[:, :, 4:] << 4)).reshape(n, k2).astype(np.uint8))


def unpack_interleaved(packed: torch.Tensor) -> torch.Tensor:
    """``dp4a_packing.py:22-27`` -> int8 signed codes."""
    p = _np(packed).astype(np.uint8)
    n, _ = p.shape
    w = p.reshape(n, -1, 4)
    u = np.concatenate([w & 15, w >> 4], -1).reshape(n, -1).astype(np.int8)
    return torch.from_numpy(np.where(u >= 8, u - 16, u).astype(np.int8))


# ------------------------------------------------------- the kernels' row-packed layout
def rowpack(q: torch.Tensor, z: torch.Tensor, s: torch.Tensor):
    """Codes -> the HIP kernels' row-packed layout (checked bit for bit against the
    device repacker).

    * ``qw uint32 [N, K/8]``: group g of row n is words ``4g..4g+3``; word j covers
      ``k = 32g + 8j + t``; the code for ``t = 2i`` sits at bits ``[4i, 4i+4)`` and for
      ``t = 2i+1`` at bits ``[16+4i, 20+4i)``.
    * ``sc bf16 [N, G]`` (unchanged order).
    * ``zp uint8 [N, G/2]`` in blocks of 128 groups: for block c with ``r = min(128, G - 128c)``
      groups, byte ``64c + b`` (``b < r/2``) holds ``z[128c + b]`` (low nibble) and
      ``z[128c + r/2 + b]`` (high nibble).  A GEMV lane owning groups ``l`` and ``l + 64`` of
      a 128-group slice finds both zero points in one byte.
    """
    qn = _np(q).astype(np.uint32)
    zn = _np(z).astype(np.uint8)
    n, k = qn.shape
    if k % 64:
        raise ValueError("row-packed layout needs K % 64 == 0")
    t = qn.reshape(n, k // 8, 8)
    w = np.zeros((n, k // 8), dtype=np.uint32)
    for i in range(4):
        w |= (t[:, :, 2 * i] & 15) << (4 * i)
        w |= (t[:, :, 2 * i + 1] & 15) << (16 + 4 * i)
    zp = np.zeros((n, zn.shape[1] // 2), dtype=np.uint8)
    for c0 in range(0, zn.shape[1], 128):
        r = min(128, zn.shape[1] - c0)
        zp[:, c0 // 2: c0 // 2 + r // 2] = (zn[:, c0: c0 + r // 2] & 15) | ((zn[:, c0 + r // 2: c0 + r] & 15) << 4)
    return (torch.from_numpy(w.view(np.int32)), s.contiguous(), torch.from_numpy(zp))


def rowunpack(qw: torch.Tensor, zp: torch.Tensor):
    """Inverse of :func:`rowpack` for codes and zeros -> ``q [N,K]``, ``z [N,G]``."""
    w = _np(qw).view(np.uint32)
    n, k8 = w.shape
    out = np.zeros((n, k8, 8), dtype=np.uint8)
    for i in range(4):
        out[:, :, 2 * i] = (w >> (4 * i)) & 15
        out[:, :, 2 * i + 1] = (w >> (16 + 4 * i)) & 15
    zb = _np(zp).astype(np.uint8)
    g = 2 * zb.shape[1]
    z = np.zeros((n, g), dtype=np.uint8)
    for c0 in range(0, g, 128):
        r = min(128, g - c0)
        blk = zb[:, c0 // 2: c0 // 2 + r // 2]
        z[:, c0: c0 + r // 2] = blk & 15
        z[:, c0 + r // 2: c0 + r] = blk >> 4
    return torch.from_numpy(out.reshape(n, k8 * 8)), torch.from_numpy(z)


_ROWPACK_SHIFTS = (0, 16, 4, 20, 8, 24, 12, 28)   # bit offset of code t = 0..7 in a row-packed word


def dequantize_rowpack_f32(qw: torch.Tensor, sc: torch.Tensor, zp: torch.Tensor,
                           out: torch.Tensor | None = None, chunk: int = 512) -> torch.Tensor:
    """The row-packed weight (layout of :func:`rowpack`) dequantized with multi-threaded torch CPU
    ops for full-size layers: ``float32 [N, K]`` holding exactly the bf16 values
    ``bf16_rne(f32(q - z) * f32(s))`` (``calibrated_quant.py:41-42``), ready for ``F.linear``.
    Works through ``chunk`` rows at a time; ``out`` (fp32, at least ``N * K`` values) is reused
    when given, so a layer loop does not fault in fresh pages for every projection."""
    w = qw.contiguous().view(torch.int32)
    n, k8 = w.shape
    k = 8 * k8
    g = k // GROUP
    shifts = torch.tensor(_ROWPACK_SHIFTS, dtype=torch.int32)
    zb = zp.contiguous().to(torch.int32)
    z = torch.empty((n, g), dtype=torch.int32)
    for c0 in range(0, g, 128):
        r = min(128, g - c0)
        blk = zb[:, c0 // 2: c0 // 2 + r // 2]
        z[:, c0: c0 + r // 2] = blk & 15
        z[:, c0 + r // 2: c0 + r] = blk >> 4
    res = torch.empty((n, k)) if out is None else out.view(-1)[: n * k].view(n, k)
    for r0 in range(0, n, chunk):
        r1 = min(n, r0 + chunk)
        codes = (w[r0:r1].unsqueeze(-1) >> shifts) & 15                       # [rows, K/8, 8] in k order
        d = (codes.view(r1 - r0, g, GROUP) - z[r0:r1, :, None]).float()
        d.mul_(sc[r0:r1].float()[:, :, None])
        res[r0:r1] = d.view(r1 - r0, k).bfloat16()
    return res


# ------------------------------------------------------------------- linear contracts
def linear(x: torch.Tensor, w_bf16: torch.Tensor) -> torch.Tensor:
    """``F.linear(x.float(), w.float())`` in fp32 on the CPU -- ``calibration.py:185-188``."""
    return torch.nn.functional.linear(x.float(), w_bf16.float())


def w4g32_linear(x: torch.Tensor, q, z, s) -> torch.Tensor:
    """Dequant-then-matmul oracle; returns fp32 ``[M, N]`` (round to bf16 to compare)."""
    return linear(x, dequantize(q, z, s))


def silu_mul_rounded(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """bf16 rounding points of the paired gate/up epilogue.

    ``g = bf16(gate)``, ``u = bf16(up)``, ``a = bf16(g / (1 + exp(-g)))`` in fp32,
    ``out = bf16(a * u)`` -- ``src/moss_tts/_runtime/dp4a_scaled.py:65-68`` and
    ``src/moss_tts/_runtime/kernels.py:124-129``.
    """
    g = gate.bfloat16().float()
    u = up.bfloat16().float()
    a = (g / (1.0 + torch.exp(-g))).bfloat16().float()
    return (a * u).bfloat16()


def w4g32_gateup_silu(x: torch.Tensor, q, z, s, n_half: int) -> torch.Tensor:
    """Fused gate||up GEMV + SiLU*mul; rows ``[0,n)`` gate, ``[n,2n)`` up
    (``src/moss_tts/_runtime/llm.py:144``).  Returns bf16 ``[M, n]``."""
    y = w4g32_linear(x, q, z, s)
    return silu_mul_rounded(y[:, :n_half], y[:, n_half:])


# ------------------------------------------------- CPU baseline (timed in bench.py only)
def gptq_dequant_cpu(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor) -> torch.Tensor:
    """The dequant half of :func:`gptq_dequant_linear_cpu`: AutoGPTQ ``qweight int32 [K/8,N]``,
    ``scales bf16 [G,N]``, ``qzeros int32 [G,N/8]`` -> ``w bf16 [K,N]`` with
    ``w = bf16((q - z) * s)`` (``calibrated_quant.py:41-42``), in multi-threaded torch CPU ops."""
    k8, n = qweight.shape
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    q = ((qweight.unsqueeze(1) >> shifts[None, :, None]) & 15).reshape(k8 * 8, n)
    z = ((qzeros.unsqueeze(2) >> shifts[None, None, :]) & 15).reshape(qzeros.shape[0], n)
    return ((q.view(-1, GROUP, n) - z[:, None, :]).float() * scales.float()[:, None, :]).bfloat16().view(k8 * 8, n)


def gptq_dequant_linear_cpu(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                            qzeros: torch.Tensor) -> torch.Tensor:
    """The reference's dequant-then-matmul on the AutoGPTQ layout with multi-threaded torch
    CPU ops, dequantizing on every call: unpack nibbles, ``w = bf16((q - z) * s)``
    (``calibrated_quant.py:41-42``), ``F.linear(x.float(), w.float())``
    (``calibration.py:185-188``).  Returns fp32 ``[M, N]``."""
    w = gptq_dequant_cpu(qweight, scales, qzeros)
    return torch.nn.functional.linear(x.float(), w.t().float())
