"""CPU oracle: the W4A8 G32 decode arithmetic (int8 activations, integer dot, fp32 combine).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference anchors
-----------------
* Grouped activation quantizer, ``src/moss_tts/_runtime/int4_dp4a.py:21-30``
  (``_int8_activation_grouped``): per group of 32, ``scale = max(div_rn(max|x|, 127), 1e-8)``,
  ``inv = div_rn(1, scale)``, ``q = nearbyint(x * inv)`` (fp32 multiply, ties to even),
  stored as int8; the same quantizer is applied to producer outputs in
  ``dp4a_fusions.py:7-21`` and ``dp4a_scaled.py:70-78``.
* Integer sums and combine, ``src/moss_tts/_runtime/dp4a_scaled.py:45-57``:
  ``isum[n, g] = sum_{k in g} w_signed[n, k] * q[k]`` exactly (int32), then
  ``y[n] = sum_g f32(isum) * (f32(s[n, g]) * sx[g])`` in fp32, stored as bf16.  With the
  row-packed codes ``w_signed = q_w - z`` (``q_w = u ^ 8``, ``z = 8`` for the reference's
  signed export).  The fp32 order of the group sum is the Triton reduction's; it is not
  restated: the oracle sums in float64 and tests allow the last-bit difference this causes.
* Paired gate/up epilogue, ``dp4a_scaled.py:64-68``: gate and up rounded to bf16,
  ``bf16(silu(gate))``, product stored as bf16.
* Fused norm + quantizer, ``dp4a_fusions.py:24-40``: the bf16 RMSNorm output is quantized.

Pinning (tests/test_oracle_w4a8.py): the quantizer against an exact rational restatement
(Python ``Fraction`` with explicit round-to-nearest-even to float32) and closed forms (the
group maximum maps to +-127, a zero group has scale 1e-8, exact ties round to even);
``group_isums`` against Python-integer brute force and against the reference's own
signed-lane decoding (``int4_dp4a.py:43-45`` sign spread, ``dp4a_scaled.py:26-40`` nibble<<4
then >>4) applied to the signed export; the combine against float64 closed forms.
"""
from __future__ import annotations

import numpy as np
import torch

from .w4g32 import GROUP, bf16_bits_to_f32, bf16_to_bits, bits_to_bf16, f32_to_bf16_bits, silu_mul_rounded

DOT4_ORDER = np.array([0, 4, 1, 5, 2, 6, 3, 7])


def _f32(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().float().numpy()
    return np.asarray(x, dtype=np.float32)


def quantize_g32(x) -> tuple[np.ndarray, np.ndarray]:
    """x [..., K] (bf16 tensor or float32 values) -> (q int8 [..., K], scale fp32 [..., K/32]).

    ``int4_dp4a.py:21-30``: every step is a float32 operation with one rounding.
    """
    v = _f32(x).astype(np.float32)
    shape = v.shape
    g = v.reshape(*shape[:-1], shape[-1] // GROUP, GROUP)
    m = np.abs(g).max(axis=-1)
    scale = np.maximum(m / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    prod = (g * inv[..., None]).astype(np.float32)
    q = np.rint(prod).astype(np.int8)  # np.rint: ties to even
    return q.reshape(shape), scale


def code_sums(q: np.ndarray) -> np.ndarray:
    """Per-group sums of the int8 codes, int32 [..., K/32] (the zero-point term)."""
    q = np.asarray(q).astype(np.int64)
    return q.reshape(*q.shape[:-1], q.shape[-1] // GROUP, GROUP).sum(-1).astype(np.int32)


def to_dot4_order(q: np.ndarray) -> np.ndarray:
    """Natural-order int8 codes [..., K] -> the byte layout the HIP kernels read."""
    q = np.asarray(q)
    b = q.reshape(*q.shape[:-1], q.shape[-1] // 8, 8)
    return np.ascontiguousarray(b[..., DOT4_ORDER]).reshape(q.shape)


def from_dot4_order(b: np.ndarray) -> np.ndarray:
    b = np.asarray(b)
    v = b.reshape(*b.shape[:-1], b.shape[-1] // 8, 8)
    out = np.empty_like(v)
    out[..., DOT4_ORDER] = v
    return out.reshape(b.shape)


def group_isums(q_w: torch.Tensor, z: torch.Tensor, qx: np.ndarray) -> np.ndarray:
    """isum[n, g] = sum_{k in g} (q_w[n, k] - z[n, g]) * qx[k], int64 [N, G] (exact).

    Computed as sum_k q_w qx - z sum_k qx, the first term as a float32 contraction: codes are at
    most 15 and |qx| at most 127, so every product and every partial sum of a group's 32 products is
    an integer below 2^24, which float32 holds exactly in any summation order."""
    w = q_w.cpu()
    n, k = w.shape
    g = k // GROUP
    xq = torch.from_numpy(np.asarray(qx).astype(np.float32)).view(g, GROUP)
    s1 = torch.einsum("ngt,gt->ng", w.to(torch.float32).view(n, g, GROUP), xq).to(torch.int64).numpy()
    return s1 - z.cpu().numpy().astype(np.int64) * code_sums(qx).astype(np.int64)[None, :]


def _combine(isum: np.ndarray, sx: np.ndarray, s, reverse_f32: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """(sum_g f32(isum) * f32(f32(s) * sx) in float64, sum of the terms' magnitudes).  With
    ``reverse_f32`` the terms are added in float32 from the last group to the first: another fp32
    order the reference's unrestated reduction could have used, for measuring how far summation
    order alone moves a composed result."""
    terms = (isum.astype(np.float32).astype(np.float64) *
             (s.cpu().float().numpy() * np.asarray(sx, dtype=np.float32)[None, :]).astype(np.float32)
             .astype(np.float64))
    if reverse_f32:
        t32 = terms.astype(np.float32)[:, ::-1]
        acc = np.zeros(t32.shape[0], dtype=np.float32)
        for gi in range(t32.shape[1]):
            acc = (acc + t32[:, gi]).astype(np.float32)
        return acc.astype(np.float64), np.abs(terms).sum(-1)
    return terms.sum(-1), np.abs(terms).sum(-1)


def w4a8_f64(qx: np.ndarray, sx: np.ndarray, q_w, z, s) -> np.ndarray:
    """Pre-rounding output in float64: sum_g f32(isum) * f32(f32(s) * sx) (``dp4a_scaled.py:53-57``)."""
    return _combine(group_isums(q_w, z, qx), sx, s)[0]


def w4a8_linear(x: torch.Tensor, q_w, z, s, reverse_f32: bool = False) -> tuple[torch.Tensor, np.ndarray, np.ndarray]:
    """bf16 x [K] -> (y bf16 [N], the float64 pre-rounding sums, per-row sum of |terms|)."""
    qx, sx = quantize_g32(x)
    y64, mag = _combine(group_isums(q_w, z, qx), sx, s, reverse_f32)
    y = bits_to_bf16(f32_to_bf16_bits(y64.astype(np.float32)))
    return y, y64, mag


def w4a8_gateup_silu(x: torch.Tensor, q_w, z, s, n_half: int, reverse_f32: bool = False):
    """Paired form (``dp4a_scaled.py:64-68``): returns (y bf16 [n_half], gate64, up64)."""
    qx, sx = quantize_g32(x)
    y64 = _combine(group_isums(q_w, z, qx), sx, s, reverse_f32)[0]
    gate64, up64 = y64[:n_half], y64[n_half:]
    g = torch.from_numpy(gate64.astype(np.float32))
    u = torch.from_numpy(up64.astype(np.float32))
    return silu_mul_rounded(g, u), gate64, up64


def quantize_bf16_output(y: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """The fused output quantizer of ``dp4a_scaled.py:70-78``: the bf16 result, grouped by 32."""
    return quantize_g32(bf16_bits_to_f32(bf16_to_bits(y)))
