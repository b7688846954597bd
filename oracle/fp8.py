"""CPU oracle: FP8 E4M3 (OCP) weight-only linear with per-output-row fp32 scales.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference anchors
-----------------
* ``src/moss_tts/_runtime/fused_mlp.py:7-23`` (``_fp8_silu_gemv``): per output row,
  ``sum_k f32(w[n, k]) * f32(x[k])`` in fp32, times the optional row scale ``S[n]``, rounded
  to bf16 (gate and up separately), then ``bf16(silu(gate))`` times ``up``, stored as bf16.
  Without a scale the factor is 1 (``HAS_SCALE`` false).
* ``fused_mlp.py:26-30``: weights ``[2 n, K]`` gate rows first, output ``[..., n]``.

The quantizer (absmax per row / 448, round to nearest even, saturating) follows the usual
per-channel FP8 weight recipe; the reference ships no FP8 quantizer (its FP8 backbone was
removed), so only the linear's arithmetic is the contract.

Pinning: ``decode_e4m3`` is a bit-field decode written from the OCP FP8 definition and is
checked against torch's ``float8_e4m3fn`` on all 256 codes and against closed forms
(``0x38 = 1``, ``0x7E = 448``, ``0x01 = 2^-9``, ``0x08 = 2^-6``, NaN at ``0x7F``/``0xFF``).
"""
from __future__ import annotations

import numpy as np
import torch

from .w4g32 import silu_mul_rounded

E4M3_MAX = 448.0


def decode_e4m3(codes) -> np.ndarray:
    """uint8 codes -> float32 values: sign bit 7, exponent bits 6..3 (bias 7), mantissa bits
    2..0; exponent 0 is subnormal ``m * 2^-9``; ``S.1111.111`` is NaN; no infinities."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = sign * val
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return val.astype(np.float32)


def codes_to_float(codes: torch.Tensor) -> torch.Tensor:
    """uint8 ``[N, K]`` -> float32 through the bit-field decode."""
    return torch.from_numpy(decode_e4m3(codes.numpy()))


def quantize_rowwise(w: torch.Tensor):
    """Per-output-row absmax quantization: ``s[n] = max_k |w[n, k]| / 448`` (1 for an all-zero
    row), codes = e4m3(clamp(w / s, -448, 448)) with round-to-nearest-even.  Returns
    (codes uint8 ``[N, K]``, s float32 ``[N]``)."""
    w = w.float()
    s = w.abs().amax(dim=1) / E4M3_MAX
    s = torch.where(s > 0, s, torch.ones_like(s))
    q = (w / s[:, None]).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), s


def fp8_linear(x: torch.Tensor, codes: torch.Tensor, scale: torch.Tensor | None) -> torch.Tensor:
    """fp32 ``[M, N]``: ``(x @ f32(w)^T) * s`` -- the reference's row sum times row scale,
    before the bf16 store."""
    y = torch.nn.functional.linear(x.float(), codes_to_float(codes))
    return y * scale.float()[None, :] if scale is not None else y


def fp8_gateup_silu(x: torch.Tensor, codes: torch.Tensor, scale: torch.Tensor | None) -> torch.Tensor:
    """bf16 ``[M, n]`` from gate rows ``[0, n)`` and up rows ``[n, 2n)``."""
    n = codes.shape[0] // 2
    y = fp8_linear(x, codes, scale)
    return silu_mul_rounded(y[:, :n], y[:, n:])
