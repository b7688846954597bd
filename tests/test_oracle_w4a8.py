"""Pins the W4A8 oracle (``oracle/w4a8.py``) on the CPU.

* ``quantize_g32`` equals an exact rational restatement (``Fraction`` arithmetic with an
  explicit round-to-nearest-even to float32 after every operation) on thousands of bf16 groups
  of all magnitudes, and meets closed forms: the group maximum maps to +-127, a zero group
  has scale f32(1e-8) and zero codes, exact ties round to even, and the reciprocal-multiply
  form differs from a direct division exactly where the reference's choice matters
  (``int4_dp4a.py:21-30`` uses the reciprocal).
* ``group_isums`` equals Python-integer brute force, and on the reference's signed export it
  equals the reference's own lane decodings: the sign spread of ``int4_dp4a.py:43-45`` and the
  nibble<<4 bytes with the final >>4 of ``dp4a_scaled.py:26-40``.
* ``w4a8_f64`` reduces to closed forms (unit scales: the integer sum; one group: one product).
* The dot4 byte order round-trips and matches the nibble expansion of the row-packed words.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import w4a8 as a
from oracle import w4g32 as o

from helpers import rn_f32 as _rn_f32


def _exact_quantize(group):
    """int4_dp4a.py:21-30 in exact rational arithmetic, rounding after every fp32 op."""
    xs = [Fraction(float(v)) for v in group]
    m = max(abs(v) for v in xs)
    scale = max(_rn_f32(m / 127), _rn_f32(Fraction(1e-8)))
    inv = _rn_f32(1 / Fraction(scale))
    q = [round(Fraction(_rn_f32(v * Fraction(inv)))) for v in xs]  # round(): ties to even
    return q, scale


def _random_bf16_groups(n, seed):
    g = torch.Generator().manual_seed(seed)
    mags = 2.0 ** torch.randint(-30, 30, (n, 1), generator=g).float()
    x = (torch.randn(n, 32, generator=g) * mags).bfloat16()
    x[torch.rand(n, 32, generator=g) < 0.05] = 0
    return x


def test_quantizer_matches_exact_rational_restatement():
    x = _random_bf16_groups(600, 1)
    q, scale = a.quantize_g32(x.flatten())
    q = q.reshape(-1, 32)
    for i in range(x.shape[0]):
        eq, es = _exact_quantize(x[i].float().tolist())
        assert float(scale[i]) == es, i
        assert q[i].tolist() == eq, i


def test_quantizer_closed_forms():
    # maximum 127 -> scale 1, inv 1: codes are x rounded half to even
    grp = torch.zeros(32)
    grp[:8] = torch.tensor([127.0, 2.5, 3.5, -2.5, 0.5, 1.5, -0.5, 126.5])
    q, s = a.quantize_g32(grp.bfloat16())
    assert s.tolist() == [1.0]
    assert q[:8].tolist() == [127, 2, 4, -2, 0, 2, 0, 126]
    # zero group: the 1e-8 floor, codes 0
    q, s = a.quantize_g32(torch.zeros(64).bfloat16())
    assert s.tolist() == [float(np.float32(1e-8))] * 2 and not q.any()
    # the maximum always lands on +-127, everything within half a step
    x = _random_bf16_groups(400, 2)
    q, s = a.quantize_g32(x.flatten())
    q = q.reshape(-1, 32).astype(np.int64)
    xf = x.float().numpy()
    arg = np.abs(xf).argmax(1)
    unclamped = s > np.float32(1e-8)
    assert unclamped.sum() > 300
    assert np.all(np.abs(q[np.arange(len(q)), arg])[unclamped] == 127)
    assert np.abs(q).max() <= 127
    err = np.abs(q * s[:, None].astype(np.float64) - xf)
    assert np.all(err <= (0.5 + 1e-4) * s[:, None])  # rint error plus the rounding of x * inv


def test_reciprocal_rounding_is_the_references():
    """max 18 and x = 9: x * RN(1/RN(18/127)) rounds to 64, x / RN(18/127) to 63."""
    grp = torch.zeros(32)
    grp[0], grp[1] = 18.0, 9.0
    q, s = a.quantize_g32(grp.bfloat16())
    assert q[1] == 64
    assert np.rint(np.float32(9.0) / s[0]) == 63


def test_isums_brute_force_and_zero_points():
    g = torch.Generator().manual_seed(3)
    n, k = 5, 128
    qw = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
    z = torch.randint(0, 16, (n, k // 32), generator=g, dtype=torch.uint8)
    qx = torch.randint(-127, 128, (k,), generator=g).numpy().astype(np.int8)
    got = a.group_isums(qw, z, qx)
    for r in range(n):
        for gi in range(k // 32):
            ref = sum((int(qw[r, 32 * gi + t]) - int(z[r, gi])) * int(qx[32 * gi + t]) for t in range(32))
            assert got[r, gi] == ref
    # sum (q - z) x == sum q x - z sum x, the identity the kernels use
    plain = a.group_isums(qw, torch.zeros_like(z), qx)
    assert np.array_equal(got, plain - z.numpy().astype(np.int64) * a.code_sums(qx)[None, :])


def _ref_sign_spread(u16):
    """int4_dp4a.py:43-45: four signed nibbles of a u16 -> four signed bytes of a u32."""
    w = np.asarray(u16, dtype=np.uint32)
    lanes = (w & 15) | ((w & 240) << 4) | ((w & 3840) << 8) | ((w & 61440) << 12)
    lanes = (lanes | ((lanes & 0x08080808) * 30)) & 0xFFFFFFFF
    return lanes.view(np.uint8).reshape(*w.shape, 4).view(np.int8)


def _ref_shifted_bytes(word32):
    """dp4a_scaled.py:26-40 on the interleaved packing (dp4a_packing.py:15-19, byte i of an
    8-code block = codes i | i+4 << 4): byte lanes (w<<4)&0xf0f0f0f0 and w&0xf0f0f0f0 hold 16x
    the signed codes 0..3 and 4..7."""
    w = np.asarray(word32, dtype=np.uint32)
    lo = ((w << 4) & 0xF0F0F0F0).astype(np.uint32).view(np.uint8).reshape(*w.shape, 4).view(np.int8)
    hi = (w & 0xF0F0F0F0).astype(np.uint32).view(np.uint8).reshape(*w.shape, 4).view(np.int8)
    return lo.astype(np.int64), hi.astype(np.int64)


def test_isums_equal_the_references_signed_lane_decodings():
    g = torch.Generator().manual_seed(4)
    n, k = 6, 256
    signed = torch.randint(-8, 8, (n, k), generator=g, dtype=torch.int8)
    packed = o.pack_signed(signed)                       # the export: byte j = codes 2j | 2j+1 << 4
    scales = (torch.rand(n, k // 32, generator=g) + 0.5).bfloat16()
    q, z, _ = o.signed_export_to_codes(packed, scales)
    qx = torch.randint(-127, 128, (k,), generator=g).numpy().astype(np.int8)
    ours = a.group_isums(q, z, qx)

    u16 = packed.numpy().view(np.uint16)                  # [n, k/4]
    lanes = _ref_sign_spread(u16).reshape(n, k).astype(np.int64)
    spread = (lanes * qx.astype(np.int64)[None, :]).reshape(n, k // 32, 32).sum(-1)
    assert np.array_equal(ours, spread)

    words = o.pack_interleaved(packed).numpy().view(np.uint32)   # [n, k/8]
    lo, hi = _ref_shifted_bytes(words)                    # [n, k/8, 4] each
    xq = qx.astype(np.int64).reshape(k // 8, 8)
    dot16 = (lo * xq[None, :, :4]).sum(-1) + (hi * xq[None, :, 4:]).sum(-1)
    assert np.all(dot16 % 16 == 0)
    shifted = (dot16 >> 4).reshape(n, k // 32, 4).sum(-1)
    assert np.array_equal(ours, shifted)


def test_combine_closed_forms():
    g = torch.Generator().manual_seed(5)
    n, k = 4, 64
    qw = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
    z = torch.full((n, 2), 8, dtype=torch.uint8)
    qx = torch.randint(-127, 128, (k,), generator=g).numpy().astype(np.int8)
    ones = torch.ones(n, 2).bfloat16()
    y = a.w4a8_f64(qx, np.ones(2, np.float32), qw, z, ones)
    assert np.array_equal(y, a.group_isums(qw, z, qx).sum(-1).astype(np.float64))
    s = torch.full((n, 2), 0.5).bfloat16()
    y = a.w4a8_f64(qx, np.array([0.25, 4.0], np.float32), qw, z, s)
    isum = a.group_isums(qw, z, qx)
    assert np.array_equal(y, isum[:, 0] * 0.125 + isum[:, 1] * 2.0)


def test_dot4_order_round_trip_and_nibble_expansion():
    g = torch.Generator().manual_seed(6)
    q = torch.randint(-127, 128, (256,), generator=g).numpy().astype(np.int8)
    assert np.array_equal(a.from_dot4_order(a.to_dot4_order(q)), q)
    # the row-packed word j of a group covers k = 8j + t: (w & 0x0F0F0F0F) bytes are t = 0,4,1,5
    codes = torch.randint(0, 16, (1, 64), generator=g, dtype=torch.uint8)
    qw, _, _ = o.rowpack(codes, torch.zeros(1, 2, dtype=torch.uint8), torch.ones(1, 2).bfloat16())
    words = qw.numpy().view(np.uint32).reshape(-1)
    lo = (words & 0x0F0F0F0F).view(np.uint8).reshape(8, 4)
    hi = ((words >> 4) & 0x0F0F0F0F).view(np.uint8).reshape(8, 4)
    expanded = np.concatenate([lo, hi], axis=1).reshape(64)
    assert np.array_equal(expanded, a.to_dot4_order(codes.numpy()[0]))


@pytest.mark.parametrize("n_half", [32, 96])
def test_paired_form_and_output_quantizer(n_half):
    g = torch.Generator().manual_seed(7)
    k = 128
    q = torch.randint(0, 16, (2 * n_half, k), generator=g, dtype=torch.uint8)
    z = torch.randint(0, 16, (2 * n_half, k // 32), generator=g, dtype=torch.uint8)
    s = (torch.rand(2 * n_half, k // 32, generator=g) * 0.02).bfloat16()
    x = torch.randn(k, generator=g).bfloat16()
    y, gate, up = a.w4a8_gateup_silu(x, q, z, s, n_half)
    full, y64, _ = a.w4a8_linear(x, q, z, s)
    assert np.array_equal(y64[:n_half], gate) and np.array_equal(y64[n_half:], up)
    ref = o.silu_mul_rounded(torch.from_numpy(gate.astype(np.float32)), torch.from_numpy(up.astype(np.float32)))
    assert torch.equal(y, ref)
    oq, osx = a.quantize_bf16_output(y)
    assert oq.shape == (n_half,) and osx.shape == (n_half // 32,)
    assert np.array_equal(oq, a.quantize_g32(y)[0])
