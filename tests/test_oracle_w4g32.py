"""Pins the CPU oracle's INT4-G32 functions (no reference golden vectors exist for this path).

Each function is pinned by at least one of: hand-derived known answers, exhaustive
enumeration, an independent implementation (torch's RNE, the C restatement in
oracle/w4g32_ref.c, an fp64 matmul), or brute force -- chosen so a dropped term, a swapped
nibble, a wrong sign or a wrong rounding mode fails.
"""
import numpy as np
import pytest
import torch

from fractions import Fraction

from oracle import cref
from oracle import w4g32 as o

from helpers import rn_f32


def _bits(t):
    return o.bf16_to_bits(t)


# ------------------------------------------------------------------------ bf16 rounding
@pytest.mark.parametrize("src,want", [
    (0x3F800000, 0x3F80),  # 1.0
    (0x3F808000, 0x3F80),  # exact tie, even kept
    (0x3F818000, 0x3F82),  # exact tie, odd rounds up
    (0x3F808001, 0x3F81),  # above the tie
    (0x3F807FFF, 0x3F80),  # below the tie
    (0x7F7FFFFF, 0x7F80),  # largest finite rounds to +inf
    (0x7F800000, 0x7F80),  # +inf
    (0x80000000, 0x8000),  # -0.0 keeps its sign
    (0x00000001, 0x0000),  # smallest denormal rounds to +0
    (0x7FC00001, 0x7FC0),  # NaN -> canonical quiet NaN
])
def test_bf16_rne_known_answers(src, want):
    f = np.array([src], dtype=np.uint32).view(np.float32)
    assert int(o.f32_to_bf16_bits(f)[0]) == want
    assert int(cref.bf16_rne(f)[0]) == want


def test_bf16_rne_three_implementations_agree():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    # force many exact ties and near-ties
    u[:50_000] = (u[:50_000] & 0xFFFF0000) | 0x8000
    u[50_000:60_000] = (u[50_000:60_000] & 0xFFFF0000) | 0x7FFF
    f = u.view(np.float32)
    finite = np.isfinite(f)
    a = o.f32_to_bf16_bits(f)
    b = cref.bf16_rne(f)
    c = o.bf16_to_bits(torch.from_numpy(f.copy()).bfloat16())
    assert np.array_equal(a, b)
    assert np.array_equal(a[finite], c[finite])


# --------------------------------------------------------------------- AutoGPTQ layout
def test_gptq_pack_known_answers():
    q = torch.zeros((8, 64), dtype=torch.uint8)
    q[0, :8] = torch.arange(8, dtype=torch.uint8)
    q[1, :8] = 15 - torch.arange(8, dtype=torch.uint8)
    z = torch.zeros((8, 2), dtype=torch.uint8)
    z[:, 0] = torch.arange(1, 9, dtype=torch.uint8)
    s = torch.ones((8, 2), dtype=torch.bfloat16)
    qweight, scales, qzeros = o.pack_gptq(q, z, s)
    assert qweight.shape == (8, 8) and scales.shape == (2, 8) and qzeros.shape == (2, 1)
    assert qweight[0, 0].item() & 0xFFFFFFFF == 0x76543210
    assert qweight[0, 1].item() & 0xFFFFFFFF == 0x89ABCDEF
    assert qzeros[0, 0].item() & 0xFFFFFFFF == 0x87654321


def test_gptq_roundtrip_numpy_and_c():
    g = torch.Generator().manual_seed(1)
    n, k = 48, 256
    q = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
    z = torch.randint(0, 16, (n, k // 32), generator=g, dtype=torch.uint8)
    s = torch.randn((n, k // 32), generator=g).bfloat16()
    qweight, scales, qzeros = o.pack_gptq(q, z, s)
    q2, z2, s2 = o.unpack_gptq(qweight, scales, qzeros)
    assert torch.equal(q2, q) and torch.equal(z2, z) and np.array_equal(_bits(s2), _bits(s))
    qc, zc = cref.unpack_gptq(qweight, qzeros)
    assert torch.equal(qc, q) and torch.equal(zc, z)


# ------------------------------------------------------------ reference signed export
def test_signed_export_known_answers():
    p = torch.tensor([[0x0F, 0x87, 0x78, 0x10]], dtype=torch.uint8)
    assert o.unpack_signed(p).tolist() == [[-1, 0, 7, -8, -8, 7, 0, 1]]
    c = torch.tensor([[0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -1, 7]], dtype=torch.int8)
    assert o.pack_signed(c).tolist() == [[0x10, 0x32, 0x54, 0x76, 0x98, 0x7F]]


def test_signed_export_exhaustive_bijection():
    p = torch.arange(256, dtype=torch.uint8).reshape(1, 256)
    signed = o.unpack_signed(p)
    assert torch.equal(signed, cref.unpack_signed(p))
    assert torch.equal(o.pack_signed(signed), p)
    q, z, _ = o.signed_export_to_codes(p, torch.ones((1, 16), dtype=torch.bfloat16))
    assert torch.equal(q.to(torch.int16) - z.to(torch.int16).repeat_interleave(32, 1), signed.to(torch.int16))
    # every signed value in [-8, 7] occurs, and q covers [0, 15]
    assert sorted(set(signed.flatten().tolist())) == list(range(-8, 8))
    assert sorted(set(q.flatten().tolist())) == list(range(16))


def test_interleaved_layout_known_answer_and_roundtrip():
    c = torch.arange(8, dtype=torch.int8).reshape(1, 8)
    inter = o.pack_interleaved(o.pack_signed(c))
    assert inter.tolist() == [[0x40, 0x51, 0x62, 0x73]]
    g = torch.Generator().manual_seed(2)
    codes = torch.randint(-8, 8, (16, 128), generator=g, dtype=torch.int8)
    assert torch.equal(o.unpack_interleaved(o.pack_interleaved(o.pack_signed(codes))), codes)


# ------------------------------------------------------------------ kernel row layout
def test_rowpack_known_answer_and_roundtrip():
    q = torch.zeros((1, 64), dtype=torch.uint8)
    q[0, :8] = torch.arange(8, dtype=torch.uint8)
    z = torch.tensor([[3, 12]], dtype=torch.uint8)
    qw, _, zp = o.rowpack(q, z, torch.ones((1, 2), dtype=torch.bfloat16))
    assert qw[0, 0].item() & 0xFFFFFFFF == 0x75316420
    assert zp.tolist() == [[0xC3]]
    g = torch.Generator().manual_seed(3)
    q = torch.randint(0, 16, (40, 384), generator=g, dtype=torch.uint8)
    z = torch.randint(0, 16, (40, 12), generator=g, dtype=torch.uint8)
    qw, _, zp = o.rowpack(q, z, torch.ones((40, 12), dtype=torch.bfloat16))
    q2, z2 = o.rowunpack(qw, zp)
    assert torch.equal(q2, q) and torch.equal(z2, z)
    qwc, zpc = cref.rowpack(q, z)
    assert np.array_equal(qwc, qw.numpy().view(np.uint32)) and np.array_equal(zpc, zp.numpy())


# ---------------------------------------------------------------------------- dequant
@pytest.mark.parametrize("d,s_bits,want", [
    (0, 0x3F81, 0x0000),    # q == z gives +0.0
    (15, 0x3F81, 0x4172),   # 15 * 1.0078125 = 15.1171875 -> 15.125 (rounds up)
    (3, 0x3F81, 0x4042),    # 3.0234375: exact tie, odd -> 3.03125
    (5, 0x3F81, 0x40A1),    # 5.0390625 -> 5.03125 (rounds down)
    (-15, 0x3F81, 0xC172),
    (7, 0x3F80, 0x40E0),    # scale 1.0 -> the integer itself
])
def test_dequant_known_answers(d, s_bits, want):
    z0 = 15 if d < 0 else 0
    q = torch.full((1, 32), z0 + d, dtype=torch.uint8)
    z = torch.tensor([[z0]], dtype=torch.uint8)
    s = o.bits_to_bf16(np.array([[s_bits]], dtype=np.uint16))
    out = o.dequantize(q, z, s)
    assert set(_bits(out).flatten().tolist()) == {want}
    assert set(cref.dequant(q, z, s).flatten().tolist()) == {want}


def test_dequant_three_implementations_agree():
    g = torch.Generator().manual_seed(4)
    n, k = 64, 512
    q = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
    z = torch.randint(0, 16, (n, k // 32), generator=g, dtype=torch.uint8)
    s = (torch.rand((n, k // 32), generator=g) * 0.01 + 1e-4).bfloat16()
    a = _bits(o.dequantize(q, z, s))
    b = cref.dequant(q, z, s)
    c = _bits(((q.float() - z.float().repeat_interleave(32, 1)) * s.float().repeat_interleave(32, 1)).bfloat16())
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_zero_point_form_reduces_to_reference_dequant():
    """(u ^ 8) - 8 with z = 8 reproduces calibrated_quant.dequantize on signed codes bit for bit."""
    g = torch.Generator().manual_seed(5)
    codes = torch.randint(-7, 8, (32, 256), generator=g, dtype=torch.int8)
    scales = (torch.rand((32, 8), generator=g) * 0.02 + 1e-5).bfloat16()
    ref = o.dequantize_signed(codes, scales)
    q, z, s = o.signed_export_to_codes(o.pack_signed(codes), scales)
    assert np.array_equal(_bits(o.dequantize(q, z, s)), _bits(ref))
    # the reference's torch expression, evaluated independently
    direct = (codes.float().view(32, -1, 32) * scales.float()[:, :, None]).reshape(32, 256).bfloat16()
    assert np.array_equal(_bits(direct), _bits(ref))


# ------------------------------------------------------------------------- quantizers
def test_minmax_quantizer_brute_force():
    g = torch.Generator().manual_seed(6)
    w = torch.randn((16, 128), generator=g) * 0.02
    q, z, s = o.quantize_minmax_g32(w)
    wn = w.numpy().reshape(16, 4, 32)
    sf = s.float().numpy()
    lo, hi = wn.min(-1), wn.max(-1)
    assert np.array_equal(_bits(s), o.f32_to_bf16_bits(((hi - lo) / np.float32(15)).astype(np.float32)))
    # brute force: the stored code is the nearest representable level to w
    qn = q.numpy().reshape(16, 4, 32).astype(np.int32)
    zn = z.numpy().astype(np.int32)
    levels = (np.arange(16)[None, None, :] - zn[..., None]) * sf[..., None]      # [16, 4, 16]
    err = np.abs(levels[:, :, None, :] - wn[..., None])                            # [16, 4, 32, 16]
    best = err.min(-1)
    got = np.take_along_axis(err, qn[..., None], -1)[..., 0]
    assert np.all(got <= best + 1e-7)
    assert q.max() <= 15 and z.max() <= 15


def test_static_scales_known_answers():
    w = torch.zeros((2, 64))
    w[0, 5] = -7.0
    w[0, 40] = 14.0
    out = _bits(o.static_scales(w))
    assert out[0].tolist() == [0x3F80, 0x4000]
    assert out[1, 0] == o.f32_to_bf16_bits(np.array([np.float32(1e-8) / np.float32(7)], dtype=np.float32))[0]


def test_rowpack_f32_dequant_equals_oracle_dequant():
    """The threaded full-size dequant of the row-packed layout equals ``dequantize(rowunpack(...))``
    bit for bit, including a ragged last 128-group block of zero points (K = 4096 + 2048)."""
    g = torch.Generator().manual_seed(13)
    for n, k in ((40, 256), (8, 6144)):
        q = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
        z = torch.randint(0, 16, (n, k // 32), generator=g, dtype=torch.uint8)
        s = (torch.rand((n, k // 32), generator=g) * 0.01 + 1e-4).bfloat16()
        qw, sc, zp = o.rowpack(q, z, s)
        got = o.dequantize_rowpack_f32(qw, sc, zp)
        assert torch.equal(got, o.dequantize(q, z, s).float())


def _symmetric_brute(w, s):
    """calibrated_quant.py:74-77 by brute force: the fp32 quotient w / s formed exactly and rounded
    once to float32, then the nearest of the 15 levels -7..7 (exact rational distances), ties to the
    even level."""
    out = []
    for v, sv in zip(w, s):
        q = Fraction(rn_f32(Fraction(float(v)) / Fraction(float(sv))))
        best = min(range(-7, 8), key=lambda c: (abs(q - c), c % 2))
        out.append(best)
    return out


def test_quantize_symmetric_brute_force():
    """Random weights of many magnitudes against their own static scales (the export recipe), and
    scales that are not the group's own (so clamping happens): every code is the brute-force level."""
    g = torch.Generator().manual_seed(11)
    mags = 2.0 ** torch.randint(-20, 4, (24, 1), generator=g).float()
    w = torch.randn((24, 64), generator=g) * mags
    w[torch.rand((24, 64), generator=g) < 0.05] = 0
    for s in (o.static_scales(w), (o.static_scales(w).float() * 0.37).bfloat16()):
        c = o.quantize_symmetric(w, s)
        sf = s.float().repeat_interleave(32, 1)
        for r in range(w.shape[0]):
            assert c[r].tolist() == _symmetric_brute(w[r].tolist(), sf[r].tolist()), r
    assert o.quantize_symmetric(w, o.static_scales(w)).abs().max() <= 7


def test_quantize_symmetric_ties_and_clamps():
    """Crafted cases at scale 1 and 0.25: exact half-way values go to the even level, values past
    +-7.5 clamp to +-7, and a zero group (scale floor 1e-8 / 7) gives zero codes."""
    vals = [0.5, 1.5, 2.5, -2.5, 3.5, -3.5, 6.5, -6.5, 7.5, -7.5, 7.49, 8.0, -100.0, 1e30, -0.0, 0.0,
            4.5, 5.5, -0.5, -1.5, 2.4999, 2.5001, 3.0, -7.0, 9.5, -8.5, 0.75, 1.25, 5.0, 6.0, 6.9, -6.9]
    want = [0, 2, 2, -2, 4, -4, 6, -6, 7, -7, 7, 7, -7, 7, 0, 0,
            4, 6, 0, -2, 2, 3, 3, -7, 7, -7, 1, 1, 5, 6, 7, -7]
    for scale in (1.0, 0.25):
        w = torch.tensor([vals], dtype=torch.float32) * scale
        s = torch.full((1, 1), scale).bfloat16()
        assert o.quantize_symmetric(w, s)[0].tolist() == want
    z = torch.zeros((1, 32))
    assert not o.quantize_symmetric(z, o.static_scales(z)).any()


def test_cpu_baseline_dequant_and_linear_match_oracle():
    """The CPU baseline (AutoGPTQ layout, dequantized on every call) against the oracle on the same
    codes: the bf16 weights are bit for bit ``dequantize``'s (transposed), the fp32 outputs agree
    with ``w4g32_linear`` to fp32 summation order (both are F.linear on the same bf16 weights)."""
    g = torch.Generator().manual_seed(12)
    w = torch.randn((96, 256), generator=g) * 0.02
    q, z, s = o.quantize_minmax_g32(w)
    qweight, scales, qzeros = o.pack_gptq(q, z, s)
    wd = o.gptq_dequant_cpu(qweight, scales, qzeros)
    assert np.array_equal(_bits(wd.t().contiguous()), _bits(o.dequantize(q, z, s)))
    x = torch.randn((3, 256), generator=g).bfloat16()
    got = o.gptq_dequant_linear_cpu(x, qweight, scales, qzeros)
    ref = o.w4g32_linear(x, q, z, s)
    bound = 1e-6 * (x.float().abs() @ o.dequantize(q, z, s).float().abs().t()) + 1e-30
    assert torch.all((got - ref).abs() <= bound)
    # a planted swap of code and zero nibble order would change the weights
    bad = o.gptq_dequant_cpu(qweight, scales, torch.flip(qzeros, [1]))
    assert not np.array_equal(_bits(bad), _bits(wd))


# ----------------------------------------------------------------- linear contracts
def test_linear_matches_fp64():
    g = torch.Generator().manual_seed(7)
    x = torch.randn((3, 256), generator=g).bfloat16()
    w = (torch.randn((40, 256), generator=g) * 0.02).bfloat16()
    y = o.linear(x, w).numpy()
    ref = cref.linear_f64(x, w)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_linear_invariants():
    g = torch.Generator().manual_seed(8)
    q = torch.randint(0, 16, (24, 128), generator=g, dtype=torch.uint8)
    z = torch.randint(0, 16, (24, 4), generator=g, dtype=torch.uint8)
    s = (torch.rand((24, 4), generator=g) * 0.01).bfloat16()
    w = o.dequantize(q, z, s)
    e = torch.zeros((1, 128), dtype=torch.bfloat16)
    e[0, 37] = 1.0
    assert torch.equal(o.w4g32_linear(e, q, z, s)[0].bfloat16(), w[:, 37])     # one-hot selects a column
    assert torch.count_nonzero(o.w4g32_linear(torch.zeros((1, 128), dtype=torch.bfloat16), q, z, s)) == 0


def test_silu_mul_rounding_points():
    g = torch.linspace(-12, 12, 4097)
    u = torch.linspace(3, -3, 4097)
    out = o.silu_mul_rounded(g, u).float()
    gb, ub = g.bfloat16().float(), u.bfloat16().float()
    ref = (torch.nn.functional.silu(gb).bfloat16().float() * ub).bfloat16().float()
    # SiLU differs between exp implementations by at most one bf16 step before the product
    diff = (out - ref).abs()
    assert (diff == 0).float().mean() > 0.99
    assert torch.all(diff <= ub.abs() * 2 ** -7 + 1e-30)
