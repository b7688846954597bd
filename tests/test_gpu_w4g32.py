"""GPU parity: INT4-G32 format kernels (bit-exact) and decode GEMVs (tolerance) vs the oracle.

Bars: integer/byte work and the materialized dequant are bit-exact; bf16 GEMV outputs
must satisfy |y - ref| <= 1e-2 + 1e-2 * |ref| against the oracle's dequant-then-matmul
(fp32, CPU) on the same seeded inputs.  Full-size shapes add size-independent properties
that are exact: y(2x) == 2 y(x) and y(e_k) == dequant(W)[:, k].
"""
import pytest
import torch

from helpers import _assert_close, _assert_epilogue_close, _assert_rne_or_adjacent, _bits
from oracle import w4g32 as o

pytestmark = pytest.mark.gpu

def _case(n, k, seed, *, scale=0.02):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn((n, k), generator=g) * scale
    q, z, s = o.quantize_minmax_g32(w)
    return q, z, s


def _packed(q, z, s, dev):
    from moss_tts._runtime.w4g32 import PackedW4G32

    qw, sc, zp = o.rowpack(q, z, s)
    return PackedW4G32(qw.to(dev), sc.to(dev), zp.to(dev))


# ------------------------------------------------------------------ format kernels
@pytest.mark.parametrize("k,n", [(64, 8), (256, 40), (4096, 512), (12288, 64), (2048, 1032)])
def test_repack_gptq_bitexact(dev, k, n):
    from moss_tts._runtime import w4g32

    print(f"repack_gptq K={k} N={n}", flush=True)
    q, z, s = _case(n, k, 11)
    qweight, scales, qzeros = o.pack_gptq(q, z, s)
    out = w4g32.repack_gptq(qweight.to(dev), scales.to(dev), qzeros.to(dev))
    qw, sc, zp = o.rowpack(q, z, s)
    assert torch.equal(out.qw.cpu(), qw)
    assert torch.equal(_bits(out.scales), _bits(sc))
    assert torch.equal(out.zeros.cpu(), zp)


@pytest.mark.parametrize("k,n", [(64, 3), (4096, 256), (12288, 96)])
def test_import_signed_bitexact(dev, k, n):
    from moss_tts._runtime import w4g32

    print(f"import_signed K={k} N={n}", flush=True)
    g = torch.Generator().manual_seed(12)
    codes = torch.randint(-7, 8, (n, k), generator=g, dtype=torch.int8)
    scales_f32 = (torch.rand((n, k // 32), generator=g) * 0.01 + 1e-4).bfloat16().float()
    packed = o.pack_signed(codes)
    out = w4g32.import_signed(packed.to(dev), scales_f32.to(dev))
    q, z, s = o.signed_export_to_codes(packed, scales_f32)
    qw, sc, zp = o.rowpack(q, z, s)
    assert torch.equal(out.qw.cpu(), qw) and torch.equal(out.zeros.cpu(), zp)
    assert torch.equal(_bits(out.scales), _bits(sc))
    # the dequant of the imported weight is the reference's signed dequant, bit for bit
    assert torch.equal(_bits(w4g32.dequantize(out)), _bits(o.dequantize_signed(codes, s)))


def test_import_signed_rejects_inexact_scales(dev):
    from moss_tts._runtime import w4g32

    packed = torch.zeros((2, 32), dtype=torch.uint8, device=dev)
    scales = torch.full((2, 2), 0.1, dtype=torch.float32, device=dev)  # 0.1 is not a bf16 value
    with pytest.raises(ValueError, match="bf16"):
        w4g32.import_signed(packed, scales)


@pytest.mark.parametrize("k,n", [(64, 5), (4096, 128), (12288, 33)])
def test_unpack_and_dequant_bitexact(dev, k, n):
    from moss_tts._runtime import w4g32

    print(f"unpack/dequant K={k} N={n}", flush=True)
    q, z, s = _case(n, k, 13)
    pw = _packed(q, z, s, dev)
    assert torch.equal(w4g32.unpack_codes(pw).cpu(), q)
    assert torch.equal(_bits(w4g32.dequantize(pw)), _bits(o.dequantize(q, z, s)))


@pytest.mark.parametrize("k,n", [(64, 7), (4096, 200), (12288, 40)])
def test_quantize_minmax_bitexact(dev, k, n):
    from moss_tts._runtime import w4g32

    print(f"quantize_minmax K={k} N={n}", flush=True)
    g = torch.Generator().manual_seed(14)
    w = torch.randn((n, k), generator=g) * 0.02
    out = w4g32.quantize_minmax(w.to(dev))
    q, z, s = o.quantize_minmax_g32(w)
    qw, sc, zp = o.rowpack(q, z, s)
    assert torch.equal(out.qw.cpu(), qw) and torch.equal(out.zeros.cpu(), zp)
    assert torch.equal(_bits(out.scales), _bits(sc))


# ------------------------------------------------------------------- decode GEMV
GEMV_SHAPES = [
    (64, 8), (128, 37), (512, 1000), (1536, 768), (2048, 64), (4096, 4096), (4096, 12288),
    (6144, 130), (12288, 4096), (16384, 72),
    (4096, 32802),  # the heads projection (32 x 1025 + 2 rows): four rows per wave in auto mode
]


# explicit rows-per-wave launches at the small shapes; the full-size shapes run the default launch
GEMV_CASES = [(k, n, rows) for k, n in GEMV_SHAPES for rows in ((0, 1, 2, 4) if k * n <= 4096 * 4096 else (0,))]


@pytest.mark.parametrize("k,n,rows", GEMV_CASES)
@pytest.mark.parametrize("mode", ["exact", "unrounded"])
def test_gemv_parity(dev, k, n, rows, mode):
    """Both dequant modes meet the 1e-2 bar; the exact mode multiplies x by the bit-exact bf16
    dequantized weights, so its bf16 outputs equal RNE of the oracle's fp32 result except
    where fp32 summation order moves a value across a rounding midpoint."""
    from moss_tts._runtime import w4g32

    print(f"gemv K={k} N={n} rows={rows} mode={mode}", flush=True)
    q, z, s = _case(n, k, 100 + k + n)
    x = torch.randn((1, k), generator=torch.Generator().manual_seed(1)).bfloat16()
    dq = w4g32.EXACT if mode == "exact" else w4g32.UNROUNDED
    y = w4g32.gemv(x.to(dev), _packed(q, z, s, dev), rows_per_wave=rows, dequant=dq)
    torch.cuda.synchronize()
    ref = o.w4g32_linear(x, q, z, s)
    _assert_close(y, ref, f"gemv K={k} N={n}")
    if mode == "exact":
        abs_sum = o.linear(x.float().abs(), o.dequantize(q, z, s).float().abs())
        _assert_rne_or_adjacent(y, ref, abs_sum, k, f"exact gemv K={k} N={n}")


@pytest.mark.parametrize("k,n_half", [(64, 8), (512, 100), (4096, 12288), (4096, 768)])
@pytest.mark.parametrize("rows", [0, 1, 4])
def test_gateup_silu_parity(dev, k, n_half, rows):
    from moss_tts._runtime import w4g32

    print(f"gateup K={k} N/2={n_half} rows={rows}", flush=True)
    q, z, s = _case(2 * n_half, k, 200 + k + n_half)
    x = torch.randn((1, k), generator=torch.Generator().manual_seed(2)).bfloat16()
    y = w4g32.gateup_silu(x.to(dev), _packed(q, z, s, dev), rows_per_wave=rows)
    torch.cuda.synchronize()
    y32 = o.w4g32_linear(x, q, z, s)
    _assert_epilogue_close(y, y32[:, :n_half], y32[:, n_half:], f"gateup K={k} N/2={n_half}")


@pytest.mark.parametrize("k,n", [(4096, 12288), (12288, 4096)])
@pytest.mark.parametrize("mode", ["exact", "unrounded"])
def test_gemv_exact_properties_full_size(dev, k, n, mode):
    """Size-independent exact checks at full size: power-of-two scaling, one-hot columns
    reproduce the bit-exact dequantized weights, zero input gives zero output."""
    from moss_tts._runtime import w4g32

    print(f"gemv properties K={k} N={n} mode={mode}", flush=True)
    dqm = w4g32.EXACT if mode == "exact" else w4g32.UNROUNDED
    pw = w4g32.quantize_minmax((torch.randn((n, k), device=dev) * 0.02).contiguous())
    x = torch.randn((1, k), device=dev).bfloat16()
    y1 = w4g32.gemv(x, pw, dequant=dqm)
    y2 = w4g32.gemv((x.float() * 2).bfloat16(), pw, dequant=dqm)
    assert torch.equal(y2, (y1.float() * 2).bfloat16())
    dq = w4g32.dequantize(pw)
    for col in (0, 31, 32, k // 2 + 5, k - 1):
        e = torch.zeros((1, k), device=dev, dtype=torch.bfloat16)
        e[0, col] = 1.0
        assert torch.equal(w4g32.gemv(e, pw, dequant=dqm)[0], dq[:, col]), f"one-hot column {col}"
    assert torch.count_nonzero(w4g32.gemv(torch.zeros_like(x), pw, dequant=dqm)) == 0


def _scale_sweep_weight():
    """One 32-code group per (bf16 scale, zero point) for every positive finite bf16 scale (bit patterns
    0x0001..0x7F7F, subnormals included) and all 16 zero points; each group holds every code 0..15
    twice, rotated by the group index so every code meets every nibble position.  Rows of K = 4096
    (8 scales each); the scales below 2^120 (0x7B80) fill whole rows, padded with scale 1, ahead of
    the larger ones, and the groups that pad the last row use scale 1."""
    below = torch.arange(1, 0x7B80, dtype=torch.int32)                     # 0x7F80 is +inf
    pad = torch.full((-below.numel() % 8,), 0x3F80, dtype=torch.int32)
    scales = torch.cat([below, pad, torch.arange(0x7B80, 0x7F80, dtype=torch.int32)])
    n_groups = scales.numel() * 16
    k, gpr = 4096, 128
    rows = -(-n_groups // gpr)
    s_bits = torch.full((rows * gpr,), 0x3F80, dtype=torch.int32)
    s_bits[:n_groups] = scales.repeat_interleave(16)
    z = torch.zeros(rows * gpr, dtype=torch.int32)
    z[:n_groups] = torch.arange(16, dtype=torch.int32).repeat(scales.numel())
    gi = torch.arange(rows * gpr, dtype=torch.int32)[:, None]
    q = (torch.arange(32, dtype=torch.int32)[None, :] + gi) % 16
    s = s_bits.to(torch.int16).view(torch.bfloat16).view(rows, gpr)
    return q.view(rows, k).to(torch.uint8), z.view(rows, gpr).to(torch.uint8), s, scales


def test_exact_dequant_every_bf16_scale(dev):
    """The bit-exact dequant bf16_rne((q - z) * s) over all 16 x 16 (q, z) pairs and every positive
    finite bf16 scale, in the three places it is formed: the dequant kernel (plain fp32 product),
    the decode GEMV's exact mode (one-hot activations select each column; the v_dot2 / v_fma_mix
    block) and the prefill GEMM's producer (identity activations give the whole matrix; same
    block).  The dequant kernel must equal the oracle bit for bit everywhere.  The GEMV and GEMM
    form (128 + q) s in fp32, finite below 2^120.8, so they are held to every scale below 2^120 (the
    bound the loaders enforce; 31,615 scales, subnormals included)."""
    from moss_tts._runtime import w4g32

    print("exact dequant over every positive finite bf16 scale", flush=True)
    q, z, s, scales = _scale_sweep_weight()
    n, k = q.shape
    ref = _bits(o.dequantize(q, z, s))
    pw = _packed(q, z, s, dev)
    assert torch.equal(_bits(w4g32.dequantize(pw)), ref), "dequant kernel"
    s_bits = s.contiguous().view(torch.int16).to(torch.int32)
    finite_rows = (s_bits < 0x7B80).all(1)                                 # 0x7B80 = 2^120
    assert int(torch.unique(s_bits[finite_rows]).numel()) == 0x7B7F       # every scale below 2^120

    def check(got_t, what):
        bad = (got_t != ref) & finite_rows[:, None]
        nbad = int(bad.sum())
        if nbad:
            rows_bad = bad.view(n, 128, 32).any(-1)
            lo = int(s_bits[rows_bad].min())
            print(f"{what}: {nbad} mismatches; smallest scale with one: 0x{lo:04x}", flush=True)
        assert nbad == 0, what

    eye = torch.eye(k, dtype=torch.bfloat16, device=dev)
    gemm = w4g32.gemm(eye, pw)                                             # [K, N] = dequant(W)^T
    torch.cuda.synchronize()
    check(_bits(gemm).t(), "GEMM producer")
    cols = torch.empty((k, n), dtype=torch.bfloat16, device=dev)
    for c in range(k):
        cols[c] = w4g32.gemv(eye[c:c + 1], pw)[0]
    torch.cuda.synchronize()
    check(_bits(cols).t(), "GEMV exact mode")


def test_loaders_reject_scales_outside_the_exact_range(dev):
    from moss_tts._runtime import w4g32

    big = torch.full((8, 2), 2.0 ** 121, device=dev).bfloat16()
    q, z, s = _case(8, 64, 5)
    qweight, _, qzeros = o.pack_gptq(q, z, s)
    with pytest.raises(ValueError, match="2\\^120"):
        w4g32.repack_gptq(qweight.to(dev), big.t().contiguous(), qzeros.to(dev))
    with pytest.raises(ValueError, match="2\\^120"):
        w4g32.import_signed(torch.zeros((8, 32), dtype=torch.uint8, device=dev), big)
    with pytest.raises(ValueError, match="2\\^120"):
        w4g32.quantize_minmax(torch.full((8, 64), 3e38, device=dev) * torch.tensor([1.0, -1.0], device=dev).repeat(32))


def test_gemv_rejects_bad_inputs(dev):
    from moss_tts._runtime import w4g32

    pw = w4g32.quantize_minmax(torch.randn((64, 128), device=dev))
    with pytest.raises(ValueError):
        w4g32.gemv(torch.randn((1, 128), device=dev), pw)                  # fp32 activations
    with pytest.raises(ValueError):
        w4g32.gemv(torch.randn((1, 64), device=dev).bfloat16(), pw)        # K mismatch
    with pytest.raises(ValueError):
        w4g32.gemv(torch.randn((1, 128)).bfloat16(), pw)                   # host tensor
    with pytest.raises(ValueError):
        w4g32.gemv(torch.randn((1, 128), device=dev).bfloat16(), pw, rows_per_wave=3)
    with pytest.raises(ValueError):
        w4g32.gemv(torch.randn((1, 128), device=dev).bfloat16(), pw, dequant=2)
    with pytest.raises(ValueError):
        w4g32.gemv(torch.randn((5, 128), device=dev).bfloat16(), pw)        # at most 4 rows
    with pytest.raises(ValueError):
        w4g32.gemv(torch.randn((2, 128), device=dev).bfloat16(), pw, dequant=w4g32.UNROUNDED)
    pw6 = w4g32.quantize_minmax(torch.randn((8, 6144), device=dev))
    with pytest.raises(ValueError):
        w4g32.gemv(torch.randn((2, 6144), device=dev).bfloat16(), pw6)      # several rows: K shape


@pytest.mark.parametrize("k,n", [(64, 8), (2112, 129), (3072, 777), (4096, 4096), (4096, 6144), (8192, 2048),
                                 (12288, 4100), (16384, 1024),
                                 # ragged last workgroup: 4 rows per wave (N = 4094) / per K-split group (4099)
                                 (4096, 4094), (12288, 4099)])
def test_gemv_tokens_equal_single_token_gemv(dev, k, n):
    """2 to 4 tokens in one pass over the weights: every output row equals the one-token GEMV of
    its input row bit for bit (same per-lane dot2 chain, same cross-lane sum), the GEMM takes that
    path for 2 and 3 tokens (4 where K <= 4096), and the result is within the oracle's bar."""
    from moss_tts._runtime import w4g32

    q, z, s = _case(n, k, 900 + k + n)
    pw = _packed(q, z, s, dev)
    dq = o.dequantize(q, z, s)
    for m in (2, 3, 4):
        print(f"gemv tokens M={m} K={k} N={n}", flush=True)
        x = torch.randn((m, k), generator=torch.Generator().manual_seed(m + k)).bfloat16().to(dev)
        y = w4g32.gemv(x, pw)
        single = torch.cat([w4g32.gemv(x[r:r + 1].contiguous(), pw) for r in range(m)])
        assert torch.equal(y, single), f"M={m} K={k} N={n}: rows differ from the one-token GEMV"
        if m <= 3 or k <= 4096:
            assert torch.equal(w4g32.gemm(x, pw), single), f"M={m} K={k} N={n}: the GEMM took another path"
        _assert_close(y, o.linear(x.cpu(), dq), f"gemv tokens M={m} K={k} N={n}")


# ------------------------------------------------------------------- prefill GEMM
@pytest.mark.parametrize("m,k,n", [(2, 64, 8), (16, 128, 64), (100, 512, 200), (128, 4096, 128), (512, 1024, 4096),
                                   (37, 4096, 32800), (512, 4096, 6144), (512, 12288, 4096), (512, 4096, 4096),
                                   # the 128 x 128 tile at full size, with ragged M and N, and an odd step count
                                   (512, 4096, 24576), (300, 1024, 32808), (260, 1088, 16448),
                                   # register-weight tile with a 16-group last zero-point chunk (G = 144)
                                   (260, 4608, 12296),
                                   # 32- and 64-token register tiles with a K split, ragged N
                                   (5, 1024, 1000), (16, 4096, 4096), (48, 4608, 2056),
                                   # N % 4 != 0: the LDS tiles take shapes the register tile would
                                   (40, 4096, 1001), (130, 4096, 258),
                                   # the small-M weight-streaming kernel (M <= 32, K % 4096 == 0): one
                                   # and two token tiles, ragged tiles, a ragged last row tile, K = 12288
                                   (1, 4096, 2048), (2, 4096, 4096), (7, 4096, 4096), (15, 4096, 4096),
                                   (4, 12288, 4096),
                                   (17, 4096, 2052), (32, 12288, 4096), (25, 4096, 12296),
                                   # just past it: the tiles again
                                   (33, 4096, 6144), (64, 4096, 4096), (50, 12288, 4100)])
def test_gemm_parity(dev, m, k, n):
    """MFMA GEMM with bit-exact bf16 dequantized weights: fp32 summation order is the only
    difference from the oracle's dequant-then-matmul."""
    from moss_tts._runtime import w4g32

    print(f"gemm M={m} K={k} N={n}", flush=True)
    q, z, s = _case(n, k, 300 + m + k + n)
    x = torch.randn((m, k), generator=torch.Generator().manual_seed(4)).bfloat16()
    y = w4g32.gemm(x.to(dev), _packed(q, z, s, dev))
    torch.cuda.synchronize()
    dq = o.dequantize(q, z, s)
    ref = o.linear(x, dq)
    _assert_close(y, ref, f"gemm M={m} K={k} N={n}")
    abs_sum = o.linear(x.float().abs(), dq.float().abs())
    _assert_rne_or_adjacent(y, ref, abs_sum, k, f"gemm M={m} K={k} N={n}")


@pytest.mark.parametrize("m,k,n,fused", [(512, 4096, 12288, True), (65, 4096, 12288, True), (200, 4096, 12260, True),
                                         (64, 4096, 12288, False), (16, 4096, 12288, False), (700, 4096, 256, False),
                                         (128, 1024, 100, False), (3, 4096, 512, False)])
def test_gemm_silu_equals_gemm_then_silu(dev, m, k, n, fused):
    """The gate||up GEMM with the SiLU*mul epilogue equals the GEMM of all 2 N rows followed by
    silu_mul, bit for bit: fused in the 128-token tile (M > 64 with no K split in the plan) and
    through the workspace otherwise (64 tokens or fewer, or few enough tiles that K is split).  The
    fused tile is the one that runs without any workspace; the other shapes refuse that call."""
    from moss_tts._runtime import native, pointwise, w4g32

    print(f"gemm_silu M={m} K={k} N={n} fused={fused}", flush=True)
    g = torch.Generator(device=dev).manual_seed(m + k + n)
    pw = w4g32.quantize_minmax(torch.randn((2 * n, k), device=dev, generator=g) * 0.02)
    x = torch.randn((m, k), device=dev, generator=g).bfloat16()
    want = pointwise.silu_mul(w4g32.gemm(x, pw))
    got = w4g32.gemm_silu(x, pw)
    assert got.shape == (m, n)
    assert torch.equal(got, want)
    bare = torch.full_like(got, float("nan"))
    rc = native.lib().moss_w4g32_gemm_silu(native.ptr(x), native.ptr(pw.qw), native.ptr(pw.scales),
                                           native.ptr(pw.zeros), native.ptr(bare), m, k, n, None, 0,
                                           native.stream_of(x))
    assert (rc == 0) == fused and (rc == 0 or rc == 1)
    if fused:
        assert torch.equal(bare, want)


@pytest.mark.parametrize("m,fused", [(512, True), (600, True), (257, True), (128, False), (37, False), (2, False)])
def test_gemm_qk_rope_equals_gemm_then_qk_rope(dev, m, fused):
    """The QKV projection with the q/k-norm + RoPE + KV write epilogue equals the GEMM followed by
    ``qk_rope`` bit for bit: the query heads, every K/V row written and every row left alone (token
    positions scattered over the cache, one clamped from past its end)."""
    from moss_tts._runtime import native, pointwise, w4g32

    print(f"gemm + qk rope M={m} fused={fused}", flush=True)
    g = torch.Generator(device=dev).manual_seed(m)
    L = 1024
    w = w4g32.quantize_minmax(torch.randn((6144, 4096), device=dev, generator=g) * 0.02)
    x = torch.randn((m, 4096), device=dev, generator=g).bfloat16()
    qn = (1 + 0.1 * torch.randn(128, device=dev, generator=g)).bfloat16()
    kn = (1 + 0.1 * torch.randn(128, device=dev, generator=g)).bfloat16()
    ang = torch.arange(L, device=dev)[:, None] * (1e-3 * torch.arange(1, 129, device=dev))[None, :]
    cos, sin = ang.cos().bfloat16().contiguous(), ang.sin().bfloat16().contiguous()
    pos = torch.randperm(L - 1, device=dev, generator=g)[:m].to(torch.int64)
    pos[0] = L + 5  # clamped to row L - 1
    base_k = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    base_v = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    k1, v1, k2, v2 = base_k.clone(), base_v.clone(), base_k.clone(), base_v.clone()
    q1 = w4g32.gemm_qk_rope(x, w, qn, kn, cos, sin, k1, v1, pos, 1e-6)
    q2 = pointwise.qk_rope(w4g32.gemm(x, w), qn, kn, cos, sin, k2, v2, pos, 1e-6, cos_by_position=True)
    torch.cuda.synchronize()
    assert torch.equal(q1.contiguous().view(torch.int16), q2.contiguous().view(torch.int16))
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))
    untouched = torch.ones(L, dtype=torch.bool, device=dev)
    untouched[pos.clamp(0, L - 1)] = False
    assert torch.equal(k1[:, :, untouched].view(torch.int16), base_k[:, :, untouched].view(torch.int16))
    # the fused tile is the form that runs without any workspace; the other shapes refuse that call
    k3, v3 = base_k.clone(), base_v.clone()
    q3 = torch.empty((m, 32, 128), device=dev, dtype=torch.bfloat16)
    lib = native.lib()
    rc = lib.moss_w4g32_gemm_qk_rope(native.ptr(x), native.ptr(w.qw), native.ptr(w.scales), native.ptr(w.zeros),
                                     native.ptr(qn), native.ptr(kn), native.ptr(cos), native.ptr(sin), native.ptr(q3),
                                     native.ptr(k3), native.ptr(v3), native.ptr(pos), m, 4096, L, 1e-6, None, 0,
                                     native.stream_of(x))
    assert (rc == 0) == fused and (rc == 0 or rc == 1)
    if fused:
        torch.cuda.synchronize()
        assert torch.equal(q3.view(torch.int16), q2.transpose(1, 2).contiguous().view(m, 32, 128).view(torch.int16))
        assert torch.equal(k3.view(torch.int16), k2.view(torch.int16))


@pytest.mark.parametrize("m,k,n", [(512, 4096, 4096), (512, 12288, 4096), (1024, 4096, 4096), (64, 4096, 4096),
                                   (16, 4096, 4096), (200, 1024, 512), (3, 4096, 4096)])
def test_gemm_add_rmsnorm_equals_gemm_then_add_rmsnorm(dev, m, k, n):
    """The projection followed by the residual add and RMSNorm equals gemm then add_rmsnorm bit for
    bit, with the split-K reduction inside the norm kernel (M=512 O and down, and the other split
    plans) and without (M=1024, the streaming kernel)."""
    from moss_tts._runtime import native, pointwise, w4g32

    split = native.lib().moss_gemm_workspace_bytes(m, k, n) // (m * n * 4)
    print(f"gemm_add_rmsnorm M={m} K={k} N={n} split={split}", flush=True)
    g = torch.Generator(device=dev).manual_seed(3 * m + k + n)
    pw = w4g32.quantize_minmax(torch.randn((n, k), device=dev, generator=g) * 0.02)
    x = torch.randn((m, k), device=dev, generator=g).bfloat16()
    res = torch.randn((m, n), device=dev, generator=g).bfloat16()
    nw = (1 + 0.05 * torch.randn(n, device=dev, generator=g)).bfloat16()
    want_s, want_y = pointwise.add_rmsnorm(w4g32.gemm(x, pw), res, nw, 1e-6)
    got_s, got_y = w4g32.gemm_add_rmsnorm(x, pw, res, nw, 1e-6)
    assert torch.equal(got_s, want_s) and torch.equal(got_y, want_y)


@pytest.mark.parametrize("m,k,n", [(512, 4096, 4096), (48, 4096, 2056)])
def test_gemm_fallbacks_match(dev, m, k, n):
    """The C-ABI's fallbacks give the same products: without a workspace the planned K split is
    dropped (one pass over K), and scales or zero points that are not 16 / 8-byte aligned send the
    register-weight tile's shapes to the LDS tiles.  Against the oracle at the GEMM tolerance."""
    from moss_tts._runtime import native

    print(f"gemm fallbacks M={m} K={k} N={n}", flush=True)
    q, z, s = _case(n, k, 700 + m)
    pw = _packed(q, z, s, dev)
    x = torch.randn((m, k), generator=torch.Generator().manual_seed(9)).bfloat16()
    xd = x.to(dev)
    ref = o.linear(x, o.dequantize(q, z, s))
    assert native.lib().moss_gemm_workspace_bytes(m, k, n) > 0  # these shapes plan a K split

    def run(sc, zp, ws, wb):
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        native.call("moss_w4g32_gemm", native.ptr(xd), native.ptr(pw.qw), native.ptr(sc), native.ptr(zp),
                    native.ptr(y), m, k, n, ws, wb, native.stream_of(xd))
        torch.cuda.synchronize()
        return y

    # no workspace: K is not split
    _assert_close(run(pw.scales, pw.zeros, None, 0), ref, f"gemm M={m} no workspace")
    # scales at +2 bytes and zero points at +1 byte from an aligned base
    sc_buf = torch.empty(pw.scales.numel() + 8, dtype=torch.bfloat16, device=dev)
    zp_buf = torch.empty(pw.zeros.numel() + 16, dtype=torch.uint8, device=dev)
    sc_off = sc_buf[1:1 + pw.scales.numel()].view(pw.scales.shape)
    zp_off = zp_buf[1:1 + pw.zeros.numel()].view(pw.zeros.shape)
    sc_off.copy_(pw.scales)
    zp_off.copy_(pw.zeros)
    assert sc_off.data_ptr() % 16 != 0 and zp_off.data_ptr() % 8 != 0
    wp, wb, _keep = native.gemm_workspace(m, k, n, dev)
    _assert_close(run(sc_off, zp_off, wp, wb), ref, f"gemm M={m} misaligned scales")


def test_gemm_rows_match_gemv(dev):
    """Row r of the GEMM equals the exact-dequant GEMV of x[r] up to fp32 summation order."""
    from moss_tts._runtime import w4g32

    pw = w4g32.quantize_minmax((torch.randn((4096, 4096), device=dev) * 0.02).contiguous())
    x = torch.randn((64, 4096), device=dev).bfloat16()
    y = w4g32.gemm(x, pw).float()
    for r in (0, 17, 63):
        g = w4g32.gemv(x[r:r + 1].contiguous(), pw).float()
        assert torch.allclose(y[r], g[0], atol=2e-2, rtol=1e-2)


# ------------------------------------------------------- fused (add+)RMSNorm + GEMV
@pytest.mark.parametrize("k,n,paired", [(4096, 6144, False), (4096, 12288, True), (2048, 200, False),
                                        (8192, 64, True), (4096, 32800, False)])
@pytest.mark.parametrize("mode", ["exact", "unrounded"])
@pytest.mark.parametrize("residual", [False, True])
def test_norm_gemv_equals_rmsnorm_then_gemv(dev, k, n, paired, mode, residual):
    """The fused kernel reproduces moss_rmsnorm followed by the GEMV bit for bit (same rounding
    points and summation order); the residual sum is bf16(x + r) exactly."""
    from moss_tts._runtime import pointwise, w4g32

    print(f"norm gemv K={k} N={n} paired={paired} mode={mode} residual={residual}", flush=True)
    dq = w4g32.EXACT if mode == "exact" else w4g32.UNROUNDED
    g = torch.Generator(device=dev).manual_seed(k + n)
    pw = w4g32.quantize_minmax((torch.randn((n, k), device=dev, generator=g) * 0.02).contiguous())
    x = (torch.randn((1, k), device=dev, generator=g) * 3).bfloat16()
    nw = (1 + 0.01 * torch.randn(k, device=dev, generator=g)).bfloat16()
    r = (torch.randn((1, k), device=dev, generator=g) * 5).bfloat16() if residual else None
    fused = w4g32.norm_gateup_silu if paired else w4g32.norm_gemv
    plain = w4g32.gateup_silu if paired else w4g32.gemv
    out = fused(x, nw, 1e-6, pw, residual=r, dequant=dq)
    if residual:
        s, y = out
        s_ref, h = pointwise.add_rmsnorm(x, r, nw, 1e-6)
        assert torch.equal(s, s_ref)
    else:
        y, h = out, pointwise.rmsnorm(x, nw, 1e-6)
    assert torch.equal(y, plain(h, pw, dequant=dq))


def test_norm_gemv_parity_with_oracle(dev):
    from moss_tts._runtime import w4g32
    from oracle import pointwise as op

    q, z, s = _case(6144, 4096, 17)
    x = (torch.randn((1, 4096), generator=torch.Generator().manual_seed(9)) * 2).bfloat16()
    r = torch.randn((1, 4096), generator=torch.Generator().manual_seed(10)).bfloat16()
    nw = (1 + 0.01 * torch.randn(4096, generator=torch.Generator().manual_seed(11))).bfloat16()
    summed, y = w4g32.norm_gemv(x.to(dev), nw.to(dev), 1e-6, _packed(q, z, s, dev), residual=r.to(dev))
    s_ref, h_ref = op.add_rmsnorm(x, r, nw, 1e-6)
    assert torch.equal(summed.cpu(), s_ref)
    _assert_close(y, o.w4g32_linear(h_ref, q, z, s), "norm gemv vs oracle")


def test_norm_gemv_rejects_bad_inputs(dev):
    from moss_tts._runtime import native, w4g32

    pw = w4g32.quantize_minmax(torch.randn((64, 4096), device=dev))
    x = torch.randn((1, 4096), device=dev).bfloat16()
    nw = torch.ones(4096, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        w4g32.norm_gemv(x, nw[:2048], 1e-6, pw)
    pw2 = w4g32.quantize_minmax(torch.randn((64, 1024), device=dev))
    with pytest.raises(ValueError):
        w4g32.norm_gemv(x[:, :1024].contiguous(), nw[:1024].contiguous(), 1e-6, pw2)     # K % 2048
    y = torch.empty((1, 64), device=dev, dtype=torch.bfloat16)
    rc = native.lib().moss_w4g32_norm_gemv(native.ptr(x), native.ptr(x), native.ptr(nw), native.ptr(x), 1e-6,
                                           native.ptr(pw.qw), native.ptr(pw.scales), native.ptr(pw.zeros),
                                           native.ptr(y), 4096, 64, 0, 0, native.stream_of(x))
    assert rc == 1                                                   # sum_out overlaps x


@pytest.mark.parametrize("k,n", [(64, 7), (4096, 200), (12288, 40), (4608, 16)])
def test_quantize_symmetric_bitexact(dev, k, n):
    """The device's static-scale symmetric quantizer equals the oracle's ``static_scales`` +
    ``quantize_symmetric`` bit for bit (codes stored as c + 8 with zero point 8), including groups of
    zeros (the 1e-8 floor) and ties; the module's ``from_float(symmetric=True)`` holds the same."""
    from moss_tts._runtime import w4g32
    from moss_tts._runtime.modules import QuantLinearG32

    print(f"quantize_symmetric K={k} N={n}", flush=True)
    g = torch.Generator().manual_seed(15)
    w = torch.randn((n, k), generator=g) * 0.02
    w[0, :32] = 0.0                                            # a zero group: the 1e-8 / 7 scale
    w[1, :32] = torch.arange(32).float() * 0.5                 # max 15.5: scale bf16(15.5 / 7), with ties
    out = w4g32.quantize_symmetric(w.to(dev))
    s = o.static_scales(w)
    c = o.quantize_symmetric(w, s)
    q, z, s2 = o.signed_export_to_codes(o.pack_signed(c), s)
    qw, sc, zp = o.rowpack(q, z, s2)
    assert torch.equal(out.qw.cpu(), qw) and torch.equal(out.zeros.cpu(), zp)
    assert torch.equal(_bits(out.scales), _bits(sc))
    mod = QuantLinearG32.from_float(w.to(dev), symmetric=True)
    assert torch.equal(mod.qw.cpu(), qw)
    assert torch.equal(_bits(w4g32.dequantize(out)), _bits(o.dequantize_signed(c, s)))
