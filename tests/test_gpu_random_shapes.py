"""GPU parity at seeded random shapes inside the documented limits, beside the hand-picked shapes of
the other tests: INT4-G32 GEMV and gate||up (both dequant modes, every rows-per-wave choice), the
same with the (add-)RMSNorm fused in (bit-identical to norm then projection), the W4A8 integer-dot
GEMV and gate||up, the INT4 GEMM (small-M streaming, tiles, K splits), the FP8 linear (GEMV and
GEMM), and decode and prompt attention at random cache lengths, positions and start rows.

Reference: fp32 torch math on the same inputs; for INT4 the weights are the bit-exact dequant
(itself pinned bit for bit against the oracle in test_gpu_w4g32.py), for FP8 the exact e4m3 -> bf16
values times the row scale, for attention softmax(q k^T / sqrt(128)) v over the visible rows with
query head h reading KV head h / 4.  Bar: relative L2 error of the bf16 output below 1e-2 (the
outputs are rounded to bf16 once; the worst case seen over 510 random cases was 7e-3, for the
gate||up SiLU*mul, which rounds three times).
"""
import math
import random

import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 1e-2
_rng = random.Random(20261202)


def _gemv_cases(count):
    out = []
    for _ in range(count):
        out.append((64 * _rng.randint(1, 256), _rng.randint(1, 5000), _rng.choice((0, 1, 2, 4)), _rng.choice((0, 1))))
    return out


def _gemm_cases(count):
    out = []
    for _ in range(count):
        m = _rng.choice((_rng.randint(2, 40), _rng.randint(2, 600)))
        k = 4096 * _rng.randint(1, 3) if _rng.random() < 0.3 else 64 * _rng.randint(1, 192)
        n = _rng.randint(1, 5000) if _rng.random() < 0.5 else 4 * _rng.randint(512, 1500)
        out.append((m, k, n))
    return out


def _fp8_cases(count):
    out = []
    for _ in range(count):
        m = _rng.choice((1, 1, _rng.randint(2, 80)))
        out.append((m, (16 if m == 1 else 64) * _rng.randint(1, 200), _rng.randint(1, 6000)))
    return out


def _decode_cases(count):
    out = []
    for _ in range(count):
        L = 64 * _rng.randint(1, 64)
        out.append((L, _rng.randint(0, L - 1)))
    return out


def _prefill_cases(count):
    out = []
    for _ in range(count):
        L = 64 * _rng.randint(1, 40)
        n = _rng.randint(1, min(L, 1100))
        out.append((L, n, _rng.randint(0, L - n)))
    return out


def _norm_cases(count):
    out = []
    for _ in range(count):
        out.append((2048 * _rng.choice((1, 2, 4)), 2 * _rng.randint(1, 3000), _rng.choice((0, 1, 2, 4)),
                    _rng.random() < 0.5))
    return out


def _w4a8_cases(count):
    out = []
    for _ in range(count):
        out.append((64 * _rng.randint(1, 256), 2 * _rng.randint(1, 3000), _rng.choice((0, 1, 2, 4))))
    return out


def _bf16_cases(count):
    out = []
    for _ in range(count):
        out.append((512 * _rng.choice((1, 2, 3, 4, 5, 6, 7, 8, 12, 16)), _rng.randint(1, 5000),
                    _rng.choice((0, 1, 2, 4))))
    return out


def _w4a8_norm_cases(count):
    out = []
    for _ in range(count):
        out.append((2048 * _rng.choice((1, 2, 4)), 2 * _rng.randint(1, 3000), _rng.random() < 0.5,
                    _rng.random() < 0.5, _rng.choice((0, 1, 2, 4))))
    return out


GEMV = _gemv_cases(12)
NORM = _norm_cases(8)
W4A8 = _w4a8_cases(8)
GEMM = _gemm_cases(12)
FP8 = _fp8_cases(12)
DECODE = _decode_cases(12)
PREFILL = _prefill_cases(12)
BF16 = _bf16_cases(8)
BF16_NORM = [(2048 * _rng.choice((1, 2, 4)), _rng.randint(1, 5000), _rng.random() < 0.5) for _ in range(6)]
FP8_GATEUP = [(16 * _rng.randint(1, 512), _rng.randint(1, 3000), _rng.choice((0, 1, 2, 4))) for _ in range(8)]
W4A8_NORM = _w4a8_norm_cases(8)
GEMM_ADDNORM = [(_rng.choice((_rng.randint(2, 64), _rng.randint(65, 1100))), 64 * _rng.choice((16, 64, 192)),
                 8 * _rng.randint(1, 1024)) for _ in range(8)]
GEMM_SILU = [(_rng.choice((_rng.randint(2, 64), _rng.randint(65, 700))), 64 * _rng.choice((16, 64, 128, 192)),
              4 * _rng.randint(1, 3500)) for _ in range(8)]
GEMM_QK_ROPE = [(_rng.randint(1, 1100), 64 * _rng.choice((16, 64, 128)), 64 * _rng.randint(18, 40)) for _ in range(6)]


def _rel(a, b):
    a, b = a.float(), b.float()
    return float((a - b).norm() / b.norm().clamp_min(1e-12))


def _packed(n, k, seed, dev):
    from moss_tts._runtime import w4g32

    g = torch.Generator(device=dev).manual_seed(seed)
    return w4g32.quantize_minmax(torch.randn((n, k), device=dev, generator=g) * 0.02), g


@pytest.mark.parametrize("k,n,rows,mode", GEMV)
def test_gemv_random_shape(dev, k, n, rows, mode):
    from moss_tts._runtime import w4g32

    print(f"gemv K={k} N={n} rows={rows} mode={mode}", flush=True)
    pw, g = _packed(n, k, k + n, dev)
    x = torch.randn((1, k), device=dev, generator=g).bfloat16()
    ref = x.float() @ w4g32.dequantize(pw).float().t()
    assert _rel(w4g32.gemv(x, pw, rows_per_wave=rows, dequant=mode), ref) < TOL
    if n % 2 == 0:
        half = n // 2
        gate, up = ref[:, :half].bfloat16().float(), ref[:, half:].bfloat16().float()
        want = torch.nn.functional.silu(gate).bfloat16().float() * up
        assert _rel(w4g32.gateup_silu(x, pw, rows_per_wave=rows, dequant=mode), want) < TOL


@pytest.mark.parametrize("k,n,rows,residual", NORM)
def test_fused_norm_random_shape(dev, k, n, rows, residual):
    """The (add-)RMSNorm fused into the GEMV and the gate||up equals norm then projection bit for bit
    for K <= 4096; at K = 8192 the plain projection splits K over two waves, so the two agree to the
    bar instead (same normalized row, different fp32 summation order)."""
    from moss_tts._runtime import pointwise, w4g32

    print(f"fused norm K={k} N={n} rows={rows} residual={residual}", flush=True)
    pw, g = _packed(n, k, 7 * k + n, dev)
    x = torch.randn((1, k), device=dev, generator=g).bfloat16()
    res = torch.randn((1, k), device=dev, generator=g).bfloat16() if residual else None
    nw = (1 + 0.01 * torch.randn(k, device=dev, generator=g)).bfloat16()
    if residual:
        summed, xn = pointwise.add_rmsnorm(x, res, nw, 1e-6)
        s2, y = w4g32.norm_gemv(x, nw, 1e-6, pw, residual=res, rows_per_wave=rows)
        s3, yg = w4g32.norm_gateup_silu(x, nw, 1e-6, pw, residual=res, rows_per_wave=rows)
        assert torch.equal(s2, summed) and torch.equal(s3, summed)
    else:
        xn = pointwise.rmsnorm(x, nw, 1e-6)
        y = w4g32.norm_gemv(x, nw, 1e-6, pw, rows_per_wave=rows)
        yg = w4g32.norm_gateup_silu(x, nw, 1e-6, pw, rows_per_wave=rows)
    y_ref = w4g32.gemv(xn, pw, rows_per_wave=rows)
    yg_ref = w4g32.gateup_silu(xn, pw, rows_per_wave=rows)
    if k <= 4096:
        assert torch.equal(y, y_ref) and torch.equal(yg, yg_ref)
    else:
        assert _rel(y, y_ref) < TOL and _rel(yg, yg_ref) < TOL


@pytest.mark.parametrize("k,n,rows", W4A8)
def test_w4a8_random_shape(dev, k, n, rows):
    """The integer-dot GEMV and gate||up against fp32 math on the same int8 activations (codes times
    group scales) and the dequantized weights."""
    from moss_tts._runtime import w4a8, w4g32

    print(f"w4a8 K={k} N={n} rows={rows}", flush=True)
    pw, g = _packed(n, k, 11 * k + n, dev)
    x = torch.randn((1, k), device=dev, generator=g).bfloat16()
    act = w4a8.quantize(x.view(-1))
    xq = (act.natural().float().view(-1, 32) * act.scales.view(-1, 1)).view(1, k)
    ref = xq @ w4g32.dequantize(pw).float().t()
    assert _rel(w4a8.linear(None, pw, prequantized=act, rows_per_wave=rows), ref) < TOL
    half = n // 2
    gate, up = ref[:, :half].bfloat16().float(), ref[:, half:].bfloat16().float()
    want = torch.nn.functional.silu(gate).bfloat16().float() * up
    assert _rel(w4a8.linear(None, pw, paired=True, prequantized=act, rows_per_wave=rows), want) < TOL


@pytest.mark.parametrize("m,k,n", GEMM)
def test_gemm_random_shape(dev, m, k, n):
    from moss_tts._runtime import w4g32

    print(f"gemm M={m} K={k} N={n}", flush=True)
    pw, g = _packed(n, k, m + k + n, dev)
    x = torch.randn((m, k), device=dev, generator=g).bfloat16()
    ref = x.float() @ w4g32.dequantize(pw).float().t()
    assert _rel(w4g32.gemm(x, pw), ref) < TOL


@pytest.mark.parametrize("m,k,n", FP8)
def test_fp8_linear_random_shape(dev, m, k, n):
    from moss_tts._runtime import fp8

    print(f"fp8 M={m} K={k} N={n}", flush=True)
    g = torch.Generator(device=dev).manual_seed(m + k + n)
    wb = torch.randint(0, 256, (n, k), device=dev, dtype=torch.uint8, generator=g)
    wb[(wb & 0x7F) == 0x7F] = 0  # no NaN codes
    s = torch.rand((n,), device=dev, generator=g) + 0.5
    x = torch.randn((m, k), device=dev, generator=g).bfloat16()
    ref = (x.float() @ fp8.to_bf16(wb).float().t()) * s
    assert _rel(fp8.linear(x, wb, s), ref) < TOL


def _attention_ref(q, kc, vc, last_row):
    """q fp32-able [T, 32, 128], caches [8, L, 128]; token t sees rows 0 .. last_row[t]."""
    out = torch.empty((q.shape[0], 32, 128), device=q.device)
    rows = torch.arange(kc.shape[1], device=q.device)[None, :]
    for h in range(32):
        kh, vh = kc[h // 4].float(), vc[h // 4].float()
        sc = (q[:, h].float() @ kh.t()) / math.sqrt(128)
        sc = sc.masked_fill(rows > last_row[:, None], float("-inf"))
        out[:, h] = torch.softmax(sc, -1) @ vh
    return out


@pytest.mark.parametrize("L,p", DECODE)
def test_decode_attention_random_shape(dev, L, p):
    from moss_tts._runtime import attention

    print(f"decode attention L={L} p={p}", flush=True)
    g = torch.Generator(device=dev).manual_seed(L + p)
    q = torch.randn((32, 128), device=dev, generator=g).bfloat16()
    kc = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    y = attention.decode_attention(q, kc, vc, torch.tensor([p], device=dev)).view(32, 128)
    ref = _attention_ref(q.view(1, 32, 128), kc[0], vc[0], torch.tensor([p], device=dev))[0]
    assert _rel(y, ref) < TOL


@pytest.mark.parametrize("L,n,start", PREFILL)
def test_prefill_attention_random_shape(dev, L, n, start):
    from moss_tts._runtime import attention

    print(f"prefill attention L={L} n={n} start={start}", flush=True)
    g = torch.Generator(device=dev).manual_seed(L + n + start)
    q = torch.randn((n, 32, 128), device=dev, generator=g).bfloat16()
    kc = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    y = attention.prefill_attention(q, kc, vc, torch.tensor([start], device=dev)).view(n, 32, 128)
    ref = _attention_ref(q, kc[0], vc[0], start + torch.arange(n, device=dev))
    assert _rel(y, ref) < TOL


@pytest.mark.parametrize("k,n,rows", BF16)
def test_bf16_gemv_random_shape(dev, k, n, rows):
    from moss_tts._runtime import bf16

    print(f"bf16 gemv K={k} N={n} rows={rows}", flush=True)
    g = torch.Generator(device=dev).manual_seed(3 * k + n)
    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).bfloat16()
    x = torch.randn((1, k), device=dev, generator=g).bfloat16()
    assert _rel(bf16.gemv(x, w, rows_per_wave=rows), x.float() @ w.float().t()) < TOL


@pytest.mark.parametrize("k,n,residual", BF16_NORM)
def test_bf16_norm_gemv_random_shape(dev, k, n, residual):
    """The fused (add-)RMSNorm + bf16 GEMV equals the norm then the GEMV bit for bit."""
    from moss_tts._runtime import bf16, pointwise

    print(f"bf16 norm gemv K={k} N={n} residual={residual}", flush=True)
    g = torch.Generator(device=dev).manual_seed(5 * k + n)
    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).bfloat16()
    x = (torch.randn((1, k), device=dev, generator=g) * 3).bfloat16()
    nw = (1 + 0.01 * torch.randn(k, device=dev, generator=g)).bfloat16()
    if residual:
        r = torch.randn((1, k), device=dev, generator=g).bfloat16()
        s, y = bf16.norm_gemv(x, nw, 1e-6, w, residual=r)
        s_ref, h = pointwise.add_rmsnorm(x, r, nw, 1e-6)
        assert torch.equal(s, s_ref)
    else:
        y, h = bf16.norm_gemv(x, nw, 1e-6, w), pointwise.rmsnorm(x, nw, 1e-6)
    assert torch.equal(y, bf16.gemv(h, w))
    assert _rel(y, h.float() @ w.float().t()) < TOL


@pytest.mark.parametrize("k,n_half,rows", FP8_GATEUP)
def test_fp8_gateup_random_shape(dev, k, n_half, rows):
    from moss_tts._runtime import fp8

    print(f"fp8 gate||up K={k} N/2={n_half} rows={rows}", flush=True)
    g = torch.Generator(device=dev).manual_seed(k + 7 * n_half)
    wb = torch.randint(0, 256, (2 * n_half, k), device=dev, dtype=torch.uint8, generator=g)
    wb[(wb & 0x7F) == 0x7F] = 0  # no NaN codes
    s = torch.rand((2 * n_half,), device=dev, generator=g) * 0.01 + 0.005
    x = torch.randn((1, k), device=dev, generator=g).bfloat16()
    ref = (x.float() @ fp8.to_bf16(wb).float().t()) * s
    gate, up = ref[:, :n_half].bfloat16().float(), ref[:, n_half:].bfloat16().float()
    want = torch.nn.functional.silu(gate).bfloat16().float() * up
    assert _rel(fp8.fp8_silu_decode(x, wb, s, rows_per_wave=rows), want) < TOL


@pytest.mark.parametrize("k,n,paired,residual,rows", W4A8_NORM)
def test_w4a8_fused_norm_random_shape(dev, k, n, paired, residual, rows):
    """(add+)RMSNorm + quantizer + W4A8 projection in one kernel equals norm_quant followed by the
    projection on its activations, bit for bit."""
    from moss_tts._runtime import w4a8

    print(f"w4a8 fused norm K={k} N={n} paired={paired} residual={residual} rows={rows}", flush=True)
    pw, g = _packed(n, k, 13 * k + n, dev)
    x = (torch.randn((1, k), device=dev, generator=g) * 3).bfloat16()
    r = torch.randn((1, k), device=dev, generator=g).bfloat16() if residual else None
    nw = (1 + 0.1 * torch.randn(k, device=dev, generator=g)).bfloat16()
    summed, _, act = w4a8.norm_quant(x, r, nw, 1e-6, normalized=False)
    want = w4a8.linear(None, pw, paired=paired, prequantized=act, rows_per_wave=rows)
    got = w4a8.norm_linear(x, nw, 1e-6, pw, residual=r, paired=paired, rows_per_wave=rows)
    if residual:
        got_sum, got = got
        assert torch.equal(got_sum, summed)
    assert torch.equal(got.view(-1), want.view(-1))


@pytest.mark.parametrize("m,k,n", GEMM_SILU)
def test_gemm_silu_random_shape(dev, m, k, n):
    """The gate||up GEMM with the SiLU*mul epilogue (fused or through the workspace) equals the GEMM
    followed by silu_mul bit for bit."""
    from moss_tts._runtime import native, pointwise, w4g32

    print(f"gemm_silu M={m} K={k} N={n}", flush=True)
    pw, g = _packed(2 * n, k, 17 * m + k + n, dev)
    x = torch.randn((m, k), device=dev, generator=g).bfloat16()
    assert torch.equal(w4g32.gemm_silu(x, pw), pointwise.silu_mul(w4g32.gemm(x, pw)))


@pytest.mark.parametrize("m,k,n", GEMM_ADDNORM)
def test_gemm_add_rmsnorm_random_shape(dev, m, k, n):
    """The projection followed by the residual add and RMSNorm (the split-K reduction inside the
    norm when the plan splits K) equals gemm then add_rmsnorm bit for bit."""
    from moss_tts._runtime import native, pointwise, w4g32

    split = native.lib().moss_gemm_workspace_bytes(m, k, n) // (m * n * 4)
    print(f"gemm_add_rmsnorm M={m} K={k} N={n} split={split}", flush=True)
    pw, g = _packed(n, k, 19 * m + k + n, dev)
    x = torch.randn((m, k), device=dev, generator=g).bfloat16()
    res = torch.randn((m, n), device=dev, generator=g).bfloat16()
    nw = (1 + 0.05 * torch.randn(n, device=dev, generator=g)).bfloat16()
    want = pointwise.add_rmsnorm(w4g32.gemm(x, pw), res, nw, 1e-6)
    got = w4g32.gemm_add_rmsnorm(x, pw, res, nw, 1e-6)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


@pytest.mark.parametrize("m,k,L", GEMM_QK_ROPE)
def test_gemm_qk_rope_random_shape(dev, m, k, L):
    """The QKV GEMM with the q/k-norm + RoPE + KV write epilogue (fused above 256 tokens, through
    the workspace otherwise) equals the GEMM followed by qk_rope bit for bit, caches included."""
    from moss_tts._runtime import pointwise, w4g32

    print(f"gemm_qk_rope M={m} K={k} L={L}", flush=True)
    g = torch.Generator(device=dev).manual_seed(m + k + L)
    w = w4g32.quantize_minmax(torch.randn((6144, k), device=dev, generator=g) * 0.02)
    x = torch.randn((m, k), device=dev, generator=g).bfloat16()
    qn = (1 + 0.1 * torch.randn(128, device=dev, generator=g)).bfloat16()
    kn = (1 + 0.1 * torch.randn(128, device=dev, generator=g)).bfloat16()
    cos = torch.randn((L, 128), device=dev, generator=g).bfloat16()
    sin = torch.randn((L, 128), device=dev, generator=g).bfloat16()
    pos = torch.randperm(L, device=dev, generator=g)[:m].to(torch.int64)
    k1 = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    v1 = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    k2, v2 = k1.clone(), v1.clone()
    q1 = w4g32.gemm_qk_rope(x, w, qn, kn, cos, sin, k1, v1, pos, 1e-6)
    q2 = pointwise.qk_rope(w4g32.gemm(x, w), qn, kn, cos, sin, k2, v2, pos, 1e-6, cos_by_position=True)
    assert torch.equal(q1.contiguous().view(torch.int16), q2.contiguous().view(torch.int16))
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))
