"""GPU parity: FP8 E4M3 weight-only linear (GEMV at M=1, MFMA GEMM at M>1) and the fused
gate||up SiLU*mul decode GEMV vs the oracle.

Bars: the e4m3 -> bf16 conversion is bit-exact on all 256 codes; bf16 outputs satisfy
|y - ref| <= 1e-2 + 1e-2 |ref| against the oracle's fp32 row sums times the row scale, and,
since the converted weights and their products with x are exact, they equal RNE of the
oracle's fp32 value except where fp32 summation order moves a value across a rounding
midpoint (checked with the same bound as the INT4 exact mode).
"""
import pytest
import torch

from helpers import _assert_close, _assert_epilogue_close, _assert_rne_or_adjacent
from oracle import fp8 as f

pytestmark = pytest.mark.gpu


def _case(n, k, seed, scaled=True):
    """Scaled: per-row absmax codes spanning +-448 with fp32 row scales.  Unscaled (the
    reference's ``scale=None`` use, ``src/moss_tts/_runtime/llm.py:57-60``): the weights'
    own e4m3 values at their natural N(0, 0.02) magnitude, many of them subnormal."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn((n, k), generator=g) * 0.02
    if scaled:
        return f.quantize_rowwise(w)
    return w.to(torch.float8_e4m3fn).view(torch.uint8), None


def test_conversion_all_codes_bitexact(dev):
    from moss_tts._runtime import fp8

    codes = torch.arange(256, dtype=torch.uint8).repeat(3).view(3, 256)
    out = fp8.to_bf16(codes.to(dev)).cpu()
    ref = codes.view(torch.float8_e4m3fn).to(torch.bfloat16)
    nan_o, nan_r = torch.isnan(out), torch.isnan(ref)
    assert torch.equal(nan_o, nan_r)
    assert torch.equal(out[~nan_o].view(torch.int16), ref[~nan_r].view(torch.int16))


LINEAR = [
    (1, 4096, 4096), (1, 4096, 12288), (64, 4096, 4096), (64, 4096, 12288),
    (1, 64, 8), (1, 4112, 300), (1, 12288, 4096), (3, 128, 40), (17, 1024, 1000), (512, 4096, 4096),
    (256, 4096, 16384), (300, 1024, 32808),   # 128 x 128 tiles, ragged M and N
    # the small-M weight-streaming kernel (M <= 16, K % 4096 == 0, N >= 2048), and just past it
    (2, 4096, 4096), (7, 4096, 4096), (15, 4096, 12288), (16, 12288, 2052), (33, 12288, 4100),
]


@pytest.mark.parametrize("m,k,n", LINEAR)
@pytest.mark.parametrize("scaled", [True, False])
def test_linear_parity(dev, m, k, n, scaled):
    from moss_tts._runtime import fp8

    print(f"fp8 linear M={m} K={k} N={n} scaled={scaled}", flush=True)
    codes, scale = _case(n, k, 10 + m + k + n, scaled)
    x = torch.randn((m, k), generator=torch.Generator().manual_seed(m + k)).bfloat16()
    y = fp8.linear(x.to(dev), codes.to(dev), scale.to(dev) if scaled else None)
    torch.cuda.synchronize()
    ref = f.fp8_linear(x, codes, scale)
    _assert_close(y, ref, f"fp8 M={m} K={k} N={n}")
    w = f.codes_to_float(codes)
    abs_sum = torch.nn.functional.linear(x.float().abs(), w.abs())
    if scaled:
        abs_sum = abs_sum * scale[None, :]
    _assert_rne_or_adjacent(y, ref, abs_sum, k, f"fp8 M={m} K={k} N={n}")


@pytest.mark.parametrize("rows", [1, 2, 4])
def test_linear_rows_per_wave(dev, rows):
    from moss_tts._runtime import fp8

    codes, s = _case(1000, 2048, 77)
    x = torch.randn((1, 2048), generator=torch.Generator().manual_seed(3)).bfloat16()
    y = fp8.linear(x.to(dev), codes.to(dev), s.to(dev), rows_per_wave=rows)
    _assert_close(y, f.fp8_linear(x, codes, s), f"rows={rows}")


@pytest.mark.parametrize("k,n_half", [(4096, 12288), (4096, 4096), (256, 100), (4112, 33)])
@pytest.mark.parametrize("scaled", [True, False])
def test_gateup_silu_parity(dev, k, n_half, scaled):
    from moss_tts._runtime import fp8

    print(f"fp8 gateup K={k} N/2={n_half} scaled={scaled}", flush=True)
    codes, scale = _case(2 * n_half, k, 20 + k + n_half, scaled)
    x = torch.randn((1, k), generator=torch.Generator().manual_seed(k)).bfloat16()
    y = fp8.fp8_silu_decode(x.to(dev), codes.to(dev), scale.to(dev) if scaled else None)
    torch.cuda.synchronize()
    y32 = f.fp8_linear(x, codes, scale)
    _assert_epilogue_close(y, y32[:, :n_half], y32[:, n_half:], f"fp8 gateup K={k} N/2={n_half}")


def test_float8_dtype_and_properties(dev):
    """float8_e4m3fn weights are accepted as such; y(2x) == 2 y(x) and one-hot inputs return the
    scaled weight column exactly (both exact in this arithmetic)."""
    from moss_tts._runtime import fp8

    codes, s = _case(4096, 4096, 5)
    wd = codes.to(dev).view(torch.float8_e4m3fn)
    sd = torch.ones(4096, device=dev)
    x = torch.randn((1, 4096), device=dev).bfloat16()
    y1 = fp8.linear(x, wd, sd)
    y2 = fp8.linear((x.float() * 2).bfloat16(), wd, sd)
    assert torch.equal(y2, (y1.float() * 2).bfloat16())
    col = fp8.to_bf16(wd)
    for c in (0, 15, 16, 1023, 1024, 4095):
        e = torch.zeros((1, 4096), device=dev, dtype=torch.bfloat16)
        e[0, c] = 1.0
        assert torch.equal(fp8.linear(e, wd, sd)[0], col[:, c])
        e64 = torch.zeros((64, 4096), device=dev, dtype=torch.bfloat16)
        e64[:, c] = 1.0
        assert torch.equal(fp8.linear(e64, wd, sd)[5], col[:, c])


def test_rejects_bad_inputs(dev):
    from moss_tts._runtime import fp8

    codes, s = _case(64, 128, 6)
    w = codes.to(dev)
    x = torch.randn((1, 128), device=dev).bfloat16()
    with pytest.raises(ValueError):
        fp8.linear(x.float(), w)                                   # fp32 activations
    with pytest.raises(ValueError):
        fp8.linear(x, w.view(torch.int8))                          # not e4m3 bits
    with pytest.raises(ValueError):
        fp8.linear(x, w, s)                                        # host scale
    with pytest.raises(ValueError):
        fp8.linear(x, w, s.to(dev)[:10])                           # wrong scale length
    with pytest.raises(ValueError):
        fp8.fp8_silu_decode(torch.randn((2, 128), device=dev).bfloat16(), w)   # two rows
    with pytest.raises(ValueError):
        fp8.linear(torch.randn((1, 64), device=dev).bfloat16(), w)             # K mismatch
