"""Pins the FP8 E4M3 oracle (``oracle/fp8.py``) on the CPU.

* ``decode_e4m3`` (bit fields) agrees with torch's ``float8_e4m3fn`` on all 256 codes, and
  with closed forms from the OCP definition.
* ``quantize_rowwise`` lands every weight within half an e4m3 step of ``w / s`` and maps the
  row maximum to +-448 exactly.
* ``fp8_linear`` equals a float64 restatement (explicit loops on a tiny case) and is linear
  in the scale; ``fp8_gateup_silu`` splits gate/up rows the way the reference does.
"""
import math

import numpy as np
import torch

from oracle import fp8 as f


def test_decode_matches_torch_on_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    mine = f.decode_e4m3(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan_m, nan_r = np.isnan(mine), np.isnan(ref)
    assert np.array_equal(nan_m, nan_r)
    assert np.array_equal(np.where(nan_m, 0, mine), np.where(nan_r, 0, ref))
    assert sorted(np.flatnonzero(nan_m).tolist()) == [0x7F, 0xFF]


def test_decode_closed_forms():
    d = dict(zip(range(256), f.decode_e4m3(np.arange(256, dtype=np.uint8)).tolist()))
    assert d[0x38] == 1.0
    assert d[0x7E] == 448.0 and d[0xFE] == -448.0
    assert d[0x01] == 2.0 ** -9
    assert d[0x08] == 2.0 ** -6
    assert d[0x07] == 7 * 2.0 ** -9          # largest subnormal
    assert d[0x00] == 0.0 and math.copysign(1.0, d[0x80]) == -1.0
    assert d[0x40] == 2.0 and d[0x3C] == 1.5


def test_every_e4m3_value_is_a_bf16_value():
    """The kernels convert e4m3 -> bf16 with no rounding; that needs every finite e4m3 value
    to have at most 8 significant bits and an exponent inside bf16's range."""
    v = torch.from_numpy(f.decode_e4m3(np.arange(256, dtype=np.uint8)))
    fin = ~torch.isnan(v)
    assert torch.equal(v[fin].bfloat16().float(), v[fin])


def test_quantize_rowwise_error_and_range():
    g = torch.Generator().manual_seed(0)
    w = torch.randn((64, 512), generator=g) * 0.02
    w[3] = 0.0
    codes, s = f.quantize_rowwise(w)
    assert codes.dtype == torch.uint8 and s.dtype == torch.float32
    assert s[3] == 1.0 and torch.count_nonzero(codes[3]) == 0
    v = f.codes_to_float(codes)
    t = w / s[:, None]
    # half a step: 2^(e-4) for normals (3 mantissa bits), 2^-10 in the subnormal range
    e = torch.floor(torch.log2(t.abs().clamp_min(2.0 ** -6)))
    assert torch.all((v - t).abs() <= 2.0 ** (e - 4) + 1e-7)
    row_max = v.abs().amax(dim=1)
    assert torch.all(row_max[torch.arange(64) != 3] == 448.0)


def test_fp8_linear_matches_float64_loops():
    g = torch.Generator().manual_seed(1)
    codes = torch.randint(0, 256, (5, 48), generator=g, dtype=torch.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38       # no NaN codes
    x = torch.randn((3, 48), generator=g).bfloat16()
    s = torch.rand(5, generator=g) + 0.5
    y = f.fp8_linear(x, codes, s)
    wv = f.decode_e4m3(codes.numpy()).astype(np.float64)
    xv = x.float().numpy().astype(np.float64)
    for m in range(3):
        for n in range(5):
            ref = sum(wv[n, k] * xv[m, k] for k in range(48)) * float(s[n])
            assert abs(float(y[m, n]) - ref) <= 1e-5 * (1 + abs(ref))
    assert torch.allclose(f.fp8_linear(x, codes, None) * s[None, :], y, rtol=1e-6, atol=1e-6)


def test_fp8_gateup_rows():
    g = torch.Generator().manual_seed(2)
    codes, s = f.quantize_rowwise(torch.randn((8, 64), generator=g) * 0.02)
    x = torch.randn((1, 64), generator=g).bfloat16()
    y = f.fp8_linear(x, codes, s)
    out = f.fp8_gateup_silu(x, codes, s)
    gate, up = y[0, :4].bfloat16().float(), y[0, 4:].bfloat16().float()
    act = (gate * torch.sigmoid(gate)).bfloat16().float()
    assert torch.allclose(out[0].float(), (act * up).bfloat16().float(), atol=1e-6, rtol=1e-2)
