"""GPU parity: the bf16-weight decode GEMV (the output heads) against fp32 ``F.linear`` on the CPU.

Bars: |y - ref| <= 1e-2 + 1e-2 |ref| against ``F.linear(x.float(), w.float())``; since the products
are exact in fp32, outputs equal RNE(ref) except where the fp32 summation order moves a value across
a rounding midpoint (``_assert_rne_or_adjacent``).  The fused-norm form equals ``moss_rmsnorm`` then
the GEMV bit for bit; one-hot inputs select a weight column exactly."""
import pytest
import torch

from helpers import _assert_close, _assert_rne_or_adjacent
from oracle import pointwise as op
from oracle import w4g32 as o

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("k,n,rows", [(4096, 32770, 0), (4096, 32770, 1), (4096, 32770, 4), (512, 7, 0),
                                      (1536, 1000, 2), (8192, 300, 0), (6144, 64, 4), (2048, 2, 0)])
def test_bf16_gemv_parity(dev, k, n, rows):
    from moss_tts._runtime import bf16

    print(f"bf16 gemv K={k} N={n} rows={rows}", flush=True)
    g = torch.Generator().manual_seed(k + n + rows)
    w = (torch.randn((n, k), generator=g) * 0.02).bfloat16()
    x = torch.randn((1, k), generator=g).bfloat16()
    y = bf16.gemv(x.to(dev), w.to(dev), rows_per_wave=rows)
    torch.cuda.synchronize()
    ref = o.linear(x, w)
    _assert_close(y, ref, f"bf16 gemv K={k} N={n}")
    _assert_rne_or_adjacent(y, ref, o.linear(x.float().abs(), w.float().abs()), k, f"bf16 gemv K={k} N={n}")


@pytest.mark.parametrize("residual", [False, True])
@pytest.mark.parametrize("k,n", [(4096, 32770), (2048, 100), (8192, 40)])
def test_bf16_norm_gemv(dev, k, n, residual):
    """The decode step's final add-RMSNorm + bf16 heads: bit-identical to the norm then the GEMV, and
    within the GEMV bar of the oracle's add-RMSNorm + F.linear."""
    from moss_tts._runtime import bf16, pointwise

    print(f"bf16 norm gemv K={k} N={n} residual={residual}", flush=True)
    g = torch.Generator().manual_seed(k * 3 + n)
    w = (torch.randn((n, k), generator=g) * 0.02).bfloat16().to(dev)
    x = (torch.randn((1, k), generator=g) * 3).bfloat16().to(dev)
    nw = (1 + 0.01 * torch.randn(k, generator=g)).bfloat16().to(dev)
    r = (torch.randn((1, k), generator=g) * 5).bfloat16().to(dev) if residual else None
    out = bf16.norm_gemv(x, nw, 1e-6, w, residual=r)
    if residual:
        s, y = out
        s_ref, h = pointwise.add_rmsnorm(x, r, nw, 1e-6)
        assert torch.equal(s, s_ref)
        _, h_cpu = op.add_rmsnorm(x.cpu(), r.cpu(), nw.cpu(), 1e-6)
    else:
        y, h = out, pointwise.rmsnorm(x, nw, 1e-6)
        h_cpu = op.rmsnorm(x.cpu(), nw.cpu(), 1e-6)
    assert torch.equal(y, bf16.gemv(h, w))
    _assert_close(y, o.linear(h_cpu, w.cpu()), f"bf16 norm gemv K={k} N={n}")


def test_bf16_gemv_one_hot_columns(dev):
    from moss_tts._runtime import bf16

    w = (torch.randn((32770, 4096), device=dev) * 0.02).bfloat16()
    for col in (0, 7, 8, 511, 512, 4095):
        e = torch.zeros((1, 4096), device=dev, dtype=torch.bfloat16)
        e[0, col] = 1.0
        assert torch.equal(bf16.gemv(e, w)[0], w[:, col]), f"column {col}"


def test_bf16_gemv_rejects_bad_inputs(dev):
    from moss_tts._runtime import bf16

    w = torch.zeros((8, 4096), device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        bf16.gemv(torch.zeros((1, 4096), device=dev), w)                                   # fp32 x
    with pytest.raises(ValueError):
        bf16.gemv(torch.zeros((1, 4608), device=dev, dtype=torch.bfloat16),
                  torch.zeros((8, 4608), device=dev, dtype=torch.bfloat16))               # K / 512 = 9
    with pytest.raises(ValueError):
        bf16.gemv(torch.zeros((2, 4096), device=dev, dtype=torch.bfloat16), w)             # two rows
