"""GPU parity: the W4A8 G32 decode mode vs the oracle (``oracle/w4a8.py``).

Bars:
* quantizer (standalone, after RMSNorm, and fused after gate/up): codes, scales and code
  sums bit-exact against the oracle applied to the same bf16 values;
* integer dot: exact -- a one-hot weight (one nonzero code difference per row) against
  integer activations with unit scales gives y == d * x[k] exactly, which pins the byte
  order, zero points and group bookkeeping;
* outputs: within half a bf16 step plus the fp32 summation bound 8 sqrt(K) 2^-24 sum|terms|
  of the oracle's float64 combine, and equal to RNE(oracle) for all but max(2, 1%) rows
  (the reference's fp32 group order is its Triton reduction's, which no order restates);
  gate/up outputs within 1e-2 + 1e-2 |ref| of the oracle's epilogue.
"""
import numpy as np
import pytest
import torch

from helpers import _assert_epilogue_close, _assert_rne_or_adjacent, _bits
from oracle import pointwise as op
from oracle import w4a8 as a
from oracle import w4g32 as o

pytestmark = pytest.mark.gpu


def _packed(q, z, s, dev):
    from moss_tts._runtime.w4g32 import PackedW4G32

    qw, sc, zp = o.rowpack(q, z, s)
    return PackedW4G32(qw.to(dev), sc.to(dev), zp.to(dev))


def _weights(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    return o.quantize_minmax_g32(torch.randn((n, k), generator=g) * 0.02)


def _row(k, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(k, generator=g) * scale).bfloat16()


def _check_activation(act, ref_values, what):
    q, s = a.quantize_g32(ref_values)
    assert np.array_equal(act.natural().cpu().numpy(), q.reshape(-1)), f"{what}: codes"
    assert np.array_equal(act.scales.cpu().numpy(), s.reshape(-1)), f"{what}: scales"
    assert np.array_equal(act.sums.cpu().numpy(), a.code_sums(q).reshape(-1)), f"{what}: code sums"


@pytest.mark.parametrize("k", [32, 64, 4096, 12288])
def test_quantize_bitexact(dev, k):
    from moss_tts._runtime import w4a8

    print(f"w4a8 quantize K={k}", flush=True)
    x = _row(k, 1)
    if k >= 4096:
        x[:32] = 0                                   # zero group: 1e-8 floor
        x[32:64] = _row(32, 2, 1e-9)                 # clamped scale
        x[64:96] = _row(32, 3, 1e30)                 # huge values
        x[96:128] = torch.tensor([18.0, 9.0] + [0.0] * 30).bfloat16()   # reciprocal rounding case
    act = w4a8.quantize(x.to(dev))
    torch.cuda.synchronize()
    _check_activation(act, x, f"quantize K={k}")


@pytest.mark.parametrize("rows,residual", [(1, False), (1, True), (3, True)])
def test_norm_quant_bitexact(dev, rows, residual):
    from moss_tts._runtime import pointwise, w4a8

    print(f"w4a8 norm_quant rows={rows} residual={residual}", flush=True)
    n = 4096
    x = torch.stack([_row(n, 10 + r) for r in range(rows)]).to(dev)
    r = torch.stack([_row(n, 20 + r) for r in range(rows)]).to(dev) if residual else None
    w = (1 + 0.1 * _row(n, 30)).to(dev)
    summed, y, act = w4a8.norm_quant(x, r, w, 1e-6)
    if residual:
        s_ref, y_ref = pointwise.add_rmsnorm(x, r, w, 1e-6)
        assert torch.equal(_bits(summed), _bits(s_ref))
        o_sum, o_y = op.add_rmsnorm(x.cpu(), r.cpu(), w.cpu(), 1e-6)
        assert torch.equal(_bits(summed), _bits(o_sum))
    else:
        y_ref = pointwise.rmsnorm(x, w, 1e-6)
    assert torch.equal(_bits(y), _bits(y_ref)), "normalized output equals moss_rmsnorm"
    _check_activation(act, y.cpu().flatten(), "norm_quant")
    # without the bf16 output the codes are the same
    _, none, act2 = w4a8.norm_quant(x, r, w, 1e-6, normalized=False)
    assert none is None and torch.equal(act2.qx, act.qx) and torch.equal(act2.scales, act.scales)


@pytest.mark.parametrize("k,n", [(64, 128), (4096, 4096), (12288, 4096)])
def test_integer_dot_is_exact_one_hot(dev, k, n):
    """Row r has code difference d_r at k_r only; x holds integers with a +-127 in each group,
    so sx = 1 and q = x; with unit scales y[r] = d_r * x[k_r] exactly (|y| <= 254)."""
    from moss_tts._runtime import w4a8

    print(f"w4a8 one-hot K={k} N={n}", flush=True)
    g = torch.Generator().manual_seed(40)
    z = torch.randint(2, 14, (n, k // 32), generator=g, dtype=torch.uint8)
    q = z.repeat_interleave(32, dim=1).clone()
    kr = torch.randperm(k, generator=g)[:n] if n <= k else torch.randint(0, k, (n,), generator=g)
    d = torch.randint(1, 3, (n,), generator=g) * (torch.randint(0, 2, (n,), generator=g) * 2 - 1)
    rows = torch.arange(n)
    q[rows, kr] = (q[rows, kr].int() + d.int()).to(torch.uint8)
    s = torch.ones(n, k // 32).bfloat16()
    x = torch.randint(-126, 127, (k,), generator=g).float()
    x[::32] = 127.0
    x = x.bfloat16()
    pw = _packed(q, z, s, dev)
    y = w4a8.linear(x.to(dev), pw)
    torch.cuda.synchronize()
    ref = (d.float() * x.float()[kr] + 0.0).bfloat16()     # an integer zero sum is +0
    bad = (_bits(y) != _bits(ref)).nonzero().flatten()
    assert len(bad) == 0, f"{len(bad)} of {n} rows differ, first {bad[:8].tolist()}"


def _oracle_rows(act, q, z, s):
    """The oracle on the GPU's own (bit-checked) activation codes."""
    qx = act.natural().cpu().numpy()
    sx = act.scales.cpu().numpy()
    y64 = a.w4a8_f64(qx, sx, q, z, s)
    isum = a.group_isums(q, z, qx).astype(np.float64)
    prod = (s.float().numpy() * sx[None, :]).astype(np.float32).astype(np.float64)
    mag = np.abs(isum * prod).sum(-1)
    return y64, mag


@pytest.mark.parametrize("k,n,rows", [(64, 37, 0), (4096, 6144, 0), (4096, 4096, 1), (4096, 4096, 2),
                                      (12288, 4096, 0), (12288, 4096, 4), (2048, 100, 4), (2112, 99, 0),
                                      (6208, 45, 2), (16384, 130, 0)])
def test_gemv_vs_oracle(dev, k, n, rows):
    """One workgroup per R rows, its ceil(K / 2048) waves splitting K (the last slice partial for
    K = 2112 and 6208, the widest K = 16384 with 8 waves)."""
    from moss_tts._runtime import w4a8

    print(f"w4a8 gemv K={k} N={n} rows={rows}", flush=True)
    q, z, s = _weights(n, k, 50 + k % 7)
    x = _row(k, 51)
    pw = _packed(q, z, s, dev)
    act = w4a8.quantize(x.to(dev))
    y = w4a8.linear(None, pw, prequantized=act, rows_per_wave=rows)
    torch.cuda.synchronize()
    _check_activation(act, x, "gemv input")
    y64, mag = _oracle_rows(act, q, z, s)
    _assert_rne_or_adjacent(y, torch.from_numpy(y64.astype(np.float32)), torch.from_numpy(mag), k,
                            f"w4a8 gemv K={k} N={n}")
    # quantize-inside form (one kernel) gives the same bits
    assert torch.equal(_bits(w4a8.linear(x.to(dev), pw, rows_per_wave=rows)), _bits(y))
    # and so does every row count per workgroup: the combine order does not depend on it
    for r in (1, 2, 4):
        assert torch.equal(_bits(w4a8.linear(None, pw, prequantized=act, rows_per_wave=r)), _bits(y)), r


@pytest.mark.parametrize("k,n_half,fused", [(4096, 12288, True), (4096, 12288, False), (2048, 64, True),
                                            (64, 33, False), (12288, 96, True)])
def test_gateup_vs_oracle(dev, k, n_half, fused):
    from moss_tts._runtime import w4a8

    print(f"w4a8 gateup K={k} N_half={n_half} fused={fused}", flush=True)
    q, z, s = _weights(2 * n_half, k, 60)
    x = _row(k, 61)
    pw = _packed(q, z, s, dev)
    act = w4a8.quantize(x.to(dev))
    res = w4a8.linear(None, pw, paired=True, fused=fused, prequantized=act)
    y, out_act = res if fused else (res, None)
    torch.cuda.synchronize()
    y64, _ = _oracle_rows(act, q, z, s)
    gate = torch.from_numpy(y64[:n_half].astype(np.float32))[None]
    up = torch.from_numpy(y64[n_half:].astype(np.float32))[None]
    _assert_epilogue_close(y[None], gate, up, f"w4a8 gateup K={k} N={n_half}")
    if fused:
        _check_activation(out_act, y.cpu(), "fused output quantizer")
        plain = w4a8.linear(None, pw, paired=True, prequantized=act)
        assert torch.equal(_bits(plain), _bits(y))


@pytest.mark.parametrize("k,n,paired,residual,rows", [(4096, 6144, False, False, 0), (4096, 6144, False, True, 2),
                                                       (4096, 12288, True, True, 0), (4096, 100, True, False, 4),
                                                       (2048, 300, False, True, 1), (8192, 256, True, True, 0)])
def test_fused_norm_projection_equals_norm_quant_then_linear(dev, k, n, paired, residual, rows):
    """The (add+)RMSNorm + quantizer inside the W4A8 projection gives the bits of norm_quant
    followed by the projection on its activations (which are pinned against the oracle)."""
    from moss_tts._runtime import w4a8

    print(f"w4a8 fused norm K={k} N={n} paired={paired} residual={residual} rows={rows}", flush=True)
    pw = _packed(*_weights(2 * n if paired else n, k, 90 + k % 5), dev)
    x, r = (_row(k, 91) * 3).to(dev), _row(k, 92).to(dev)
    w = (1 + 0.1 * _row(k, 93)).to(dev)
    summed, _, act = w4a8.norm_quant(x, r if residual else None, w, 1e-6, normalized=False)
    want = w4a8.linear(None, pw, paired=paired, prequantized=act, rows_per_wave=rows)
    got = w4a8.norm_linear(x, w, 1e-6, pw, residual=r if residual else None, paired=paired, rows_per_wave=rows)
    if residual:
        got_sum, got = got
        assert torch.equal(_bits(got_sum), _bits(summed))
    assert torch.equal(_bits(got), _bits(want))


def test_w4a8_mlp_chain_matches_oracle_chain(dev):
    """norm_quant -> fused gate/up -> down, with every activation bit-checked against the
    oracle quantizer on the previous bf16 output."""
    from moss_tts._runtime import w4a8

    print("w4a8 mlp chain", flush=True)
    h, inter = 4096, 12288
    gu = _packed(*_weights(2 * inter, h, 70), dev)
    dq, dz, ds = _weights(h, inter, 71)
    down = _packed(dq, dz, ds, dev)
    x, r = _row(h, 72).to(dev), _row(h, 73).to(dev)
    w = (1 + 0.1 * _row(h, 74)).to(dev)
    summed, y, act = w4a8.norm_quant(x, r, w, 1e-6)
    mid, mid_act = w4a8.linear(None, gu, paired=True, fused=True, prequantized=act)
    out = w4a8.linear(None, down, prequantized=mid_act)
    # the down projection quantizing its bf16 input inside its own kernel: the same bits
    assert torch.equal(_bits(w4a8.linear(mid, down)), _bits(out))
    torch.cuda.synchronize()
    _check_activation(act, y.cpu(), "norm")
    _check_activation(mid_act, mid.cpu(), "gate/up output")
    y64, mag = _oracle_rows(mid_act, dq, dz, ds)
    _assert_rne_or_adjacent(out, torch.from_numpy(y64.astype(np.float32)), torch.from_numpy(mag), inter, "down")


def test_argument_errors(dev):
    from moss_tts._runtime import w4a8

    pw = _packed(*_weights(64, 128, 80), dev)
    x = _row(128, 81).to(dev)
    with pytest.raises(ValueError):
        w4a8.linear(x, pw, fused=True)                       # fused needs paired
    with pytest.raises(ValueError):
        w4a8.linear(x, pw, paired=True, fused=True, rows_per_wave=1)
    with pytest.raises(ValueError):
        w4a8.linear(x[:64], pw)                              # wrong K
    with pytest.raises(ValueError):
        w4a8.linear(None, pw, prequantized=w4a8.quantize(_row(64, 82).to(dev)))
    with pytest.raises(ValueError):
        w4a8.quantize(x.float())
