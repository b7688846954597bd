"""GPU parity: RMSNorm / add-RMSNorm, q/k-norm + RoPE + KV write, SiLU*mul vs the oracle.

Bars: exact where the operation is a single correctly rounded step (the bf16 residual add,
the V copy, KV row placement); elsewhere the 1e-2 atol + 1e-2 rtol bar, plus >= 99% of
outputs bit-identical (rsqrt/exp and fp32 summation order may move a value across a bf16
rounding midpoint).
"""
import pytest
import torch

from oracle import pointwise as p

pytestmark = pytest.mark.gpu


def _close(got, ref, what, exact_frac=0.99):
    got = got.cpu()
    ref = ref.cpu()
    gf, rf = got.float(), ref.float()
    bad = (gf - rf).abs() > 1e-2 + 1e-2 * rf.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} outside tolerance, max err {float((gf - rf).abs().max())}"
    same = (got.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
    assert same >= exact_frac, f"{what}: only {same:.4f} bit-identical"


@pytest.mark.parametrize("rows,n", [(1, 4096), (3, 4096), (512, 4096), (2, 1024), (1, 8192), (5, 8)])
def test_rmsnorm(dev, rows, n):
    from moss_tts._runtime import pointwise

    print(f"rmsnorm rows={rows} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + n)
    x = (torch.randn((rows, n), generator=g) * 2).bfloat16()
    w = (1 + torch.randn(n, generator=g) * 0.01).bfloat16()
    y = pointwise.rmsnorm(x.to(dev), w.to(dev), 1e-6)
    _close(y, p.rmsnorm(x, w, 1e-6), f"rmsnorm {rows}x{n}")


@pytest.mark.parametrize("rows,n", [(1, 4096), (512, 4096)])
def test_add_rmsnorm(dev, rows, n):
    from moss_tts._runtime import pointwise

    print(f"add_rmsnorm rows={rows} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows + n)
    x = torch.randn((rows, n), generator=g).bfloat16()
    r = (torch.randn((rows, n), generator=g) * 8).bfloat16()
    w = (1 + torch.randn(n, generator=g) * 0.01).bfloat16()
    s, y = pointwise.add_rmsnorm(x.to(dev), r.to(dev), w.to(dev), 1e-6)
    s_ref, y_ref = p.add_rmsnorm(x, r, w, 1e-6)
    assert torch.equal(s.cpu().view(torch.int16), s_ref.view(torch.int16))
    _close(y, y_ref, f"add_rmsnorm {rows}x{n}")


@pytest.mark.parametrize("ntok,L,start", [(1, 2048, 2047), (1, 1024, 0), (7, 64, 20), (512, 1024, 0)])
def test_qk_norm_rope_kv(dev, ntok, L, start):
    from moss_tts._runtime import pointwise

    print(f"qk_rope ntok={ntok} L={L} start={start}", flush=True)
    g = torch.Generator().manual_seed(ntok + L)
    qkv = (torch.randn((ntok, 6144), generator=g) * 2).bfloat16()
    qw = (1 + torch.randn(128, generator=g) * 0.05).bfloat16()
    kw = (1 + torch.randn(128, generator=g) * 0.05).bfloat16()
    pos = torch.arange(start, start + ntok)
    cos, sin = p.rope_tables(pos)
    kc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    q = pointwise.qk_rope(qkv.to(dev), qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), kc_d, vc_d,
                          pos.to(dev), 1e-6)
    q_ref = p.qk_norm_rope_kv(qkv, qw, kw, cos, sin, kc, vc, pos, 1e-6)
    assert q.shape == (1, 32, ntok, 128)
    _close(q[0].transpose(0, 1), q_ref, "q")
    sl = slice(start, start + ntok)
    _close(kc_d[:, :, sl], kc[:, :, sl], "k cache rows")
    assert torch.equal(vc_d.cpu().view(torch.int16), vc.view(torch.int16))          # V copy + untouched rows
    untouched = torch.ones(L, dtype=torch.bool)
    untouched[sl] = False
    assert torch.equal(kc_d.cpu()[:, :, untouched].view(torch.int16), kc[:, :, untouched].view(torch.int16))


@pytest.mark.parametrize("rows,n", [(1, 12288), (512, 12288), (3, 4)])
def test_silu_mul(dev, rows, n):
    from moss_tts._runtime import pointwise

    print(f"silu_mul rows={rows} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows + n)
    x = (torch.randn((rows, 2 * n), generator=g) * 3).bfloat16()
    _close(pointwise.silu_mul(x.to(dev)), p.silu_mul(x), f"silu_mul {rows}x{n}")


@pytest.mark.parametrize("L,position", [(2048, 2047), (2048, 0), (2048, 1000), (1024, 63), (1024, 64), (128, 127),
                                        (2560, 2500), (4096, 4095), (32768, 20000)])
def test_decode_attention(dev, L, position):
    """Split-softmax GQA decode attention vs the oracle's exact fp32 softmax; bf16 output."""
    from moss_tts._runtime import attention
    from oracle import attention as oa

    print(f"decode_attention L={L} p={position}", flush=True)
    g = torch.Generator().manual_seed(L + position)
    q = torch.randn((32, 128), generator=g).bfloat16()
    kc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    pos = torch.tensor([position], dtype=torch.int64)
    ws = attention.workspace(L, dev)
    out = attention.decode_attention(q.to(dev), kc.to(dev), vc.to(dev), pos.to(dev), ws=ws)
    ref = oa.decode_attention(q, kc, vc, position).reshape(1, 1, 4096)
    _close(out, ref.bfloat16(), f"attention L={L} p={position}", exact_frac=0.95)
    # a second call on the same workspace reproduces the first bit for bit
    again = attention.decode_attention(q.to(dev), kc.to(dev), vc.to(dev), pos.to(dev), ws=ws)
    assert torch.equal(out, again)


def test_decode_attention_workspace_across_positions(dev):
    """One workspace through positions with different numbers of active splits: every call
    matches the oracle and a call on a fresh workspace."""
    from moss_tts._runtime import attention
    from oracle import attention as oa

    L = 2048
    g = torch.Generator().manual_seed(77)
    q = torch.randn((32, 128), generator=g).bfloat16()
    kc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    ws = attention.workspace(L, dev)
    for position in (2047, 5, 63, 64, 1000, 0, 2047, 130):
        print(f"attention workspace reuse p={position}", flush=True)
        pos = torch.tensor([position], dtype=torch.int64, device=dev)
        out = attention.decode_attention(qd, kd, vd, pos, ws=ws)
        fresh = attention.decode_attention(qd, kd, vd, pos, ws=attention.workspace(L, dev))
        assert torch.equal(out, fresh), position
        ref = oa.decode_attention(q, kc, vc, position).reshape(1, 1, 4096)
        _close(out, ref.bfloat16(), f"attention reuse p={position}", exact_frac=0.95)


def test_decode_attention_rejects_unaligned_length(dev):
    from moss_tts._runtime import attention

    q = torch.zeros((32, 128), device=dev, dtype=torch.bfloat16)
    kc = torch.zeros((1, 8, 96, 128), device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        attention.decode_attention(q, kc, kc.clone(), torch.zeros(1, device=dev, dtype=torch.int64))


@pytest.mark.parametrize("L,position", [(2048, 2047), (2048, 0), (2048, 1000), (1024, 63), (1024, 64), (128, 5),
                                        (4096, 3000)])
def test_fused_qkv_attention_equals_rope_then_attention(dev, L, position):
    """q/k-norm + RoPE + KV write fused into the attention kernel reproduces moss_qk_norm_rope_kv
    followed by moss_decode_attention bit for bit, output and both caches."""
    from moss_tts._runtime import attention, pointwise

    print(f"fused qkv attention L={L} p={position}", flush=True)
    g = torch.Generator(device=dev).manual_seed(L + position)
    qkv = (torch.randn((1, 6144), device=dev, generator=g) * 2).bfloat16()
    qn = (1 + 0.05 * torch.randn(128, device=dev, generator=g)).bfloat16()
    kn = (1 + 0.05 * torch.randn(128, device=dev, generator=g)).bfloat16()
    cos, sin = p.rope_tables(torch.arange(L))
    cos, sin = cos.to(dev), sin.to(dev)
    kc = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), device=dev, generator=g).bfloat16()
    pos = torch.tensor([position], device=dev)
    k1, v1, k2, v2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    q = pointwise.qk_rope(qkv, qn, kn, cos, sin, k1, v1, pos, 1e-6, cos_by_position=True)
    ref = attention.decode_attention(q, k1, v1, pos)
    out = attention.decode_attention_qkv(qkv, qn, kn, cos, sin, k2, v2, pos, 1e-6)
    assert torch.equal(out, ref)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    # the merge with the int8 quantizer: the same bf16 output, and the activation the standalone
    # quantizer (bit-exact against the oracle) forms from it
    from moss_tts._runtime import w4a8

    k3, v3 = kc.clone(), vc.clone()
    out_q, act = attention.decode_attention_qkv(qkv, qn, kn, cos, sin, k3, v3, pos, 1e-6, quantize=True)
    assert torch.equal(out_q, ref) and torch.equal(k3, k1) and torch.equal(v3, v1)
    want = w4a8.quantize(ref.view(-1))
    assert torch.equal(act.qx, want.qx) and torch.equal(act.scales, want.scales) and torch.equal(act.sums, want.sums)


def test_decode_attention_ignores_rows_after_position(dev):
    from moss_tts._runtime import attention

    g = torch.Generator().manual_seed(5)
    q = torch.randn((32, 128), generator=g).bfloat16().to(dev)
    kc = torch.randn((1, 8, 256, 128), generator=g).bfloat16().to(dev)
    vc = torch.randn((1, 8, 256, 128), generator=g).bfloat16().to(dev)
    pos = torch.tensor([100], dtype=torch.int64, device=dev)
    a = attention.decode_attention(q, kc, vc, pos)
    kc[:, :, 101:] = 1e4
    vc[:, :, 101:] = float("nan")
    b = attention.decode_attention(q, kc, vc, pos)
    assert torch.equal(a, b)


def test_embedding_sum(dev):
    from moss_tts._runtime import attention
    from oracle import attention as oa

    g = torch.Generator().manual_seed(3)
    text = torch.randn((300, 4096), generator=g).bfloat16()
    audio = torch.randn((32, 1025, 4096), generator=g).bfloat16()
    ids = torch.cat([torch.tensor([[17]]), torch.randint(0, 1025, (1, 32), generator=g)], 1)
    out = attention.embedding_sum(ids.to(dev), text.to(dev), audio.to(dev))
    ref = oa.embedding_sum(ids[0], text, audio)
    assert torch.equal(out.cpu()[0].view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("T,H,Q", [(37, 4096, 32), (5, 4098, 32), (3, 1000, 40), (2, 8, 2), (4, 12, 1), (3, 1004, 33)])
def test_embedding_sum_rows(dev, T, H, Q):
    """Several tokens at once, bit-exact: 16-, 8- and 2-byte loads (H % 8, H % 4, other H), Q beyond
    one batch of 32 codebooks, a single codebook."""
    from moss_tts._runtime import attention
    from oracle import attention as oa

    print(f"embedding sum T={T} H={H} Q={Q}", flush=True)
    g = torch.Generator().manual_seed(T + H + Q)
    text = torch.randn((50, H), generator=g).bfloat16()
    audio = torch.randn((Q, 70, H), generator=g).bfloat16()
    ids = torch.cat([torch.randint(0, 50, (T, 1), generator=g), torch.randint(0, 70, (T, Q), generator=g)], 1)
    out = attention.embedding_sum(ids.to(dev), text.to(dev), audio.to(dev)).cpu()
    for t in range(T):
        ref = oa.embedding_sum(ids[t], text, audio)
        assert torch.equal(out[t].view(torch.int16), ref.view(torch.int16)), t
