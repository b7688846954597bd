"""GPU: the prompt pass (prefill) against the oracle.

* ``moss_prefill_attention`` (MFMA causal GQA attention) against the oracle's fp32 causal attention,
  |y - ref| <= 1e-2 + 1e-2 |ref| per output, for prompts of 1..700 tokens starting at row 0 or
  after a cache prefix (both workgroup shapes); every output row covered; NaN in cache rows after
  the prompt never reaches the output.
* The composed prompt pass (``DecodeStepG32.prefill``: embedding sum, 2 full-width layers of INT4
  GEMMs, q/k-norm + RoPE + KV write, causal attention, norms, SiLU*mul, then the final norm and the
  heads on the last token) against ``oracle.decode.prefill`` on the same dequantized weights: the
  last token's logits and every K/V row written within relative L2 2e-2 (the decode step's bar),
  through the captured bucket graphs and eagerly; rows outside the prompt untouched by the eager
  pass.
* Handoff: the decode step that follows the prompt (position n) against the oracle's decode step
  on the oracle's own caches, relative L2 2e-2.
"""
import pytest
import torch

from helpers import _assert_close
from oracle import attention as oa
from oracle import decode as od
from oracle import w4g32 as o

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,start,L", [(1, 0, 64), (5, 0, 64), (32, 0, 128), (33, 7, 128), (100, 0, 256),
                                       (128, 300, 1024), (512, 0, 2048), (200, 1777, 2048), (64, 0, 64),
                                       (513, 0, 576), (700, 60, 1024)])
def test_prefill_attention_parity(dev, n, start, L):
    from moss_tts._runtime import attention

    print(f"prefill attention n={n} start={start} L={L}", flush=True)
    g = torch.Generator().manual_seed(n * 7 + start)
    q = torch.randn((n, 32, 128), generator=g).bfloat16()
    kc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    st = torch.tensor([start], dtype=torch.int64, device=dev)
    out = attention.prefill_attention(q.to(dev), kc.to(dev), vc.to(dev), st)
    torch.cuda.synchronize()
    ref = oa.prefill_attention(q, kc, vc, start).reshape(n, 4096)
    _assert_close(out, ref, f"prefill attention n={n} start={start}")


@pytest.mark.parametrize("n,start,L", [(37, 5, 2048), (1, 0, 128), (100, 1900, 2048), (600, 0, 1024)])
def test_prefill_attention_ignores_rows_after_the_prompt(dev, n, start, L):
    """Cache rows after the last prompt token may never have been written: NaN there must not reach
    the output, although those rows share a key block with the prompt's last keys."""
    from moss_tts._runtime import attention

    print(f"prefill attention, NaN rows after the prompt: n={n} start={start} L={L}", flush=True)
    g = torch.Generator().manual_seed(n + start + L)
    q = torch.randn((n, 32, 128), generator=g).bfloat16()
    kc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    kc[:, :, start + n:] = float("nan")
    vc[:, :, start + n:] = float("nan")
    st = torch.tensor([start], dtype=torch.int64, device=dev)
    out = attention.prefill_attention(q.to(dev), kc.to(dev), vc.to(dev), st)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    ref = oa.prefill_attention(q, kc, vc, start).reshape(n, 4096)
    _assert_close(out, ref, f"prefill attention n={n} start={start}")


def _layers_cpu(eng):
    def deq(m):
        return o.dequantize_rowpack_f32(m.qw.cpu(), m.scales.cpu(), m.zeros.cpu())

    return [dict(qkv=deq(l.qkv.packed), o=deq(l.o.packed), gate_up=deq(l.gate_up.packed), down=deq(l.down.packed),
                 input_norm=l.input_norm.cpu(), post_norm=l.post_norm.cpu(), q_norm=l.q_norm.cpu(),
                 k_norm=l.k_norm.cpu()) for l in eng.layers]


def _rel(a, b):
    a, b = a.float().flatten(), b.float().flatten()
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("n,graphs", [(128, True), (512, True), (100, True), (37, False)])
def test_prefill_step_and_decode_handoff(dev, n, graphs):
    from moss_tts._runtime.decode import DecodeStepG32

    print(f"prefill step n={n} graphs={graphs}", flush=True)
    L = 1024
    eng = DecodeStepG32.random(2, max_length=L, device=dev, seed=21 + n, text_vocab=512)
    if graphs:
        eng.capture_prefill()
    eng.capture()                                  # the decode step's warm-up writes KV row 0
    keys0 = [k.cpu() for k in eng.keys]
    values0 = [v.cpu() for v in eng.values]
    g = torch.Generator().manual_seed(n)
    ids = torch.cat([torch.randint(0, 512, (n, 1), generator=g), torch.randint(0, 1025, (n, 32), generator=g)], 1)
    logits = eng.prefill(ids.view(1, n, 33)).float().cpu()
    torch.cuda.synchronize()
    layers = _layers_cpu(eng)
    heads = o.dequantize_rowpack_f32(eng.heads.packed.qw.cpu(), eng.heads.packed.scales.cpu(),
                                     eng.heads.packed.zeros.cpu())
    keys = [k.clone() for k in keys0]
    values = [v.clone() for v in values0]
    ref = od.prefill(layers, eng.final_norm.cpu(), heads, eng.text_embedding.cpu(), eng.audio_embedding.cpu(),
                     ids, 0, keys, values, eng.cos.cpu(), eng.sin.cpu())
    rel = _rel(logits, ref)
    print(f"prefill logits: relative L2 {rel:.3e}", flush=True)
    assert rel < 2e-2
    bucket = min((b for b in eng.prefill_graphs if b >= n), default=n)
    for i in range(2):
        for got, want, before in ((eng.keys[i].cpu(), keys[i], keys0[i]), (eng.values[i].cpu(), values[i], values0[i])):
            err = _rel(got[:, :, :n], want[:, :, :n])
            assert err < 2e-2, (i, err)
            assert torch.equal(got[:, :, bucket:], before[:, :, bucket:])      # past the prompt (and padding)
    # the decode step that follows the prompt, on the GPU's caches and on the oracle's
    step_ids = torch.tensor([[17] + [i * 29 % 1025 for i in range(32)]], dtype=torch.int64)
    dec = eng.step(step_ids, n).float().cpu()
    ref_dec = od.decode_step(layers, eng.final_norm.cpu(), heads, eng.text_embedding.cpu(),
                             eng.audio_embedding.cpu(), step_ids, n, keys, values, eng.cos.cpu(), eng.sin.cpu())
    rel = _rel(dec, ref_dec)
    print(f"decode after prefill: relative L2 {rel:.3e}", flush=True)
    assert rel < 2e-2


def test_prefill_graph_equals_eager(dev):
    """A prompt that fills its bucket exactly runs the same kernels with the same shapes through the
    graph and eagerly: identical logits and cache rows."""
    from moss_tts._runtime.decode import DecodeStepG32

    eng = DecodeStepG32.random(1, max_length=512, device=dev, seed=5, text_vocab=256)
    g = torch.Generator().manual_seed(1)
    ids = torch.cat([torch.randint(0, 256, (128, 1), generator=g), torch.randint(0, 1025, (128, 32), generator=g)], 1)
    eager = eng.prefill(ids).clone()
    k_e = eng.keys[0][:, :, :128].clone()
    eng.capture_prefill((128,))
    graph = eng.prefill(ids)
    assert torch.equal(graph, eager)
    assert torch.equal(eng.keys[0][:, :, :128], k_e)
    with pytest.raises(ValueError, match="KV capacity"):
        eng.prefill(ids, start=400)


def test_prefill_full_depth(dev):
    """The benchmarked prompt pass at full depth: 36 layers, a 128-token prompt through its bucket
    graph (KV capacity 1024).

    * The graph's logits and K/V rows equal an eager run of the same pass bit for bit.
    * Layer by layer (teacher forcing): each oracle layer (``oracle.decode.prefill_layer``) starts from
      the GPU's own stream state entering that layer (the residual sum and its normalization, whose
      normalization is checked too); the RoPE'd queries, attention, the state after the O projection,
      SiLU*mul, the state after the MLP (normalized with the next layer's input norm) and every K/V
      row written are within relative L2 1e-2 of the GPU's; the last layer's attention, O and MLP,
      which run for the last token alone, against the oracle's last row; then the heads' logits from
      the GPU's final state.
    * End to end: the free-running GPU logits within max(2e-2, 1.5x the oracle's distance to itself
      with every product's K axis summed in reverse) of the free-running oracle, as for the decode
      step; the bar must stay at or below 5e-2."""
    import time

    from moss_tts._runtime.decode import DecodeStepG32
    from oracle import pointwise as op

    n, L, n_layers = 128, 1024, 36
    print(f"prefill full depth: {n_layers} layers, {n} tokens (bucket graph)", flush=True)
    eng = DecodeStepG32.random(n_layers, max_length=L, device=dev, seed=77)
    eng.capture_prefill((n,))
    keys0 = [k.cpu() for k in eng.keys]
    values0 = [v.cpu() for v in eng.values]
    g = torch.Generator().manual_seed(3)
    ids = torch.cat([torch.randint(0, 151643, (n, 1), generator=g), torch.randint(0, 1024, (n, 32), generator=g)], 1)
    logits = eng.prefill(ids).float().cpu()
    assert eng.last_prefill_bucket == n
    kv_graph = [(eng.keys[i][:, :, :n].cpu(), eng.values[i][:, :, :n].cpu()) for i in range(n_layers)]
    trace = []
    with torch.inference_mode():
        eager = eng._prefill_body(*eng._prefill_inputs(ids.to(dev), 0, n), trace=trace)[0].float().cpu()
    torch.cuda.synchronize()
    assert torch.equal(eager, logits), "graph replay differs from the eager pass"
    for i in range(n_layers):
        assert torch.equal(eng.keys[i][:, :, :n].cpu(), kv_graph[i][0])
        assert torch.equal(eng.values[i][:, :, :n].cpu(), kv_graph[i][1])
    print("GPU pass done; oracle layer by layer", flush=True)

    bufs = {}

    def deq(name, m):
        if name not in bufs:
            bufs[name] = torch.empty(m.N * m.K)
        return o.dequantize_rowpack_f32(m.qw.cpu(), m.scales.cpu(), m.zeros.cpu(), out=bufs[name])

    cos, sin, eps = eng.cos.cpu(), eng.sin.cpu(), eng.eps
    caches = {m: ([k.clone() for k in keys0], [v.clone() for v in values0]) for m in ("tf", "free", "rev")}
    x0 = oa.embedding_sum(ids, eng.text_embedding.cpu(), eng.audio_embedding.cpu())
    assert torch.equal(trace[0]["residual_in"].cpu(), x0)
    state = {m: (x0, None) for m in ("free", "rev")}
    worst, t0 = 0.0, time.time()

    def check(key, got, want, i):
        nonlocal worst
        err = _rel(got, want)
        worst = max(worst, err)
        assert err < 1e-2, f"layer {i} {key}: relative L2 {err:.3e}"

    for i, l in enumerate(eng.layers):
        lw = dict(qkv=deq("qkv", l.qkv.packed), o=deq("o", l.o.packed), gate_up=deq("gate_up", l.gate_up.packed),
                  down=deq("down", l.down.packed), input_norm=l.input_norm.cpu(), post_norm=l.post_norm.cpu(),
                  q_norm=l.q_norm.cpu(), k_norm=l.k_norm.cpu())
        t = {k: v.cpu() for k, v in trace[i].items()}
        check("state_in", t["state_in"], op.rmsnorm(t["residual_in"], lw["input_norm"], eps), i)
        ref = od.prefill_layer(lw, i, t["residual_in"], t["state_in"], 0, *caches["tf"], cos, sin, eps)
        check("q", t["q"], ref["q"].reshape(n, -1), i)
        for kv in (0, 1):
            check("K/V rows", kv_graph[i][kv], caches["tf"][kv][i][:, :, :n], i)
        last = i + 1 == n_layers
        rows = slice(n - 1, n) if last else slice(0, n)
        for key in ("attn", "residual_mid", "act") + (("o", "mlp") if last else ("state_mid",)):
            check(key, t[key], ref[key][rows], i)
        if not last:
            res_out, st_out = op.add_rmsnorm(ref["mlp"], ref["residual_mid"], eng.layers[i + 1].input_norm.cpu(), eps)
            check("residual_out", t["residual_out"], res_out, i)
            check("state_out", t["state_out"], st_out, i)
        for mode, lin in (("free", None), ("rev", od.reversed_linear)):
            res, mlp = state[mode]
            if mlp is None:
                st = op.rmsnorm(res, lw["input_norm"], eps)
            else:
                res, st = op.add_rmsnorm(mlp, res, lw["input_norm"], eps)
            out = od.prefill_layer(lw, i, res, st, 0, *caches[mode], cos, sin, eps, lin)
            state[mode] = (out["residual_mid"], out["mlp"])
        if i % 6 == 5:
            print(f"  oracle layer {i + 1}/{n_layers} ({time.time() - t0:.1f} s); worst layer error {worst:.2e}",
                  flush=True)
    heads_w = deq("heads", eng.heads.packed)
    final = eng.final_norm.cpu()

    def head(res, mlp, lin=o.linear):
        _, h = op.add_rmsnorm(mlp[-1:], res[-1:], final, eps)
        return lin(h, heads_w).bfloat16().float().view(-1)

    err = _rel(logits, head(trace[-1]["residual_mid"].cpu(), trace[-1]["mlp"].cpu()))
    print(f"heads from the GPU's final state: relative L2 {err:.3e}", flush=True)
    assert err < 1e-2
    free = head(*state["free"])
    rev = head(*state["rev"], od.reversed_linear)
    e2e, self_dist = _rel(logits, free), _rel(rev, free)
    bar = max(2e-2, 1.5 * self_dist)
    print(f"end to end: GPU vs oracle {e2e:.3e}; oracle vs reversed-order oracle {self_dist:.3e}; bar {bar:.3e}; "
          f"worst layer error {worst:.3e}", flush=True)
    assert e2e < bar and bar <= 5e-2
