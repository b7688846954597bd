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
