"""GPU: the drop-in boundary end to end.  A one-layer, full-width MOSS-TTS-shaped model is
built from transformers' own Qwen3 modules, its weights are exported in the reference's
calibrated format, and ``MossTTS.from_pretrained(preset="gptq", model=...)`` installs the
export (module swap) and captures the decode step.

Bars: installed weights equal the reference's dequant of the export bit for bit; the model's
own (rebound) MLP forward at M=1 (GEMV) and M=64 (GEMM) meets 1e-2 atol + 1e-2 rtol against
dequant-then-matmul; the captured decode step's logits are within 2e-2 relative L2 of the
oracle's composed step (the same bound as the synthetic decode test), whose heads are the model's
own bf16 head rows."""
import pytest
import torch

from helpers import _assert_close, export_model, model_layer_cpu, moss_model
from oracle import decode as od
from oracle import w4g32 as o

pytestmark = pytest.mark.gpu


def test_from_pretrained_install_and_decode(dev, tmp_path):
    from moss_tts import MossTTS
    from moss_tts._runtime import w4g32
    from moss_tts._runtime.modules import Bf16Linear, QuantGateUpG32, QuantLinearG32
    from moss_tts._runtime.presets import install_gptq

    print("boundary: building the one-layer model", flush=True)
    model = moss_model(dev)
    deq = export_model(model, tmp_path)
    print("boundary: from_pretrained", flush=True)
    tts = MossTTS.from_pretrained(preset="gptq", calibration_path=tmp_path, device="cuda:0", model=model)
    layer = model.language_model.layers[0]
    a, m = layer.self_attn, layer.mlp
    assert isinstance(a.qkv_proj, QuantLinearG32) and isinstance(m.gate_up_proj, QuantGateUpG32)
    assert a.q_proj.qw.data_ptr() == a.qkv_proj.qw.data_ptr()             # row views, no copies
    assert m.up_proj.qw.data_ptr() == m.gate_up_proj.qw[12288:].data_ptr()

    for name, mod in (("qkv", a.qkv_proj), ("out", a.o_proj), ("up", m.gate_up_proj), ("down", m.down_proj)):
        got = w4g32.dequantize(mod.packed).cpu()
        assert torch.equal(got.view(torch.int16), deq[name].view(torch.int16)), name

    print("boundary: rebound MLP forward, M=1 and M=64", flush=True)
    for rows in (1, 64):
        x = torch.randn((1, rows, 4096), generator=torch.Generator().manual_seed(rows)).bfloat16()
        y = m(x.to(dev))
        gu = o.linear(x.view(rows, 4096), deq["up"])
        act = o.silu_mul_rounded(gu[:, :12288], gu[:, 12288:])
        ref = o.linear(act, deq["down"])
        _assert_close(y.view(rows, 4096), ref, f"mlp M={rows}")
    q = a.q_proj(x.to(dev))                                                   # a row view on the GEMM path
    _assert_close(q.view(64, 4096), o.linear(x.view(64, 4096), deq["qkv"][:4096]), "q_proj view")

    print("boundary: captured decode step vs oracle", flush=True)
    eng = tts.engine.decode
    assert eng.graph is not None
    keys0 = [k.cpu().clone() for k in eng.keys]
    values0 = [v.cpu().clone() for v in eng.values]
    ids = torch.tensor([[17] + [i * 29 % 1025 for i in range(32)]], dtype=torch.int64)
    position = 5
    logits = tts.step(ids, position).float().cpu()
    # the heads stay bf16, as the reference keeps them (llm.py:188-191): audio rows [:1024] of the
    # 32 codebook heads, then the gen-slot / delay-slot rows of the text head
    heads = torch.cat([h.weight[:1024] for h in model.lm_heads[1:]] +
                      [model.lm_heads[0].weight[[100, 101]]]).detach().cpu()
    assert isinstance(eng.heads, Bf16Linear) and torch.equal(eng.heads.weight.cpu(), heads)
    L0 = model_layer_cpu(model, deq)
    ref = od.decode_step([L0], model.language_model.norm.weight.detach().cpu(), heads,
                         eng.text_embedding.detach().cpu(), eng.audio_embedding.detach().cpu(), ids, position,
                         keys0, values0, eng.cos.cpu(), eng.sin.cpu()).float()
    rel = float((logits - ref).norm() / ref.norm())
    print(f"boundary decode: relative L2 {rel:.3e}", flush=True)
    assert logits.shape == (32 * 1024 + 2,) and rel < 2e-2
    # the reference's step contract: sampled next ids, here greedy-free (temperature sampling)
    nxt = tts.next_ids(ids, position, 32, -1)
    assert nxt.shape == (1, 1, 33) and int(nxt[0, 0, 0]) in (100, 101)
    assert bool(((nxt[0, 0, 1:] >= 0) & (nxt[0, 0, 1:] < 1024)).all())
    nxt = tts.next_ids(ids, position, 32, 32)                                   # delay 32: audio end token
    assert int(nxt[0, 0, 0]) == 102 and bool((nxt[0, 0, 1:] == 1024).all())
    # the 32 steps after the audio start in one graph
    with pytest.raises(RuntimeError, match="Warm"):
        tts.first_audio(nxt, position)
    assert tts.engine.enable_first_audio_graph() == {"codebooks": 32, "steps": 32}
    with pytest.raises(RuntimeError, match="once"):
        tts.engine.enable_first_audio_graph()
    start = torch.full((1, 1, 33), 1024, dtype=torch.int64, device=dev)
    start[0, 0, 0] = eng.audio_start_id
    history, status = tts.first_audio(start, position)
    history, status = history.cpu(), status.cpu()
    assert history.shape == (32, 33) and set(history[:, 0].tolist()) <= {100, 101}
    assert int(status[1]) == 33 and int(status[3]) == position + 32
    assert bool((history[0, 2:] == 1024).all())                                # audio length 1: channel 0 only

    with pytest.raises(RuntimeError, match="before graph capture"):
        install_gptq(tts.engine, tmp_path)
    tts.close()
    with pytest.raises(RuntimeError, match="closed"):
        tts.step(ids, position)
