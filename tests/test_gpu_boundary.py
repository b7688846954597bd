"""GPU: the drop-in boundary end to end.  A one-layer, full-width MOSS-TTS-shaped model is
built from transformers' own Qwen3 modules, its weights are exported in the reference's
calibrated format, and ``MossTTS.from_pretrained(preset="gptq", model=...)`` installs the
export (module swap) and captures the decode step.

Bars: installed weights equal the reference's dequant of the export bit for bit; the model's
own (rebound) MLP forward at M=1 (GEMV) and M=64 (GEMM) meets 1e-2 atol + 1e-2 rtol against
dequant-then-matmul; the captured decode step's logits are within 2e-2 relative L2 of the
oracle's composed step (the same bound as the synthetic decode test), whose heads are the model's
own bf16 head rows."""
import os
from types import SimpleNamespace

import pytest
import torch

from helpers import _assert_close, write_export
from oracle import decode as od
from oracle import w4g32 as o

pytestmark = pytest.mark.gpu


def _model(dev, seed=0):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model

    cfg = Qwen3Config(hidden_size=4096, intermediate_size=12288, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, num_hidden_layers=1, vocab_size=512, rms_norm_eps=1e-6, rope_theta=1e6)
    torch.manual_seed(seed)
    with torch.device(dev):
        lm = Qwen3Model(cfg).bfloat16()
        for p in lm.parameters():
            torch.nn.init.normal_(p, 0.0, 0.02)
        for norm in (lm.norm, lm.layers[0].input_layernorm, lm.layers[0].post_attention_layernorm,
                     lm.layers[0].self_attn.q_norm, lm.layers[0].self_attn.k_norm):
            norm.weight.data = (1 + 0.01 * torch.randn_like(norm.weight.float())).bfloat16()
        lm.embed_tokens.weight.data.normal_(0, 1)
        model = torch.nn.Module()
        model.language_model = lm
        model.emb_ext = torch.nn.ModuleList(torch.nn.Embedding(1025, 4096).bfloat16() for _ in range(32))
        model.lm_heads = torch.nn.ModuleList([torch.nn.Linear(4096, 512, bias=False).bfloat16()] +
                                             [torch.nn.Linear(4096, 1025, bias=False).bfloat16() for _ in range(32)])
        for h in model.lm_heads:
            torch.nn.init.normal_(h.weight, 0.0, 0.02)
    # the text head of this small model has 512 rows: special token ids inside it
    model.config = SimpleNamespace(language_config=cfg, audio_assistant_gen_slot_token_id=100,
                                   audio_assistant_delay_slot_token_id=101, audio_end_token_id=102)
    return model


def _export(model, folder):
    layer = model.language_model.layers[0]
    a, m = layer.self_attn, layer.mlp
    weights = {
        (0, "qkv"): torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]).float().cpu(),
        (0, "out"): a.o_proj.weight.float().cpu(),
        (0, "up"): torch.cat([m.gate_proj.weight, m.up_proj.weight]).float().cpu(),
        (0, "down"): m.down_proj.weight.float().cpu(),
    }
    written = write_export(folder, weights, n_layers=1)
    # the public entry point checks all 36 layers' files exist; the model has one layer
    for i in range(1, 36):
        for p in ("qkv", "out", "up", "down"):
            os.symlink(folder / f"00_{p}.pt", folder / f"{i:02d}_{p}.pt")
    return {name: o.dequantize_signed(*written[0, name]) for name in ("qkv", "out", "up", "down")}


def test_from_pretrained_install_and_decode(dev, tmp_path):
    from moss_tts import MossTTS
    from moss_tts._runtime import w4g32
    from moss_tts._runtime.modules import Bf16Linear, QuantGateUpG32, QuantLinearG32
    from moss_tts._runtime.presets import install_gptq

    print("boundary: building the one-layer model", flush=True)
    model = _model(dev)
    deq = _export(model, tmp_path)
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
    L0 = dict(qkv=deq["qkv"], o=deq["out"], gate_up=deq["up"], down=deq["down"],
              input_norm=layer.input_layernorm.weight.detach().cpu(),
              post_norm=layer.post_attention_layernorm.weight.detach().cpu(),
              q_norm=a.q_norm.weight.detach().cpu(), k_norm=a.k_norm.weight.detach().cpu())
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
