"""GPU: the text phase of the drop-in engine, through the public entry point.

A one-layer, full-width MOSS-TTS-shaped model whose text head has the real vocabulary of 151,936
rows (the special token ids at their model-config values) is installed with
``MossTTS.from_pretrained(preset="gptq", model=...)``.  Then:

* ``prefill`` returns ``FastLLM.prefill``'s pair (``src/moss_tts/_runtime/llm.py:204-207,318``):
  the last token's text logits over the whole text head ``[1, 151936]`` and its audio logits
  ``[32, 1024]``.  A 150-token prompt replays the 160-token bucket graph (the gptq preset's buckets
  are 128/160/256/512, ``src/moss_tts/_runtime/presets.py:45``).
* ``full_step`` (``llm.py:321-325``) at the next position returns the text logits of that step.

Bars: each logit vector within relative L2 2e-2 of the oracle (``oracle.decode.prefill`` /
``decode_step`` with ``heads_w`` = the text head, on the exported projections' dequantization and
the model's own norms), the bar of the decode step tests; the K/V rows the text step writes within
the same bar; the greedy choice (argmax) equal to the oracle's, or -- only where the oracle's two
largest logits are within one bf16 step of each other -- one of those near-tied tokens.
"""
import pytest
import torch

from helpers import export_model, model_layer_cpu, moss_model
from oracle import decode as od

pytestmark = pytest.mark.gpu

VOCAB = 151936


def _rel(a, b):
    a, b = a.float().flatten(), b.float().flatten()
    return float((a - b).norm() / b.norm())


def _greedy_agrees(got, ref, what):
    got, ref = got.float().flatten(), ref.float().flatten()
    gi, ri = int(got.argmax()), int(ref.argmax())
    top = torch.topk(ref, 2).values
    step = 2.0 ** (torch.floor(torch.log2(top[0].abs())) - 7)          # one bf16 step at the maximum
    print(f"{what}: argmax {gi} (oracle {ri}), oracle top-2 gap {float(top[0] - top[1]):.4g}", flush=True)
    if gi == ri:
        return
    assert float(top[0] - top[1]) <= float(step), f"{what}: argmax {gi} != oracle {ri}"
    assert float(ref[ri] - ref[gi]) <= float(step), f"{what}: argmax {gi} is not a near-tied choice"


def test_text_phase_prefill_and_full_step(dev, tmp_path):
    from moss_tts import MossTTS
    from moss_tts._runtime.decode import AUDIO_END_ID, DELAY_SLOT_ID, GEN_SLOT_ID

    print("text phase: building the one-layer model with a 151936-row text head", flush=True)
    model = moss_model(dev, seed=3, text_vocab=VOCAB, token_ids=(GEN_SLOT_ID, DELAY_SLOT_ID, AUDIO_END_ID))
    deq = export_model(model, tmp_path)
    tts = MossTTS.from_pretrained(preset="gptq", calibration_path=tmp_path, device="cuda:0", model=model)
    eng = tts.engine.decode
    assert sorted(eng.prefill_graphs) == [128, 160, 256, 512]
    assert eng.text_graph is not None and eng.text_head.weight.data_ptr() == model.lm_heads[0].weight.data_ptr()

    keys = [k.cpu().clone() for k in eng.keys]
    values = [v.cpu().clone() for v in eng.values]
    n = 150
    g = torch.Generator().manual_seed(n)
    ids = torch.cat([torch.randint(0, VOCAB, (n, 1), generator=g), torch.randint(0, 1025, (n, 32), generator=g)], 1)
    print(f"text phase: prefill of {n} tokens", flush=True)
    text, audio = tts.prefill(ids.view(1, n, 33).to(dev))
    assert eng.last_prefill_bucket == 160
    assert text.shape == (1, VOCAB) and audio.shape == (32, 1024)
    text, audio = text.float().cpu(), audio.float().cpu()

    L0 = model_layer_cpu(model, deq)
    text_w = model.lm_heads[0].weight.detach().cpu()
    audio_w = torch.cat([h.weight[:1024] for h in model.lm_heads[1:]]).detach().cpu()
    both = torch.cat([audio_w, text_w])                       # one oracle pass yields both logit sets
    final = model.language_model.norm.weight.detach().cpu()
    text_emb, audio_emb = eng.text_embedding.cpu(), eng.audio_embedding.cpu()
    ref = od.prefill([L0], final, both, text_emb, audio_emb, ids, 0, keys, values, eng.cos.cpu(), eng.sin.cpu())
    ref_audio, ref_text = ref[:32 * 1024].view(32, 1024), ref[32 * 1024:]
    rel_t, rel_a = _rel(text, ref_text), _rel(audio, ref_audio)
    print(f"prefill: text logits relative L2 {rel_t:.3e}, audio logits {rel_a:.3e}", flush=True)
    assert rel_t < 2e-2 and rel_a < 2e-2
    _greedy_agrees(text, ref_text, "prefill text")

    # the next token of the text phase at row n (llm.py:321-325, streaming.py:96-101)
    nxt = torch.full((1, 1, 33), 1024, dtype=torch.int64)
    nxt[0, 0, 0] = int(ref_text.argmax())
    print("text phase: full_step", flush=True)
    step_text = tts.full_step(nxt.to(dev), n)
    assert step_text.shape == (1, VOCAB)
    step_text = step_text.float().cpu()
    ref_step = od.decode_step([L0], final, text_w, text_emb, audio_emb, nxt.view(1, 33), n, keys, values,
                              eng.cos.cpu(), eng.sin.cpu())
    rel = _rel(step_text, ref_step)
    print(f"full_step: text logits relative L2 {rel:.3e}", flush=True)
    assert rel < 2e-2
    _greedy_agrees(step_text, ref_step, "full_step text")
    for got, want in ((eng.keys[0], keys[0]), (eng.values[0], values[0])):
        assert _rel(got[:, :, n].cpu(), want[:, :, n]) < 2e-2

    # the graph replays what the eager pass computes, bit for bit
    with torch.inference_mode():
        eager = eng._text_forward().float().cpu()
    assert torch.equal(eager, step_text)
    tts.close()
