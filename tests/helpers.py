"""Shared comparison helpers of the parity tests (bars written out in each docstring)."""
from fractions import Fraction

import torch

from oracle import w4g32 as o

ATOL = 1e-2
RTOL = 1e-2


def rn_f32(fr: Fraction) -> float:
    """Round a rational to the nearest float32 (ties to even), subnormals included."""
    if fr == 0:
        return 0.0
    sign = -1.0 if fr < 0 else 1.0
    v = abs(fr)
    e = v.numerator.bit_length() - v.denominator.bit_length()
    if Fraction(2) ** e > v:
        e -= 1
    ulp = max(e - 23, -149)
    scaled = v / Fraction(2) ** ulp
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * float(n) * 2.0 ** ulp


def _assert_close(got, ref, what):
    got = got.float().cpu()
    ref = ref.float().cpu()
    bad = (got - ref).abs() > ATOL + RTOL * ref.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} mismatches, max err {float((got - ref).abs().max())}"


def _bits(t):
    return t.cpu().contiguous().view(torch.int16)


def _assert_rne_or_adjacent(got, ref32, abs_sum, k, what):
    """Exact-dequant outputs are an fp32 dot of the bit-exact bf16 weights with x, so they
    differ from RNE(oracle fp32) only through fp32 summation order: each must lie within
    half a bf16 step plus 8 sqrt(K) 2^-24 sum|w x| of the oracle, and at most
    max(2, 1%) of them may differ from RNE(oracle) at all."""
    g = got.cpu().float().flatten()
    r = ref32.float().flatten()
    gb = got.cpu().contiguous().view(torch.int16).flatten()
    rb = ref32.bfloat16().contiguous().view(torch.int16).flatten()
    n_bad = int((gb != rb).sum())
    assert n_bad <= max(2, int(0.01 * g.numel())), f"{what}: {n_bad} outputs differ from RNE(oracle)"
    half_step = torch.where(g == 0, torch.zeros_like(g), 2.0 ** (torch.floor(torch.log2(g.abs())) - 8))
    bound = half_step + 8 * (k ** 0.5) * 2.0 ** -24 * abs_sum.float().flatten()
    err = (g - r).abs()
    assert torch.all(err <= bound), f"{what}: max excess {float((err - bound).max())}"


def _bf16_choices(v, window=2.0 ** -12):
    """bf16 roundings of fp32 ``v`` that a different fp32 summation order could produce:
    the RNE value, plus the other neighbour where ``v`` lies within ``window * |v|`` of the
    midpoint between them (the GEMV and the oracle sum in different orders, ~1e-6 apart)."""
    u = v.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    down = ((u >> 16) << 16).to(torch.int32).view(torch.float32)          # towards zero
    up = (((u >> 16) + 1) << 16).to(torch.int32).view(torch.float32)      # away from zero
    rne = v.bfloat16().float()
    mid = (down + up) / 2
    near = (v - mid).abs() <= window * v.abs()
    other = torch.where(rne == down, up, down)
    return rne, torch.where(near, other, rne)


def _assert_epilogue_close(got, gate32, up32, what):
    """Gate/up outputs: atol/rtol against the oracle's epilogue, where gate and up may take
    either bf16 rounding when their fp32 value sits on a rounding midpoint."""
    got = got.float().cpu()[0]
    gs = _bf16_choices(gate32[0])
    us = _bf16_choices(up32[0])
    ok = torch.zeros_like(got, dtype=torch.bool)
    for g in gs:
        for u in us:
            ref = o.silu_mul_rounded(g, u).float()
            ok |= (got - ref).abs() <= ATOL + RTOL * ref.abs()
    assert ok.all(), f"{what}: {int((~ok).sum())} outputs outside tolerance"
    plain = o.silu_mul_rounded(gate32[0], up32[0]).float()
    strict = (got - plain).abs() <= ATOL + RTOL * plain.abs()
    assert strict.float().mean() >= 0.999, f"{what}: {int((~strict).sum())} midpoint cases"


def write_export(folder, weights, *, n_layers, revision=None, complete=True, record_sha=True):
    """Write a calibrated export in the reference's format (``src/moss_tts/calibration.py:156-212``)
    from fp32 weights ``{(layer, name): [N, K]}``: static bf16 absmax/7 scales, round-to-nearest
    codes in [-7, 7], two's-complement nibbles.  Returns ``{(layer, name): (codes, scales)}``."""
    import hashlib
    import json
    from pathlib import Path

    from moss_tts.models import TTS_REVISION

    folder = Path(folder)
    folder.mkdir(parents=True, exist_ok=True)
    config = {"complete": complete, "group": 32, "tts_revision": revision or TTS_REVISION, "projections": {}}
    out = {}
    for (layer, name), w in weights.items():
        s = o.static_scales(w)
        c = o.quantize_symmetric(w, s)
        path = folder / f"{layer:02d}_{name}.pt"
        torch.save({"packed": o.pack_signed(c), "scales": s, "shape": list(w.shape), "group": 32}, path)
        if record_sha:
            config["projections"][f"{layer:02d}_{name}"] = {"sha256": hashlib.sha256(path.read_bytes()).hexdigest()}
        out[layer, name] = (c, s)
    assert n_layers * 4 == len(weights)
    (folder / "config.json").write_text(json.dumps(config))
    return out


def moss_model(dev, seed=0, *, text_vocab=512, token_ids=(100, 101, 102)):
    """A one-layer, full-width MOSS-TTS-shaped model built from transformers' own Qwen3 modules
    (hidden 4096, 32 query / 8 KV heads of 128, MLP 12288), with the reference's module names:
    ``language_model``, 32 audio embeddings ``emb_ext`` and ``lm_heads`` (the text head of
    ``text_vocab`` rows, then 32 codebook heads of 1025 rows).  Weights N(0, 0.02), norm weights
    1 + N(0, 0.01), text embeddings N(0, 1).  ``token_ids``: gen slot, delay slot and audio end ids,
    which must lie inside the text head."""
    from types import SimpleNamespace

    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model

    cfg = Qwen3Config(hidden_size=4096, intermediate_size=12288, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, num_hidden_layers=1, vocab_size=text_vocab, rms_norm_eps=1e-6, rope_theta=1e6)
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
        model.lm_heads = torch.nn.ModuleList([torch.nn.Linear(4096, text_vocab, bias=False).bfloat16()] +
                                             [torch.nn.Linear(4096, 1025, bias=False).bfloat16() for _ in range(32)])
        for h in model.lm_heads:
            torch.nn.init.normal_(h.weight, 0.0, 0.02)
    gen, delay, end = token_ids
    model.config = SimpleNamespace(language_config=cfg, audio_assistant_gen_slot_token_id=gen,
                                   audio_assistant_delay_slot_token_id=delay, audio_end_token_id=end)
    return model


def export_model(model, folder):
    """Export the one-layer model's projections in the reference's calibrated format (layer 0's files
    linked for layers 1..35, which the public entry point checks for); returns the reference's
    dequantization of each exported projection (bf16)."""
    import os

    layer = model.language_model.layers[0]
    a, m = layer.self_attn, layer.mlp
    weights = {
        (0, "qkv"): torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]).float().cpu(),
        (0, "out"): a.o_proj.weight.float().cpu(),
        (0, "up"): torch.cat([m.gate_proj.weight, m.up_proj.weight]).float().cpu(),
        (0, "down"): m.down_proj.weight.float().cpu(),
    }
    written = write_export(folder, weights, n_layers=1)
    for i in range(1, 36):
        for p in ("qkv", "out", "up", "down"):
            os.symlink(folder / f"00_{p}.pt", folder / f"{i:02d}_{p}.pt")
    return {name: o.dequantize_signed(*written[0, name]) for name in ("qkv", "out", "up", "down")}


def model_layer_cpu(model, deq):
    """The oracle's layer dict of the one-layer model: the exported projections' dequantization and
    the model's own norm weights."""
    layer = model.language_model.layers[0]
    a = layer.self_attn
    return dict(qkv=deq["qkv"], o=deq["out"], gate_up=deq["up"], down=deq["down"],
                input_norm=layer.input_layernorm.weight.detach().cpu(),
                post_norm=layer.post_attention_layernorm.weight.detach().cpu(),
                q_norm=a.q_norm.weight.detach().cpu(), k_norm=a.k_norm.weight.detach().cpu())
