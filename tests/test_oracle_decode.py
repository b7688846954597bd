"""Pins the oracle's decode-step composition (``oracle/decode.py``) against transformers' own
Qwen3 model, the layers the reference's backbone runs (``src/moss_tts/_runtime/llm.py:227-266``
fuses the projections of transformers' ``Qwen3DecoderLayer``; ``TF/qwen3``).

The same bf16 weights, the same input embedding and the same KV-cache rows ``[0, p)`` go into
both; one decode step at position ``p`` must give the same logits and write the same K/V row.
This fixes what the per-operation checks leave open: the order of the operations in a layer,
the residual wiring across layers, the GQA head mapping (query head h reads KV head h // 4),
the q/k head-norm and RoPE placement, the SiLU*mul placement and the final norm.  Both run bf16
matmuls and attention with different accumulation orders, so the bar is a relative L2 error,
written below.
"""
import pytest
import torch
import torch.nn.functional as F
from transformers import DynamicCache, Qwen3Config
from transformers.models.qwen3.modeling_qwen3 import Qwen3Model

from oracle import attention as oa
from oracle import decode as od
from oracle import pointwise as op

REL_L2 = 1e-2


def _layer_dict(layer):
    a, m = layer.self_attn, layer.mlp
    return dict(qkv=torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]).detach(),
                o=a.o_proj.weight.detach(), gate_up=torch.cat([m.gate_proj.weight, m.up_proj.weight]).detach(),
                down=m.down_proj.weight.detach(), input_norm=layer.input_layernorm.weight.detach(),
                post_norm=layer.post_attention_layernorm.weight.detach(), q_norm=a.q_norm.weight.detach(),
                k_norm=a.k_norm.weight.detach())


@pytest.mark.parametrize("position", [0, 37])
def test_decode_step_matches_transformers_qwen3(position):
    torch.manual_seed(0)
    cfg = Qwen3Config(hidden_size=4096, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6, vocab_size=64,
                      max_position_embeddings=256, attn_implementation="eager")
    model = Qwen3Model(cfg).to(torch.bfloat16).eval()
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if "norm" in name:       # non-trivial norm weights, so their placement matters
                prm.copy_(1 + 0.1 * torch.randn_like(prm, dtype=torch.float32))
    L, p = 64, position
    keys = [torch.randn((1, 8, L, 128)).bfloat16() for _ in range(2)]
    values = [torch.randn((1, 8, L, 128)).bfloat16() for _ in range(2)]
    text = torch.randn((64, 4096)).bfloat16()
    audio = torch.randn((32, 16, 4096)).bfloat16()
    ids = torch.tensor([[5] + [i % 16 for i in range(32)]])
    heads = (torch.randn((96, 4096)) * 0.02).bfloat16()
    cos, sin = op.rope_tables(torch.arange(L))
    layers = [_layer_dict(layer) for layer in model.layers]
    k_or, v_or = [k.clone() for k in keys], [v.clone() for v in values]
    with torch.no_grad():
        ref = od.decode_step(layers, model.norm.weight.detach(), heads, text, audio, ids, p, k_or, v_or, cos, sin)
        x = oa.embedding_sum(ids.view(-1), text, audio).view(1, 1, 4096)
        cache = DynamicCache(config=cfg)
        for i in range(2):
            cache.update(keys[i][:, :, :p].clone(), values[i][:, :, :p].clone(), i)
        out = model(inputs_embeds=x, position_ids=torch.tensor([[p]]), past_key_values=cache, use_cache=True)
        got = F.linear(out.last_hidden_state.view(1, 4096), heads).view(-1)
    rel = float((got.float() - ref.float()).norm() / ref.float().norm())
    assert rel < REL_L2, rel
    for i in range(2):
        k_hf = cache.layers[i].keys[:, :, p].float()
        v_hf = cache.layers[i].values[:, :, p].float()
        k_rel = float((k_hf - k_or[i][:, :, p].float()).norm() / k_hf.norm())
        assert k_rel < REL_L2, (i, k_rel)
        assert torch.allclose(v_hf, v_or[i][:, :, p].float(), rtol=2e-2, atol=2e-2), i


def test_w4a8_step_follows_the_same_composition():
    """``decode_step_w4a8`` is ``decode_step`` with the four projections in the W4A8 arithmetic:
    on the same INT4 weights (dequantized for ``decode_step``) the two steps differ only by the
    int8 activation rounding, a few parts in a thousand of the logits; a wiring error (a dropped
    residual, a wrong head mapping) moves them by tens of percent."""
    from oracle import w4g32 as ow

    torch.manual_seed(1)
    L, p = 64, 21
    codes, deq = [], []
    for _ in range(2):
        c, d = {}, {}
        for name, shape in (("qkv", (6144, 4096)), ("o", (4096, 4096)), ("gate_up", (2048, 4096)),
                            ("down", (4096, 1024))):
            q, z, s = ow.quantize_minmax_g32(torch.randn(shape) * 0.02)
            c[name], d[name] = (q, z, s), ow.dequantize(q, z, s)
        for name, n in (("input_norm", 4096), ("post_norm", 4096), ("q_norm", 128), ("k_norm", 128)):
            c[name] = d[name] = (1 + 0.1 * torch.randn(n)).bfloat16()
        codes.append(c)
        deq.append(d)
    keys = [torch.randn((1, 8, L, 128)).bfloat16() for _ in range(2)]
    values = [torch.randn((1, 8, L, 128)).bfloat16() for _ in range(2)]
    text, audio = torch.randn((64, 4096)).bfloat16(), torch.randn((32, 16, 4096)).bfloat16()
    ids = torch.tensor([[7] + [i % 16 for i in range(32)]])
    heads = (torch.randn((96, 4096)) * 0.02).bfloat16()
    final = (1 + 0.1 * torch.randn(4096)).bfloat16()
    cos, sin = op.rope_tables(torch.arange(L))
    a = od.decode_step(deq, final, heads, text, audio, ids, p, [k.clone() for k in keys],
                       [v.clone() for v in values], cos, sin).float()
    b = od.decode_step_w4a8(codes, final, heads, text, audio, ids, p, [k.clone() for k in keys],
                            [v.clone() for v in values], cos, sin).float()
    rel = float((a - b).norm() / a.norm())
    assert rel < 3e-2, rel


@pytest.mark.parametrize("n,start", [(5, 0), (19, 0), (7, 9)])
def test_prefill_matches_transformers_qwen3(n, start):
    """The oracle's prompt pass against transformers' ``Qwen3Model`` run on the same prompt with its
    causal mask (and, for ``start > 0``, on top of the same cache prefix): the last token's logits and
    every K/V row the pass writes agree within the relative L2 bar; rows before ``start`` are left
    alone.  Planted wiring errors (a dropped mask, a wrong position offset) fail it."""
    torch.manual_seed(2)
    cfg = Qwen3Config(hidden_size=4096, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6, vocab_size=64,
                      max_position_embeddings=256, attn_implementation="eager")
    model = Qwen3Model(cfg).to(torch.bfloat16).eval()
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if "norm" in name:
                prm.copy_(1 + 0.1 * torch.randn_like(prm, dtype=torch.float32))
    L = 64
    keys = [torch.randn((1, 8, L, 128)).bfloat16() for _ in range(2)]
    values = [torch.randn((1, 8, L, 128)).bfloat16() for _ in range(2)]
    text = torch.randn((64, 4096)).bfloat16()
    audio = torch.randn((32, 16, 4096)).bfloat16()
    ids = torch.stack([torch.tensor([3 + t] + [(t + i) % 16 for i in range(32)]) for t in range(n)])
    heads = (torch.randn((96, 4096)) * 0.02).bfloat16()
    cos, sin = op.rope_tables(torch.arange(L))
    layers = [_layer_dict(layer) for layer in model.layers]
    k_or, v_or = [k.clone() for k in keys], [v.clone() for v in values]
    with torch.no_grad():
        ref = od.prefill(layers, model.norm.weight.detach(), heads, text, audio, ids, start, k_or, v_or, cos, sin)
        x = oa.embedding_sum(ids, text, audio).view(1, n, 4096)
        cache = DynamicCache(config=cfg)
        if start:
            for i in range(2):
                cache.update(keys[i][:, :, :start].clone(), values[i][:, :, :start].clone(), i)
        pos = torch.arange(start, start + n)
        out = model(inputs_embeds=x, position_ids=pos[None], past_key_values=cache, use_cache=True)
        got = F.linear(out.last_hidden_state[0, -1:], heads).view(-1)
    rel = float((got.float() - ref.float()).norm() / ref.float().norm())
    assert rel < REL_L2, rel
    for i in range(2):
        assert torch.equal(k_or[i][:, :, :start], keys[i][:, :, :start])
        k_hf = cache.layers[i].keys[:, :, start:start + n].float()
        v_hf = cache.layers[i].values[:, :, start:start + n].float()
        k_rel = float((k_hf - k_or[i][:, :, start:start + n].float()).norm() / k_hf.norm())
        assert k_rel < REL_L2, (i, k_rel)
        v_rel = float((v_hf - v_or[i][:, :, start:start + n].float()).norm() / v_hf.norm())
        assert v_rel < REL_L2, (i, v_rel)
    if n > 1:
        # planted errors: attention without the causal mask, RoPE positions shifted by one
        from oracle import attention as oa_mod

        plain = oa_mod.prefill_attention

        def unmasked(q, kc, vc, s0):
            end = s0 + q.shape[0]
            k = kc[0, :, :end].float()
            v = vc[0, :, :end].float()
            qh = q.float().view(q.shape[0], 8, 4, 128).permute(1, 2, 0, 3)
            w = torch.softmax(torch.matmul(qh, k[:, None].transpose(-1, -2)) * oa_mod.SCALE, -1)
            return torch.matmul(w, v[:, None]).permute(2, 0, 1, 3).reshape(q.shape[0], 32, 128).contiguous()

        oa_mod.prefill_attention = unmasked
        k_bad = [k.clone() for k in keys]
        try:
            od.prefill(layers, model.norm.weight.detach(), heads, text, audio, ids, start, k_bad,
                       [v.clone() for v in values], cos, sin)
        finally:
            oa_mod.prefill_attention = plain
        # the mask shapes every earlier token's layer-0 output, so layer 1's K rows move
        k_hf = cache.layers[1].keys[:, :, start:start + n - 1].float()
        moved = float((k_bad[1][:, :, start:start + n - 1].float() - k_hf).norm() / k_hf.norm())
        assert moved > 5 * REL_L2, moved
    # positions one further: RoPE is relative, so attention hardly changes, but the K rows land one
    # row later with the wrong absolute rotation
    k_shift = [k.clone() for k in keys]
    od.prefill(layers, model.norm.weight.detach(), heads, text, audio, ids, start + 1, k_shift,
               [v.clone() for v in values], cos, sin)
    k_hf = cache.layers[0].keys[:, :, start:start + n].float()
    moved = float((k_shift[0][:, :, start:start + n].float() - k_hf).norm() / k_hf.norm())
    assert moved > 5 * REL_L2, moved


def test_prefill_attention_brute_force():
    """The causal attention restated with float64 loops on a small case (two KV heads' worth of
    queries, a cache prefix): same values within fp32 rounding; and at start 0 it equals torch's
    ``scaled_dot_product_attention(is_causal=True)`` with each KV head repeated for its 4 queries."""
    g = torch.Generator().manual_seed(3)
    n, start, L = 6, 4, 16
    q = torch.randn((n, 32, 128), generator=g).bfloat16()
    kc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    vc = torch.randn((1, 8, L, 128), generator=g).bfloat16()
    got = oa.prefill_attention(q, kc, vc, start)
    for t in range(n):
        for h in (0, 5, 31):
            keys = range(start + t + 1)
            sc = [sum(float(q[t, h, d]) * float(kc[0, h // 4, j, d]) for d in range(128)) / 128 ** 0.5 for j in keys]
            mx = max(sc)
            w = [pow(2.718281828459045, v - mx) for v in sc]
            tot = sum(w)
            ref = [sum(w[j] * float(vc[0, h // 4, j, d]) for j in keys) / tot for d in range(0, 128, 17)]
            assert torch.allclose(got[t, h, ::17].double(), torch.tensor(ref, dtype=torch.float64), atol=1e-5), (t, h)
    sdpa = F.scaled_dot_product_attention(q.float().permute(1, 0, 2)[None],
                                          kc[:, :, :n].float().repeat_interleave(4, 1),
                                          vc[:, :, :n].float().repeat_interleave(4, 1), is_causal=True)
    assert torch.allclose(oa.prefill_attention(q, kc, vc, 0), sdpa[0].permute(1, 0, 2), atol=1e-5)
