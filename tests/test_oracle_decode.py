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
