"""Pins the pointwise oracle against the third-party modules the reference calls.

The reference's RMSNorm and RoPE semantics come from transformers' Qwen3 modules
(``Qwen3RMSNorm``, ``Qwen3RotaryEmbedding``, ``apply_rotary_pos_emb``; called at
``src/moss_tts/_runtime/llm.py:6,107,230``).  Those modules are importable here, so the
oracle is checked against them bit for bit, plus closed forms.
"""
import math

import pytest
import torch
from transformers import Qwen3Config
from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, Qwen3RotaryEmbedding, apply_rotary_pos_emb

from oracle import pointwise as p


def _norm_module(w, eps):
    m = Qwen3RMSNorm(w.numel(), eps=eps).to(torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(w)
    return m


def test_rmsnorm_matches_qwen3_module():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn((7, 4096), generator=g) * 3).bfloat16()
    w = (1 + torch.randn(4096, generator=g) * 0.01).bfloat16()
    with torch.no_grad():
        ref = _norm_module(w, 1e-6)(x)
    assert torch.equal(p.rmsnorm(x, w, 1e-6).view(torch.int16), ref.view(torch.int16))


def test_add_rmsnorm_matches_bf16_add_then_module():
    g = torch.Generator().manual_seed(1)
    x = torch.randn((3, 4096), generator=g).bfloat16()
    r = (torch.randn((3, 4096), generator=g) * 10).bfloat16()
    w = (1 + torch.randn(4096, generator=g) * 0.01).bfloat16()
    s, y = p.add_rmsnorm(x, r, w, 1e-6)
    assert torch.equal(s.view(torch.int16), (x + r).view(torch.int16))     # torch bf16 add rounds once
    with torch.no_grad():
        assert torch.equal(y.view(torch.int16), _norm_module(w, 1e-6)(x + r).view(torch.int16))


def test_rmsnorm_closed_form():
    x = torch.full((1, 4096), -3.0, dtype=torch.bfloat16)
    w = torch.full((4096,), 2.0, dtype=torch.bfloat16)
    y = p.rmsnorm(x, w, 0.0)
    assert torch.all(y == -2.0)          # x / rms(x) = -1 exactly, times 2


def test_rope_tables_match_qwen3_rotary():
    cfg = Qwen3Config(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                      rope_theta=1e6)
    rot = Qwen3RotaryEmbedding(cfg)
    pos = torch.tensor([0, 1, 7, 511, 2047])
    cos_ref, sin_ref = rot(torch.zeros(1, dtype=torch.bfloat16), pos[None])
    cos, sin = p.rope_tables(pos)
    assert torch.equal(cos.view(torch.int16), cos_ref[0].view(torch.int16))
    assert torch.equal(sin.view(torch.int16), sin_ref[0].view(torch.int16))
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)            # position 0 is the identity
    assert math.isclose(float(cos[1, 0]), math.cos(1.0), abs_tol=4e-3)  # inv_freq[0] = 1


@pytest.mark.parametrize("n", [1, 5])
def test_qk_norm_rope_matches_norm_module_then_apply_rotary(n):
    g = torch.Generator().manual_seed(2 + n)
    qkv = (torch.randn((n, 6144), generator=g) * 2).bfloat16()
    qw = (1 + torch.randn(128, generator=g) * 0.05).bfloat16()
    kw = (1 + torch.randn(128, generator=g) * 0.05).bfloat16()
    pos = torch.arange(3, 3 + n)
    cos, sin = p.rope_tables(pos)
    L = 16
    kc = torch.zeros((1, 8, L, 128), dtype=torch.bfloat16)
    vc = torch.zeros((1, 8, L, 128), dtype=torch.bfloat16)
    q = p.qk_norm_rope_kv(qkv, qw, kw, cos, sin, kc, vc, pos, 1e-6)
    # third-party composition used by the reference's unfused path (llm.py:102-114)
    qh = qkv[:, :4096].view(1, n, 32, 128)
    kh = qkv[:, 4096:5120].view(1, n, 8, 128)
    with torch.no_grad():
        qn = _norm_module(qw, 1e-6)(qh).transpose(1, 2)
        kn = _norm_module(kw, 1e-6)(kh).transpose(1, 2)
        q_ref, k_ref = apply_rotary_pos_emb(qn, kn, cos[None], sin[None])
    assert torch.equal(q.view(torch.int16), q_ref[0].transpose(0, 1).contiguous().view(torch.int16))
    assert torch.equal(kc[0][:, 3:3 + n].view(torch.int16), k_ref[0].view(torch.int16))
    assert torch.equal(vc[0][:, 3:3 + n], qkv[:, 5120:].view(n, 8, 128).transpose(0, 1))
    assert torch.count_nonzero(kc[0][:, :3]) == 0 and torch.count_nonzero(vc[0][:, 3 + n:]) == 0


def test_rope_negative_zero_rule():
    """Float negation of +0 gives -0 (prefill_qkv.py:52-53): both rotated terms zero gives +0 + -0 = +0,
    and with the cos term also -0 the result keeps the minus sign."""
    qkv = torch.zeros((1, 6144), dtype=torch.bfloat16)
    cos, sin = p.rope_tables(torch.tensor([5]))
    kc = torch.zeros((1, 8, 8, 128), dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    q = p.qk_norm_rope_kv(qkv, torch.ones(128, dtype=torch.bfloat16), torch.ones(128, dtype=torch.bfloat16),
                          cos, sin, kc, vc, torch.tensor([5]), 1e-6)
    assert torch.count_nonzero(q.float()) == 0


def test_silu_mul_matches_torch_silu():
    g = torch.Generator().manual_seed(9)
    x = (torch.randn((4, 2 * 1024), generator=g) * 4).bfloat16()
    y = p.silu_mul(x)
    gate, up = x[:, :1024].float(), x[:, 1024:].float()
    ref = (torch.nn.functional.silu(gate).bfloat16().float() * up).bfloat16()
    same = (y.view(torch.int16) == ref.view(torch.int16)).float().mean()
    assert same > 0.995
    assert torch.allclose(y.float(), ref.float(), rtol=2 ** -7, atol=1e-6)
