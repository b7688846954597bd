"""CPU oracle: one batch-1 decode step, and the prompt pass (prefill), composed from the
per-operation oracles.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Order of operations:
``src/moss_tts/_runtime/llm.py:227-260`` (fused residual path) with the projections as
dequant-then-matmul (``src/moss_tts/calibration.py:185-188``) rounded to bf16 at each
projection output, heads ``src/moss_tts/_runtime/llm.py:271-279``.

Pinning (tests/test_oracle_decode.py): ``decode_step`` against transformers' own ``Qwen3Model``
(the layers the reference's backbone runs) on the same bf16 weights, input embedding and KV rows:
logits and the written K/V row within 1e-2 relative L2 at positions 0 and 37; a wrong GQA head
mapping (0.11) or a dropped residual (1.45) fails it.  ``decode_step_w4a8`` against
``decode_step`` on the same INT4 weights: 4.9e-3 relative L2 (the int8 activation rounding), bar
3e-2; a dropped residual gives 1.41.
"""
from __future__ import annotations

import torch

from . import attention as oa
from . import pointwise as op
from . import w4a8 as o8
from . import w4g32 as ow


def decode_layer(L, i, residual, mlp, position, keys, values, cos, sin, eps=1e-6, linear=None):
    """One layer of the step (``src/moss_tts/_runtime/llm.py:227-260``) from the stream state
    ``(residual, mlp)`` (``mlp`` None at layer 0, where ``residual`` is the embedding).  Returns the
    layer's intermediates ``qkv, attn, o, act, mlp`` and the new ``residual`` (bf16 ``[1, n]``).
    ``linear(h, w)`` is the fp32 product (default ``F.linear(h.float(), w.float())``)."""
    lin = linear or ow.linear
    p = int(position)
    if mlp is None:
        h = op.rmsnorm(residual, L["input_norm"], eps)
    else:
        residual, h = op.add_rmsnorm(mlp, residual, L["input_norm"], eps)
    qkv = lin(h, L["qkv"]).bfloat16()
    q = op.qk_norm_rope_kv(qkv, L["q_norm"], L["k_norm"], cos[p:p + 1], sin[p:p + 1], keys[i], values[i],
                           torch.tensor([p]), eps)
    attn = oa.decode_attention(q, keys[i], values[i], p).bfloat16().view(1, -1)
    o = lin(attn, L["o"]).bfloat16()
    residual, h = op.add_rmsnorm(o, residual, L["post_norm"], eps)
    y = lin(h, L["gate_up"])
    n = y.shape[1] // 2
    act = ow.silu_mul_rounded(y[:, :n], y[:, n:])
    mlp = lin(act, L["down"]).bfloat16()
    return dict(qkv=qkv, attn=attn, o=o, act=act, mlp=mlp, residual=residual)


def decode_step(layers, final_norm, heads_w, text, audio, ids, position, keys, values, cos, sin, eps=1e-6,
                linear=None):
    """``layers``: an iterable of dicts with bf16 dequantized ``qkv``, ``o``, ``gate_up``, ``down``
    weights (or fp32 tensors holding bf16 values) and ``input_norm``, ``post_norm``, ``q_norm``,
    ``k_norm``; it is consumed once, in order, so a generator can dequantize one layer at a time.
    ``keys``/``values`` lists of ``[1, 8, L, 128]`` caches (updated in place).  Returns bf16 logits."""
    lin = linear or ow.linear
    residual = oa.embedding_sum(ids.view(-1), text, audio).view(1, -1)
    mlp = None
    for i, L in enumerate(layers):
        out = decode_layer(L, i, residual, mlp, position, keys, values, cos, sin, eps, lin)
        residual, mlp = out["residual"], out["mlp"]
    _, h = op.add_rmsnorm(mlp, residual, final_norm, eps)
    return lin(h, heads_w).bfloat16().view(-1)


def reversed_linear(h: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``F.linear`` with the K axis reversed: the same exact products summed in another fp32 order.
    The distance between ``decode_step`` with it and without it measures how far summation order
    alone moves a composed step (the oracle's own noise floor)."""
    return torch.nn.functional.linear(h.float().flip(-1), w.float().flip(-1))


def decode_layer_w4a8(L, i, residual, mlp, position, keys, values, cos, sin, eps=1e-6, reverse_f32=False):
    """One layer of the step in the W4A8 arithmetic (``oracle.w4a8``; order
    ``src/moss_tts/_runtime/llm.py:29-56,71-92``) from the stream state ``(residual, mlp)`` as in
    ``decode_layer``: ``L`` holds ``(q, z, s)`` code triples for ``qkv``, ``o``, ``gate_up``,
    ``down``.  Returns ``qkv, attn, o, act, mlp`` and the new ``residual``.  ``reverse_f32``: every
    projection's group combine in float32 in reverse group order (``oracle.w4a8._combine``)."""
    p = int(position)
    r = reverse_f32
    if mlp is None:
        h = op.rmsnorm(residual, L["input_norm"], eps)
    else:
        residual, h = op.add_rmsnorm(mlp, residual, L["input_norm"], eps)
    qkv = o8.w4a8_linear(h.view(-1), *L["qkv"], reverse_f32=r)[0].view(1, -1)
    q = op.qk_norm_rope_kv(qkv, L["q_norm"], L["k_norm"], cos[p:p + 1], sin[p:p + 1], keys[i], values[i],
                           torch.tensor([p]), eps)
    attn = oa.decode_attention(q, keys[i], values[i], p).bfloat16().view(1, -1)
    o = o8.w4a8_linear(attn.view(-1), *L["o"], reverse_f32=r)[0].view(1, -1)
    residual, h = op.add_rmsnorm(o, residual, L["post_norm"], eps)
    n = L["gate_up"][0].shape[0] // 2
    act = o8.w4a8_gateup_silu(h.view(-1), *L["gate_up"], n, reverse_f32=r)[0].view(1, -1)
    mlp = o8.w4a8_linear(act.view(-1), *L["down"], reverse_f32=r)[0].view(1, -1)
    return dict(qkv=qkv, attn=attn, o=o, act=act, mlp=mlp, residual=residual)


def decode_step_w4a8(layers, final_norm, heads_w, text, audio, ids, position, keys, values, cos, sin, eps=1e-6):
    """The same step with the four layer projections in the W4A8 arithmetic (``decode_layer_w4a8``);
    the heads stay dequant-then-matmul on ``heads_w``.  ``layers`` is consumed once, in order."""
    residual = oa.embedding_sum(ids.view(-1), text, audio).view(1, -1)
    mlp = None
    for i, L in enumerate(layers):
        out = decode_layer_w4a8(L, i, residual, mlp, position, keys, values, cos, sin, eps)
        residual, mlp = out["residual"], out["mlp"]
    _, h = op.add_rmsnorm(mlp, residual, final_norm, eps)
    return ow.linear(h, heads_w).bfloat16().view(-1)


def prefill_layer(L, i, residual, state, start, keys, values, cos, sin, eps=1e-6, linear=None):
    """One layer of the prompt pass (layer loop ``src/moss_tts/_runtime/prefill_pointwise.py:46-57``)
    from the stream state entering it: ``residual`` bf16 ``[n, 4096]`` and ``state``, its
    normalization with the layer's input norm.  q||k||v -> q/k head-norm + RoPE, K/V rows written
    at positions ``start .. start + n - 1`` of ``keys[i]``/``values[i]`` (``prefill_qkv.py:7-28``)
    -> causal attention over cache rows ``0 .. position`` (``llm.py:116-128``) -> O -> add-RMSNorm
    -> gate||up -> SiLU*mul -> down, all projections dequant-then-matmul rounded to bf16.  Returns
    ``q`` (after RoPE), ``attn``, ``o``, ``residual_mid``, ``state_mid`` (after the O projection's
    add-RMSNorm), ``act`` and ``mlp``."""
    lin = linear or ow.linear
    n = state.shape[0]
    pos = torch.arange(int(start), int(start) + n)
    qkv = lin(state, L["qkv"]).bfloat16()
    q = op.qk_norm_rope_kv(qkv, L["q_norm"], L["k_norm"], cos[pos], sin[pos], keys[i], values[i], pos, eps)
    attn = oa.prefill_attention(q, keys[i], values[i], int(start)).bfloat16().view(n, -1)
    o = lin(attn, L["o"]).bfloat16()
    residual_mid, state_mid = op.add_rmsnorm(o, residual, L["post_norm"], eps)
    y = lin(state_mid, L["gate_up"])
    h = y.shape[1] // 2
    act = ow.silu_mul_rounded(y[:, :h], y[:, h:])
    mlp = lin(act, L["down"]).bfloat16()
    return dict(q=q, attn=attn, o=o, residual_mid=residual_mid, state_mid=state_mid, act=act, mlp=mlp)


def prefill(layers, final_norm, heads_w, text, audio, ids, start, keys, values, cos, sin, eps=1e-6,
            linear=None):
    """The prompt pass (``src/moss_tts/_runtime/llm.py:204-207``, layer loop
    ``src/moss_tts/_runtime/prefill_pointwise.py:46-57``): ``ids [n, 33]`` at absolute positions
    ``start .. start + n - 1``; per layer ``prefill_layer``, the next layer's input norm applied to
    the residual sum ``mlp + residual``.  ``layers`` is consumed once, in order.  Returns the bf16
    logits of the last token through the final norm and the heads (``llm.py:206-207``)."""
    x = oa.embedding_sum(ids, text, audio)
    residual, mlp = x, None
    for i, L in enumerate(layers):
        if i == 0:
            state = op.rmsnorm(x, L["input_norm"], eps)
        else:
            residual, state = op.add_rmsnorm(mlp, residual, L["input_norm"], eps)
        out = prefill_layer(L, i, residual, state, start, keys, values, cos, sin, eps, linear)
        residual, mlp = out["residual_mid"], out["mlp"]
    _, h = op.add_rmsnorm(mlp[-1:], residual[-1:], final_norm, eps)
    return (linear or ow.linear)(h, heads_w).bfloat16().view(-1)
