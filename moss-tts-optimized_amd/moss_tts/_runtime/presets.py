"""``install_gptq``: the quantized-Linear module swap of the G32 preset.

The reference wires its G32 path in by registering packed buffers and flags on the fused
attention/MLP modules and branching on them (``src/moss_tts/_runtime/presets.py:6-41``,
``calibrated_backend.py:30-56``, ``llm.py:26-130``).  Here every projection of each decoder
layer becomes an explicit quantized module holding the row-packed INT4-G32 weight:

* ``self_attn.qkv_proj``  QuantLinearG32, the fused q||k||v weight (N = 6144 on Qwen3-8B), and
  ``q_proj``/``k_proj``/``v_proj`` as row views of it (no copy), so the model's own attention
  forward keeps working;
* ``self_attn.o_proj``    QuantLinearG32;
* ``mlp.gate_up_proj``    QuantGateUpG32 (gate rows first, SiLU*mul epilogue), with
  ``gate_proj``/``up_proj`` as row views, and ``mlp.forward`` rebound to
  ``down_proj(gate_up_proj(x))``;
* ``mlp.down_proj``       QuantLinearG32.

A one-row input runs the decode GEMV, more rows the MFMA prefill GEMM.  As in the reference,
installing after graph capture is an error (``calibrated_backend.py:36``).
"""
from __future__ import annotations

import types
from pathlib import Path

from . import export


def _backbone(target):
    """The MossTTS model (``.language_model.layers``) behind an engine, a FastLLM-like object or
    the model itself."""
    for path in (("llm", "model"), ("model",), ()):
        obj = target
        for attr in path:
            obj = getattr(obj, attr, None)
            if obj is None:
                break
        if obj is not None and hasattr(getattr(obj, "language_model", None), "layers"):
            return obj
    raise ValueError("install_gptq needs a MOSS-TTS model (with language_model.layers) or an engine holding one")


def _captured(target) -> bool:
    for obj in (target, getattr(target, "llm", None), getattr(target, "decode", None)):
        if obj is None:
            continue
        if getattr(obj, "graph", None) is not None or getattr(obj, "prefill_graphs", None):
            return True
    return False


def _mlp_forward(self, x):
    return self.down_proj(self.gate_up_proj(x))


def _weight_shape(module) -> tuple:
    """[out, in] of a bf16 Linear or of an already installed quantized module."""
    if hasattr(module, "weight"):
        return tuple(module.weight.shape)
    return (module.out_features, module.in_features)


def _device(module):
    for t in list(module.parameters()) + list(module.buffers()):
        return t.device
    raise ValueError("projection module holds no tensors")


def install_gptq(target, calibration_path, *, verify_sha256: bool = True, dequant: int | None = None) -> dict:
    """Load the calibrated export at ``calibration_path`` into ``target``'s decoder layers.
    Returns the export's ``config.json``.  ``ValueError`` for a bad export or a model it does
    not fit, ``RuntimeError`` after graph capture."""
    import torch

    from . import w4g32
    from .modules import QuantGateUpG32, QuantLinearG32

    if _captured(target):
        raise RuntimeError("Install calibrated projections before graph capture")
    model = _backbone(target)
    layers = list(model.language_model.layers)
    folder = Path(calibration_path)
    config = export.read_config(folder, n_layers=len(layers))
    mode = w4g32.EXACT if dequant is None else dequant

    # validate every shape against the model before touching any module
    plans = []
    for i, layer in enumerate(layers):
        a, m = layer.self_attn, layer.mlp
        q, k, v = (_weight_shape(p) for p in (a.q_proj, a.k_proj, a.v_proj))
        g, u = _weight_shape(m.gate_proj), _weight_shape(m.up_proj)
        if not (q[1] == k[1] == v[1] and g == u):
            raise ValueError(f"layer {i}: unexpected projection shapes")
        plans.append({"qkv": (q[0] + k[0] + v[0], q[1]), "out": _weight_shape(a.o_proj),
                      "up": (2 * g[0], g[1]), "down": _weight_shape(m.down_proj),
                      "split_qkv": (q[0], k[0], v[0]), "inter": g[0]})

    # every record is read (memory-mapped) and checked before anything is converted or swapped
    records = [{name: export.read_projection(folder, i, name, config, expected_shape=plan[name],
                                             verify_sha256=verify_sha256) for name in export.PROJECTIONS}
               for i, plan in enumerate(plans)]
    devices = [_device(layer.self_attn.o_proj) for layer in layers]
    if any(d.type != "cuda" for d in devices):
        raise ValueError("the model must be on the HIP device before install_gptq")

    with torch.no_grad():
        packed = [{name: export.to_device(rec, dev) for name, rec in recs.items()}
                  for recs, dev in zip(records, devices)]
        for layer, plan, pk in zip(layers, plans, packed):
            a, m = layer.self_attn, layer.mlp
            nq, nk, nv = plan["split_qkv"]
            qkv = pk["qkv"]
            a.qkv_proj = QuantLinearG32(qkv, dequant=mode)
            a.q_proj = QuantLinearG32(qkv.rows(0, nq), dequant=mode)
            a.k_proj = QuantLinearG32(qkv.rows(nq, nq + nk), dequant=mode)
            a.v_proj = QuantLinearG32(qkv.rows(nq + nk, nq + nk + nv), dequant=mode)
            a.o_proj = QuantLinearG32(pk["out"], dequant=mode)
            gu = pk["up"]
            n = plan["inter"]
            m.gate_up_proj = QuantGateUpG32(gu, dequant=mode)
            m.gate_proj = QuantLinearG32(gu.rows(0, n), dequant=mode)
            m.up_proj = QuantLinearG32(gu.rows(n, 2 * n), dequant=mode)
            m.down_proj = QuantLinearG32(pk["down"], dequant=mode)
            m.forward = types.MethodType(_mlp_forward, m)
            for mod in (a, m):
                mod._use_quantized = True
                mod._quant_group = export.GROUP
    model.weight_quantization = "gptq_w4g32"
    return config
