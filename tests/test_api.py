"""The drop-in boundary on the CPU: ``MossTTS.from_pretrained`` configuration errors (the
reference's list, ``tests/test_api.py:101-114`` there), calibrated-export validation and
reading (``src/moss_tts/api.py:83-98``, ``_runtime/calibrated_backend.py:30-51``), and the
install-before-capture rule.  Nothing here launches a kernel."""
import json
import os
import subprocess
import sys
from types import SimpleNamespace

import pytest
import torch

from helpers import write_export
from oracle import w4g32 as o

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "moss-tts-optimized_amd")


def test_import_does_not_load_torch():
    subprocess.run([sys.executable, "-c", "import moss_tts, sys; assert 'torch' not in sys.modules"],
                   check=True, env={**os.environ, "PYTHONPATH": PKG})


@pytest.mark.parametrize("kwargs", [
    {"preset": "4b"},
    {"preset": "gptq"},
    {"calibration_path": "unwanted"},
    {"max_length": 127},
    {"cpu_threads": 0},
    {"preset": "gptq", "calibration_path": "unused", "max_length": 512},
    {},                                            # bf16 preset: not provided by this library
])
def test_configuration_rejected_before_loading(kwargs):
    from moss_tts import MossTTS

    with pytest.raises(ValueError):
        MossTTS.from_pretrained(**kwargs)


def _small_weights(n_layers, seed=0, hidden=128, inter=192, nq=128, nkv=64):
    g = torch.Generator().manual_seed(seed)
    shapes = {"qkv": (nq + 2 * nkv, hidden), "out": (hidden, nq), "up": (2 * inter, hidden), "down": (hidden, inter)}
    return {(i, p): torch.randn(shapes[p], generator=g) * 0.02 for i in range(n_layers) for p in shapes}


@pytest.mark.parametrize("mutate,match", [
    (lambda cfg, d: cfg.update(complete=False), "incomplete"),
    (lambda cfg, d: cfg.update(group=128), "G32 export"),
    (lambda cfg, d: cfg.update(tts_revision="0" * 40), "G32 export"),
    (lambda cfg, d: (d / "01_down.pt").unlink(), "1 projections missing"),
])
def test_export_validation_rejects(tmp_path, mutate, match):
    from moss_tts import MossTTS
    from moss_tts._runtime import export

    write_export(tmp_path, _small_weights(2), n_layers=2)
    cfg = json.loads((tmp_path / "config.json").read_text())
    mutate(cfg, tmp_path)
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match=match):
        export.read_config(tmp_path, n_layers=2)
    # from_pretrained validates the 36-layer export before touching a device
    with pytest.raises(ValueError):
        MossTTS.from_pretrained(preset="gptq", calibration_path=tmp_path)


def test_export_records_read_back_exactly(tmp_path):
    """Records come back as written; the exact bijection to the kernel layout (q = u ^ 8,
    z = 8) reproduces the reference's dequant bit for bit."""
    from moss_tts._runtime import export

    written = write_export(tmp_path, _small_weights(2, seed=1), n_layers=2)
    cfg = export.read_config(tmp_path, n_layers=2)
    for (layer, name), (codes, scales) in written.items():
        rec = export.read_projection(tmp_path, layer, name, cfg)
        assert rec.shape == tuple(codes.shape)
        assert torch.equal(o.unpack_signed(rec.packed), codes)
        assert torch.equal(rec.scales.view(torch.int16), scales.view(torch.int16))
        q, z, s = o.signed_export_to_codes(rec.packed, rec.scales)
        assert torch.equal(o.dequantize(q, z, s).view(torch.int16), o.dequantize_signed(codes, scales).view(torch.int16))


def test_export_sha_and_shape_checks(tmp_path):
    from moss_tts._runtime import export

    write_export(tmp_path, _small_weights(1, seed=2), n_layers=1)
    cfg = export.read_config(tmp_path, n_layers=1)
    with pytest.raises(ValueError, match="shape/group"):
        export.read_projection(tmp_path, 0, "qkv", cfg, expected_shape=(128, 128))
    rec = torch.load(tmp_path / "00_out.pt", weights_only=True)
    rec["packed"][0, 0] ^= 1
    torch.save(rec, tmp_path / "00_out.pt")
    with pytest.raises(ValueError, match="sha256"):
        export.read_projection(tmp_path, 0, "out", cfg)
    export.read_projection(tmp_path, 0, "out", cfg, verify_sha256=False)
    rec["scales"] = rec["scales"].float() * (1 + 2 ** -12)
    torch.save(rec, tmp_path / "00_out.pt")
    with pytest.raises(ValueError, match="bf16-exact"):
        export.read_projection(tmp_path, 0, "out", cfg, verify_sha256=False)


def test_install_refuses_after_capture_and_non_models(tmp_path):
    from moss_tts._runtime.presets import install_gptq

    with pytest.raises(RuntimeError, match="before graph capture"):
        install_gptq(SimpleNamespace(llm=SimpleNamespace(graph=object())), tmp_path)
    with pytest.raises(ValueError, match="language_model"):
        install_gptq(SimpleNamespace(), tmp_path)


def test_install_rejects_mismatched_export_before_swapping(tmp_path):
    """A shape mismatch is found before any module is replaced (CPU model: the device check
    comes after validation, so nothing is launched)."""
    from moss_tts._runtime.presets import install_gptq

    write_export(tmp_path, _small_weights(1, seed=3), n_layers=1)
    attn = torch.nn.Module()
    attn.q_proj, attn.k_proj, attn.v_proj = (torch.nn.Linear(128, n, bias=False) for n in (128, 64, 64))
    attn.o_proj = torch.nn.Linear(128, 128, bias=False)
    mlp = torch.nn.Module()
    mlp.gate_proj, mlp.up_proj = torch.nn.Linear(128, 96, bias=False), torch.nn.Linear(128, 96, bias=False)
    mlp.down_proj = torch.nn.Linear(96, 128, bias=False)
    layer = SimpleNamespace(self_attn=attn, mlp=mlp)
    model = SimpleNamespace(language_model=SimpleNamespace(layers=[layer]))
    with pytest.raises(ValueError, match="shape/group"):
        install_gptq(model, tmp_path)
    assert isinstance(mlp.gate_proj, torch.nn.Linear)
