"""Reader of the reference's calibrated GPTQ export (the on-disk contract of the G32 preset).

Layout (written by ``src/moss_tts/calibration.py:156-212``): ``config.json`` plus one file
``{layer:02d}_{projection}.pt`` per layer and projection (``qkv``, ``out``, ``up``, ``down``)
holding ``{"packed": u8 [N, K/2], "scales": bf16 [N, K/32], "shape": [N, K], "group": 32}``;
byte j of a packed row holds the two's-complement nibbles of codes 2j (low) and 2j+1 (high),
codes in [-7, 7] (``calibration.py:190-191``).  Validation follows the reference's
``MossTTS.from_pretrained`` (``src/moss_tts/api.py:83-98``) and ``install_calibrated``
(``src/moss_tts/_runtime/calibrated_backend.py:30-47``); in addition the per-file sha256 that
the export records in ``config["projections"][name]["sha256"]`` is checked when present.

Files are read with ``torch.load(..., weights_only=True)``: nothing in them is executed.
Reading and validation run on the CPU; ``to_device`` converts one record into the row-packed
kernel layout on the GPU (``w4g32.import_signed``, codes ``q = u ^ 8`` with zero point 8).
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass
from pathlib import Path

from ..models import TTS_REVISION

PROJECTIONS = ("qkv", "out", "up", "down")
GROUP = 32
LAYERS = 36


def _projection_paths(folder: Path, n_layers: int) -> dict:
    return {(i, p): folder / f"{i:02d}_{p}.pt" for i in range(n_layers) for p in PROJECTIONS}


def read_config(folder, n_layers: int = LAYERS) -> dict:
    """Parse and check ``config.json`` and the presence of every projection file.  Raises
    ``ValueError`` with the reference's messages (``api.py:83-98``)."""
    folder = Path(folder)
    path = folder / "config.json"
    if not path.is_file():
        raise ValueError(f"No config.json in the calibrated export {folder}")
    try:
        config = json.loads(path.read_text())
    except ValueError as exc:
        raise ValueError(f"Unreadable config.json in {folder}: {exc}") from None
    if not isinstance(config, dict):
        raise ValueError("config.json must hold an object")
    if config.get("complete") is False:
        raise ValueError("The calibrated export is incomplete")
    if config.get("group") != GROUP or config.get("tts_revision") != TTS_REVISION:
        raise ValueError("A G32 export of the pinned 8B revision is required")
    missing = [p for p in _projection_paths(folder, n_layers).values() if not p.is_file()]
    if missing:
        raise ValueError(f"Incomplete calibrated export: {len(missing)} projections missing")
    return config


@dataclass
class ExportRecord:
    layer: int
    name: str
    packed: "object"      # torch.uint8 [N, K/2] (CPU)
    scales: "object"      # torch.bfloat16 [N, K/32] (CPU)
    shape: tuple

    @property
    def N(self) -> int:
        return self.shape[0]

    @property
    def K(self) -> int:
        return self.shape[1]


def read_projection(folder, layer: int, name: str, config: dict | None = None, *,
                    expected_shape=None, verify_sha256: bool = True) -> ExportRecord:
    """Load one ``{layer:02d}_{name}.pt`` on the CPU and check it (``calibrated_backend.py:46-49``):
    shape and group, packed/scales dtypes and sizes, and the recorded sha256."""
    import torch

    folder = Path(folder)
    if name not in PROJECTIONS:
        raise ValueError(f"unknown projection {name!r}")
    key = f"{layer:02d}_{name}"
    path = folder / f"{key}.pt"
    if verify_sha256 and config is not None:
        digest = config.get("projections", {}).get(key, {}).get("sha256")
        if digest is not None and hashlib.sha256(path.read_bytes()).hexdigest() != digest:
            raise ValueError(f"sha256 mismatch for {path.name}")
    saved = torch.load(path, map_location="cpu", weights_only=True, mmap=True)
    if not isinstance(saved, dict) or not {"packed", "scales", "shape", "group"} <= set(saved):
        raise ValueError(f"{path.name} is not a calibrated projection record")
    shape = tuple(int(v) for v in saved["shape"])
    group = config.get("group", GROUP) if config is not None else GROUP
    if saved["group"] != group or len(shape) != 2:
        raise ValueError(f"Projection shape/group mismatch: {layer} {name}")
    if expected_shape is not None and tuple(expected_shape) != shape:
        raise ValueError(f"Projection shape/group mismatch: {layer} {name}")
    n, k = shape
    packed, scales = saved["packed"], saved["scales"]
    if k % 64 != 0:
        raise ValueError(f"{key}: K={k} must be a multiple of 64")
    if not (isinstance(packed, torch.Tensor) and packed.dtype == torch.uint8 and tuple(packed.shape) == (n, k // 2)):
        raise ValueError(f"{key}: packed must be uint8 [{n}, {k // 2}]")
    if not (isinstance(scales, torch.Tensor) and tuple(scales.shape) == (n, k // GROUP)
            and scales.dtype in (torch.bfloat16, torch.float32)):
        raise ValueError(f"{key}: scales must be bf16 (or bf16-exact fp32) [{n}, {k // GROUP}]")
    if scales.dtype == torch.float32:
        if not torch.equal(scales.bfloat16().float(), scales):
            raise ValueError(f"{key}: fp32 scales are not bf16-exact")
        scales = scales.bfloat16()
    return ExportRecord(layer, name, packed, scales, shape)


def to_device(record: ExportRecord, device):
    """Row-packed INT4-G32 weight on ``device`` (bit-exact: ``q = u ^ 8``, ``z = 8``)."""
    from . import w4g32

    return w4g32.import_signed(record.packed.contiguous().to(device), record.scales.contiguous().to(device))
