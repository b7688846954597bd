"""MI355X (gfx950) INT4-G32 quantized-linear path of the MOSS-TTS 8B backbone.

``MossTTS.from_pretrained(preset="gptq", calibration_path=...)`` validates a calibrated export
and installs it into a loaded model as quantized projection modules running hand-written
HIP kernels (``moss_tts._runtime``).  Importing this package does not import torch.
"""

__all__ = ["MossTTS"]


def __getattr__(name):
    if name == "MossTTS":
        from .api import MossTTS

        return MossTTS
    raise AttributeError(name)
