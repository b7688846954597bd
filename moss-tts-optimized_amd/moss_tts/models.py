"""Pinned checkpoint identities of the MOSS-TTS 8B model (``src/moss_tts/models.py:5-8``).

The checkpoint download and model construction of the reference (``models.py:11-38``) are not
part of this library: the quantized-linear path installs into a model the caller has already
loaded (``MossTTS.from_pretrained(..., model=...)``).
"""

MODEL_ID = "OpenMOSS-Team/MOSS-TTS-v1.5"
CODEC_ID = "OpenMOSS-Team/MOSS-Audio-Tokenizer"
TTS_REVISION = "cdd3b911b1585e3f2dbc7775ef10f9926f58850a"
CODEC_REVISION = "3cd226ba2947efa357ef453bcad111b6eafba782"


def load_models(*, cache_dir=None, local_files_only: bool = False):
    raise RuntimeError(
        "Loading the MOSS-TTS checkpoint and codec is outside this library; load the model "
        "yourself and pass it as MossTTS.from_pretrained(..., model=model)")
