"""Public entry point: ``MossTTS.from_pretrained(preset="gptq", calibration_path=...)``.

Signature, argument meaning and the configuration errors raised before anything is loaded
follow the reference (``src/moss_tts/api.py:36-99``; its checks are pinned by
``tests/test_api.py:101-114``).  The SM90 / Triton / nvcc checks of the reference
(``api.py:79-82,99``) become a gfx950 device check and a check that ``libmoss_hip.so`` loads.
What this library provides after loading is the INT4-G32 path: the model's projections swapped
for quantized modules (``install_gptq``), the prompt pass captured per bucket length (``prefill``),
the text-phase step over the whole text head (``full_step``) and the batch-1 decode step captured
as one HIP graph (``step``).  The streaming product loop,
codec and voice cloning of the reference are not part of it.
"""
from __future__ import annotations

import threading
from contextlib import contextmanager
from pathlib import Path
from typing import Literal


class GptqEngine:
    """The installed model plus its decode step (``DecodeStepG32``)."""

    def __init__(self, model, *, max_length: int):
        from ._runtime.decode import DecodeStepG32

        self.model = model
        self.max_length = max_length
        self.decode = DecodeStepG32.from_model(model, max_length=max_length)
        self.first_audio = None

    @property
    def graph(self):
        return self.decode.graph

    def warmup(self) -> None:
        """Capture the prompt-pass buckets, the decode step and the text-phase step
        (``llm.py:209-225,289-301``; buckets ``presets.py:45``)."""
        self.decode.capture_prefill()
        self.decode.capture()
        if self.decode.text_head is not None:
            self.decode.capture_text()

    def prefill(self, ids, start: int = 0):
        """``(text logits [1, V], audio logits [32, 1024])`` of the prompt's last token."""
        return self.decode.prefill_logits(ids, start)

    def prefill_heads(self, ids, start: int = 0):
        """The same pass with the head logits in the decode step's layout."""
        return self.decode.prefill(ids, start)

    def full_step(self, ids, position: int):
        return self.decode.full_step(ids, position)

    def step(self, ids, position: int):
        return self.decode.step(ids, position)

    def next_ids(self, ids, position: int, audio_length: int, delay_length: int, seed: int | None = None):
        return self.decode.decode(ids, position, audio_length, delay_length, seed=seed)

    def enable_first_audio_graph(self, steps: int = 32) -> dict:
        """Capture the steps right after the audio start as one graph
        (``src/moss_tts/_runtime/first_audio_graph.py:93-110``); one graph serves every position."""
        from ._runtime.decode import FirstAudioGraph

        if self.first_audio is not None:
            raise RuntimeError("Install initial-audio graphs once, before accepting requests")
        if self.decode.graph is None:
            raise ValueError("Initial-audio graphs require a warmed decode step")
        graph = FirstAudioGraph(self.decode, steps)
        graph.warmup()
        self.first_audio = graph
        return {"codebooks": 32, "steps": graph.steps}

    def run_first_audio(self, ids, position: int, delay: int = -1, seed: int | None = None):
        if self.first_audio is None:
            raise RuntimeError("Warm the first-audio graph before use")
        return self.first_audio.run(ids, position, delay=delay, seed=seed)


class MossTTS:
    """One HIP device, one active request, all 32 acoustic codebooks."""

    sample_rate = 48000
    codebooks = 32

    def __init__(self, engine, *, device, preset: str):
        self._engine = engine
        self.device = device
        self.preset = preset
        self._lock = threading.Lock()
        self._closed = False

    @classmethod
    def from_pretrained(
        cls,
        *,
        preset: Literal["bf16", "gptq"] = "bf16",
        calibration_path: str | Path | None = None,
        device: str = "cuda:0",
        cache_dir: str | Path | None = None,
        local_files_only: bool = False,
        max_length: int = 1024,
        cpu_threads: int = 4,
        model=None,
    ) -> "MossTTS":
        """Validate the configuration, install the calibrated export into ``model`` and capture
        the decode graph.  ``model`` is an already loaded MOSS-TTS model on ``device`` (this
        library does not download checkpoints)."""
        if preset not in ("bf16", "gptq"):
            raise ValueError("preset must be 'bf16' or 'gptq'")
        if (preset == "gptq") != (calibration_path is not None):
            raise ValueError("Provide calibration_path exactly when preset='gptq'")
        if not isinstance(max_length, int) or max_length < 128 or max_length % 128:
            raise ValueError("max_length must be a positive multiple of 128")
        if preset == "gptq" and max_length != 1024:
            raise ValueError("Bundled gptq kernels require max_length=1024")
        if not isinstance(cpu_threads, int) or cpu_threads < 1:
            raise ValueError("cpu_threads must be positive")
        if preset != "gptq":
            raise ValueError("This library provides the 'gptq' (INT4-G32) preset only")
        from ._runtime import export

        export.read_config(calibration_path)

        import torch

        target = torch.device(device)
        if target.type != "cuda" or not torch.cuda.is_available():
            raise RuntimeError("MOSS-TTS 8B on this library requires an AMD Instinct MI355X (gfx950) HIP device")
        if target.index is None:
            target = torch.device("cuda", torch.cuda.current_device())
        from ._runtime import native

        native.lib()  # raises when libmoss_hip.so is not built
        try:
            native.device_arch(target.index)
        except RuntimeError as exc:
            raise ValueError(f"The gptq preset is qualified for gfx950 (MI355X) only: {exc}") from None

        if model is None:
            from .models import load_models

            model = load_models(cache_dir=cache_dir, local_files_only=local_files_only)
        from ._runtime.presets import install_gptq

        torch.set_num_threads(cpu_threads)
        with torch.cuda.device(target):
            install_gptq(model, calibration_path)
            engine = GptqEngine(model, max_length=max_length)
            engine.warmup()
        return cls(engine, device=target, preset=preset)

    @contextmanager
    def _request(self):
        if not self._lock.acquire(blocking=False):
            raise RuntimeError("This model is busy; finish or close the active stream first")
        try:
            if self._closed:
                raise RuntimeError("This model is closed")
            yield
        finally:
            self._lock.release()

    def prefill(self, ids, start: int = 0):
        """The prompt pass (``FastLLM.prefill``, ``src/moss_tts/_runtime/llm.py:204-207,303-318``):
        ``ids`` int64 ``[1, n, 33]`` written into the KV cache at rows ``start .. start + n - 1``;
        returns the last token's text logits over the whole text head ``[1, V]`` and its audio logits
        ``[32, 1024]`` (views of the bucket graph's output buffers, valid until the next prompt).
        Prompts of up to 128, 160, 256 or 512 tokens replay that bucket's graph."""
        with self._request():
            return self._engine.prefill(ids, start)

    def full_step(self, ids, position: int):
        """The text-phase step (``FastLLM.full_step``, ``src/moss_tts/_runtime/llm.py:321-325``): ``ids``
        int64 ``[1, 1, 33]`` at cache row ``position`` -> the text logits ``[1, V]`` over the whole
        text head (a view of the text graph's output buffer, valid until the next text step)."""
        with self._request():
            return self._engine.full_step(ids, position)

    def step(self, ids, position: int):
        """One batch-1 decode step: ``ids`` int64 ``[1, 33]`` (text token, 32 codebook codes) at
        cache row ``position`` -> head logits bf16 (32 audio heads, then the 2 text-head rows; a
        view of the graph's output buffer, valid until the next step)."""
        with self._request():
            return self._engine.step(ids, position)

    def next_ids(self, ids, position: int, audio_length: int = 32, delay_length: int = -1,
                 seed: int | None = None):
        """The same step with the reference's sampling and delay-pattern logic
        (``FastLLM.step``, ``src/moss_tts/_runtime/llm.py:327-338``): the next ids int64
        ``[1, 1, 33]``.  ``seed`` sets the sampler's seed first; ``None`` keeps the current one
        (the draws also depend on ``position``)."""
        with self._request():
            return self._engine.next_ids(ids, position, audio_length, delay_length, seed)

    def first_audio(self, ids, position: int, delay: int = -1, seed: int | None = None):
        """The steps after the audio start in one graph replay (``FirstAudioGraph.run``): ``ids`` is
        the audio-start row int64 ``[1, 1, 33]``; returns the next-id rows ``[steps, 33]`` and the
        final (text token, audio length, delay, position).  Needs
        ``engine.enable_first_audio_graph()`` first.  This starts a request's audio: with
        ``seed=None`` a fresh 63-bit seed is drawn from torch's default CPU generator, which the
        reference's ``torch.multinomial`` draws also advance, so repeated requests sample
        differently and ``torch.manual_seed`` makes a run reproducible."""
        if seed is None:
            import torch

            seed = int(torch.randint(0, 2**63 - 1, (1,)).item())
        with self._request():
            return self._engine.run_first_audio(ids, position, delay, seed)

    @property
    def engine(self):
        return self._engine

    def close(self) -> None:
        if not self._lock.acquire(blocking=False):
            raise RuntimeError("Close the active stream before closing the model")
        try:
            self._closed = True
        finally:
            self._lock.release()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
