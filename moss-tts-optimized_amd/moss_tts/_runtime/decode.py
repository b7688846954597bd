"""Batch-1 decode step of the Qwen3-8B backbone on the gfx950 kernels, captured as one graph.

Per layer (the order of ``src/moss_tts/_runtime/llm.py:227-260`` with fused residuals):
add-RMSNorm + q||k||v GEMV (one kernel) -> q/k head-norm + RoPE + KV write + split GQA
attention (one kernel) -> split merge -> O GEMV -> add-RMSNorm + gate||up GEMV with SiLU*mul
(one kernel) -> down GEMV.  The step starts with the
33-row embedding sum (``src/moss_tts/_runtime/kernels.py:7-26``) and ends with the final norm
and the 32 concatenated audio-codebook heads (``src/moss_tts/_runtime/llm.py:188-191,271-279``):
bf16 for an installed model, as the reference keeps them, or INT4-G32 for the synthetic
36-layer benchmark step.  With ``w4a8`` the four layer projections run the reference's serving
arithmetic instead (int8 activations per group of 32, integer dot products, fp32 group combine;
``src/moss_tts/_runtime/dp4a_scaled.py:22-95``): add-RMSNorm + int8 quantizer + q||k||v (one
kernel) -> attention with the int8 quantizer in its merge -> O -> add-RMSNorm + quantizer +
gate||up with SiLU*mul (one kernel) -> int8 quantizer + down (one kernel)
(``src/moss_tts/_runtime/llm.py:29-56,71-92``).
The heads matrix holds the 32 audio heads (``audio_stride`` rows each, the first 1024 sampled)
followed by the 2 text-head rows (gen slot, delay slot; ``llm.py:190-191``); the step ends with the
reference's sampling and token logic (``llm.py:278-287``): ``sample_topk`` on the text and audio
logits and the delay-pattern composition of the next 33 ids.
Static input buffers (ids, position, audio/delay lengths) make the step graph-capturable;
``decode()`` copies new inputs into them and replays the graph, as ``FastLLM.step`` does
(``src/moss_tts/_runtime/llm.py:327-338``); ``step()`` returns the logits of the same graph.
The text phase before the audio starts reads the whole text head (``lm_heads[0]``, bf16 as the
reference keeps it): ``prefill_logits`` returns the prompt's last-token text logits and its audio
logits (``FastLLM.prefill``, ``llm.py:204-207,303-318``) and ``full_step`` runs the layers and the
text head alone (``FastLLM.full_step``, ``llm.py:321-325``), captured as a graph of its own.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import attention, bf16, pointwise, sampling, w4a8, w4g32
from .modules import Bf16Linear, QuantGateUpG32, QuantLinearG32
from .w4g32 import _require

HIDDEN, INTER, QH, KH, HD = 4096, 12288, 32, 8, 128
CODEBOOKS, AUDIO_VOCAB = 32, 1025
SAMPLED_CODES = 1024                      # audio codes a head can emit (1024 is the pad code)
# MossTTSDelay token ids (the reference model config's defaults)
GEN_SLOT_ID, DELAY_SLOT_ID, AUDIO_START_ID, AUDIO_END_ID = 151656, 151662, 151652, 151653
PAD_ID = 151643                           # the text pad token of the prompt buckets
PREFILL_BUCKETS = (128, 160, 256, 512)    # prompt lengths captured as graphs for gptq (presets.py:45)


@dataclass
class DecoderLayerG32:
    qkv: QuantLinearG32
    o: QuantLinearG32
    gate_up: QuantGateUpG32
    down: QuantLinearG32
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor

    @property
    def nbytes(self) -> int:
        return sum(m.packed.nbytes for m in (self.qkv, self.o, self.gate_up, self.down))


def rope_tables(length: int, theta: float, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin ``[length, 128]`` bf16, as Qwen3RotaryEmbedding forms them: fp32
    ``inv_freq = 1/theta^(2i/128)``, ``freqs = position * inv_freq``, ``emb = cat(freqs,
    freqs)``, cos/sin in fp32, then bf16 (transformers ``modeling_qwen3.py:106-138``)."""
    inv = 1.0 / (theta ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))
    freqs = torch.arange(length, dtype=torch.float32)[:, None] @ inv[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().bfloat16().to(device), emb.sin().bfloat16().to(device)


class DecodeStepG32:
    """The INT4-G32 decode step.  ``max_length`` is the static KV capacity; the KV caches
    are ``[1, 8, max_length, 128]`` bf16 per layer and kind, like the reference's StaticCache
    (``src/moss_tts/_runtime/llm.py:192-193``)."""

    def __init__(self, layers: list[DecoderLayerG32], final_norm: torch.Tensor, heads: QuantLinearG32 | Bf16Linear,
                 text_embedding: torch.Tensor, audio_embedding: torch.Tensor, *, max_length: int,
                 eps: float = 1e-6, theta: float = 1e6, w4a8: bool = False, audio_stride: int = AUDIO_VOCAB,
                 greedy: bool = False, seed: int = 0, text_ids=(GEN_SLOT_ID, DELAY_SLOT_ID),
                 audio_end_id: int = AUDIO_END_ID, audio_start_id: int = AUDIO_START_ID,
                 text_head: Bf16Linear | None = None):
        _require(len(layers) > 0, "at least one layer")
        dev = final_norm.device
        _require(dev.type == "cuda", "the decode step runs on a HIP device")
        _require(max_length > 0 and max_length % 64 == 0, "max_length must be a positive multiple of 64")
        _require(heads.in_features == HIDDEN, "heads must read the 4096-wide hidden state")
        _require(audio_stride >= SAMPLED_CODES and heads.out_features == CODEBOOKS * audio_stride + 2,
                 "heads must hold 32 audio heads of audio_stride rows, then the 2 text-head rows")
        _require(text_head is None or (isinstance(text_head, Bf16Linear) and text_head.in_features == HIDDEN
                                       and text_head.weight.device == dev),
                 "text_head must be a bf16 [V, 4096] head on the step's device")
        self.layers = layers
        self.final_norm = final_norm
        self.heads = heads
        self.text_head = text_head
        self.text_embedding = text_embedding
        self.audio_embedding = audio_embedding
        self.max_length = max_length
        self.eps = eps
        self.w4a8 = bool(w4a8)
        self.device = dev
        self.keys = [torch.zeros((1, KH, max_length, HD), device=dev, dtype=torch.bfloat16) for _ in layers]
        self.values = [torch.zeros((1, KH, max_length, HD), device=dev, dtype=torch.bfloat16) for _ in layers]
        self.cos, self.sin = rope_tables(max_length, theta, dev)
        self.ids = torch.zeros((1, CODEBOOKS + 1), device=dev, dtype=torch.int64)
        self.position = torch.zeros(1, device=dev, dtype=torch.int64)
        self.ws = attention.workspace(max_length, dev)
        self.audio_stride = audio_stride
        self.greedy = bool(greedy)
        # the sampler's Philox key, read on the device at every replay: set per request
        self.seed_buf = sampling.seed_buffer(int(seed), dev)
        self.audio_end_id = int(audio_end_id)
        self.audio_start_id = int(audio_start_id)
        self.text_ids_host = tuple(int(t) for t in text_ids)
        self.text_ids = torch.tensor(list(self.text_ids_host), device=dev, dtype=torch.int64)
        self.audio_length = torch.full((1,), CODEBOOKS, device=dev, dtype=torch.int64)
        self.delay_length = torch.full((1,), -1, device=dev, dtype=torch.int64)
        self.text_index = torch.zeros(1, device=dev, dtype=torch.int64)
        self.audio_index = torch.zeros(CODEBOOKS, device=dev, dtype=torch.int64)
        self.next_ids = torch.zeros(CODEBOOKS + 1, device=dev, dtype=torch.int64)
        self.graph = None
        self.logits = None
        self.text_graph = None
        self.text_out = None
        self.pad_id = PAD_ID
        self.prefill_graphs = {}
        self.last_prefill_bucket = None           # the bucket graph the last prompt replayed (None: eager)

    # ------------------------------------------------------------------ forward
    def forward(self, head_count: int = CODEBOOKS, trace: list | None = None) -> torch.Tensor:
        """One step from the static ``ids``/``position`` buffers -> logits bf16 ``[N_heads]``.
        Every (add+)RMSNorm runs inside the projection that consumes it (``norm_gemv``).
        ``head_count`` < 32 computes and samples only the first ``head_count`` audio heads: valid
        while ``audio_length <= head_count``, when the composition masks every later channel
        (``src/moss_tts/_runtime/llm.py:272-279``, ``audio_head_buckets.py``).  The reference fills
        the skipped heads with zeros and samples all 32 rows to keep torch's RNG sequence; here each
        row's Philox draw is independent of the others, so the skipped rows are left unwritten and
        unsampled and the emitted ids are those of the full step.  ``trace`` (eager runs only): a list
        that receives, per layer, copies of the stream state it started from (``residual_in``,
        ``mlp_in``) and of its intermediates (``qkv``, ``attn``, ``o``, ``act``, ``mlp``, ``residual``),
        for layer-by-layer checks."""
        _require(head_count in (8, 16, 24, CODEBOOKS), "head_count must be 8, 16, 24 or 32")
        mlp, residual = self._layers(trace)
        logits = self._heads(mlp, residual, head_count)
        self._sample(logits, head_count)
        return logits

    def _layers(self, trace: list | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """The embedding sum and every layer from the static ``ids``/``position`` buffers -> the last
        layer's MLP output and the residual stream (bf16 ``[1, 4096]`` each), before the final norm."""
        if self.w4a8:
            return self._layers_w4a8(trace)
        eps = self.eps
        x = attention.embedding_sum(self.ids, self.text_embedding, self.audio_embedding).view(1, HIDDEN)
        residual = x
        mlp = None
        for i, layer in enumerate(self.layers):
            state = (residual.clone(), None if mlp is None else mlp.clone()) if trace is not None else None
            if i == 0:
                qkv = w4g32.norm_gemv(x, layer.input_norm, eps, layer.qkv.packed, dequant=layer.qkv.dequant)
            else:
                residual, qkv = w4g32.norm_gemv(mlp, layer.input_norm, eps, layer.qkv.packed, residual=residual,
                                                dequant=layer.qkv.dequant)
            attn = attention.decode_attention_qkv(qkv, layer.q_norm, layer.k_norm, self.cos, self.sin, self.keys[i],
                                                  self.values[i], self.position, eps, ws=self.ws)
            o = layer.o(attn.view(1, HIDDEN))
            residual, act = w4g32.norm_gateup_silu(o, layer.post_norm, eps, layer.gate_up.packed,
                                                   residual=residual, dequant=layer.gate_up.dequant)
            mlp = layer.down(act)
            if trace is not None:
                trace.append(dict(residual_in=state[0], mlp_in=state[1], qkv=qkv.clone(), attn=attn.clone(),
                                  o=o.clone(), act=act.clone(), mlp=mlp.clone(), residual=residual.clone()))
        return mlp, residual

    def _text_logits(self, mlp: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        """Final add-RMSNorm + the whole text head (``F.linear(h, lm_heads[0].weight)``,
        ``src/moss_tts/_runtime/llm.py:207,318,325``) -> bf16 ``[1, V]``."""
        _require(self.text_head is not None, "the text phase needs the model's text head (lm_heads[0])")
        return bf16.norm_gemv(mlp, self.final_norm, self.eps, self.text_head.weight,
                              residual=residual)[1].view(1, -1)

    def _heads(self, mlp: torch.Tensor, residual: torch.Tensor, head_count: int) -> torch.Tensor:
        """Final add-RMSNorm + the heads (bf16 as the reference keeps them, or INT4-G32): all rows,
        or the first ``head_count`` audio heads and the 2 text rows written into one full-size
        logits buffer."""
        eps, heads = self.eps, self.heads

        def run(start, stop, out=None):
            if isinstance(heads, Bf16Linear):
                w = heads.weight if (start, stop) == (0, heads.out_features) else heads.weight[start:stop]
                return bf16.norm_gemv(mlp, self.final_norm, eps, w, residual=residual, out=out)[1]
            w = heads.packed if (start, stop) == (0, heads.out_features) else heads.packed.rows(start, stop)
            return w4g32.norm_gemv(mlp, self.final_norm, eps, w, residual=residual, dequant=heads.dequant,
                                   out=out)[1]

        if head_count == CODEBOOKS:
            return run(0, heads.out_features).view(-1)
        n_audio = CODEBOOKS * self.audio_stride
        logits = torch.empty(heads.out_features, device=self.device, dtype=torch.bfloat16)
        rows = head_count * self.audio_stride
        run(0, rows, logits[:rows])
        run(n_audio, n_audio + 2, logits[n_audio:])
        return logits

    def _sample(self, logits: torch.Tensor, head_count: int = CODEBOOKS) -> None:
        """Text and audio sampling and the next-id composition into ``next_ids`` (``llm.py:278-287``):
        text top-2 at temperature 1.5, audio top-25 / top-p 0.8 at temperature 1.7, or argmax when
        greedy."""
        n_audio = CODEBOOKS * self.audio_stride
        sampling.sample_topk_pair(
            dict(logits=logits[n_audio:n_audio + 2], temperature=0.0 if self.greedy else 1.5, top_k=2, top_p=1.0,
                 salt=1, out=self.text_index),
            dict(logits=logits[:head_count * self.audio_stride].view(head_count, self.audio_stride),
                 temperature=0.0 if self.greedy else 1.7, top_k=25, top_p=0.8, salt=0, vocab=SAMPLED_CODES,
                 out=self.audio_index[:head_count]),
            seed=self.seed_buf, position=self.position)
        sampling.compose_next_ids(self.text_index, self.audio_index, self.text_ids, self.audio_length,
                                  self.delay_length, delay_slot_id=int(self.text_ids_host[1]),
                                  audio_end_id=self.audio_end_id, out=self.next_ids)

    def _layers_w4a8(self, trace: list | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        eps = self.eps
        x = attention.embedding_sum(self.ids, self.text_embedding, self.audio_embedding).view(1, HIDDEN)
        residual = x
        mlp = None
        for i, layer in enumerate(self.layers):
            state = (residual.clone(), None if mlp is None else mlp.clone()) if trace is not None else None
            # add-RMSNorm + quantizer + q||k||v in one kernel (8 waves per workgroup: 2 K slices x
            # 4 row groups of 2 rows, so 768 workgroups repeat the normalization); measured faster
            # than one row per wave over the whole K and than the separate norm_quant in front of
            # the K-split projection
            if i == 0:
                qkv = w4a8.norm_linear(x, layer.input_norm, eps, layer.qkv.packed, rows_per_wave=2)
            else:
                residual, qkv = w4a8.norm_linear(mlp, layer.input_norm, eps, layer.qkv.packed, residual=residual,
                                                 rows_per_wave=2)
            attn, act = attention.decode_attention_qkv(qkv, layer.q_norm, layer.k_norm, self.cos, self.sin,
                                                       self.keys[i], self.values[i], self.position, eps, ws=self.ws,
                                                       quantize=True)
            o = w4a8.linear(None, layer.o.packed, prequantized=act)
            # add-RMSNorm + quantizer + gate/up + SiLU*mul in one kernel (the same K-split fused
            # form as q||k||v: 1536 workgroups repeat the normalization), measured faster than the
            # separate norm_quant in front of the K-split gate/up; the SiLU*mul output is quantized
            # inside the down projection's kernel (each lane its own group of 32), faster than the
            # gate/up's fused output quantizer (its 32-row workgroups hold fewer rows in flight) and
            # than a separate quantizer launch
            residual, hidden = w4a8.norm_linear(o.view(1, HIDDEN), layer.post_norm, eps, layer.gate_up.packed,
                                                residual=residual, paired=True, rows_per_wave=2)
            mlp = w4a8.linear(hidden, layer.down.packed).view(1, HIDDEN)
            if trace is not None:
                trace.append(dict(residual_in=state[0], mlp_in=state[1], qkv=qkv.clone(), attn=attn.clone(),
                                  o=o.clone(), act=hidden.clone(), mlp=mlp.clone(), residual=residual.clone()))
        return mlp, residual

    @torch.inference_mode()
    def capture(self) -> None:
        """Warm up on a side stream, then capture one step as a graph (``llm.py:289-301``)."""
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(2):
                self.forward()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self.forward()
        torch.cuda.synchronize(self.device)

    @torch.inference_mode()
    def step(self, ids: torch.Tensor, position: int) -> torch.Tensor:
        """``ids`` int64 ``[1, 33]`` (host or device), ``0 <= position < max_length``."""
        if not 0 <= position < self.max_length:
            raise ValueError("KV capacity exceeded")
        self.ids.copy_(ids.reshape(1, CODEBOOKS + 1))
        self.position.fill_(position)
        if self.graph is None:
            return self.forward()
        self.graph.replay()
        return self.logits

    @property
    def seed(self) -> int:
        """The sampler's 64-bit seed (reads the device buffer)."""
        return int(self.seed_buf.item()) & 0xFFFFFFFFFFFFFFFF

    @seed.setter
    def seed(self, value: int) -> None:
        with torch.inference_mode():
            self.seed_buf.fill_(sampling.seed_value(int(value)))

    @torch.inference_mode()
    def decode(self, ids: torch.Tensor, position: int, audio_length: int = CODEBOOKS,
               delay_length: int = -1, *, seed: int | None = None) -> torch.Tensor:
        """One step with the reference's ``FastLLM.step`` contract (``llm.py:327-338``): int64 ids
        ``[1, 33]`` in, the next ids ``[1, 1, 33]`` out (sampled on the device).  ``seed`` sets the
        sampler's key first (a captured graph reads it at replay); ``None`` keeps the current one."""
        if not 0 <= position < self.max_length:
            raise ValueError("KV capacity exceeded")
        if seed is not None:
            self.seed = seed
        self.audio_length.fill_(audio_length)
        self.delay_length.fill_(delay_length)
        self.step(ids, position)
        return self.next_ids.clone().view(1, 1, CODEBOOKS + 1)

    # ------------------------------------------------------------------ text phase
    def _text_forward(self) -> torch.Tensor:
        mlp, residual = self._layers()
        return self._text_logits(mlp, residual)

    @torch.inference_mode()
    def capture_text(self) -> None:
        """Capture the text-phase step (every layer, then the final norm and the whole text head) as
        a graph of its own.  The reference runs ``full_step`` eagerly (``llm.py:321-325``); the graph
        gives the same result without a host launch per kernel."""
        _require(self.text_head is not None, "the text phase needs the model's text head (lm_heads[0])")
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(2):
                self._text_forward()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self._text_forward()
        torch.cuda.synchronize(self.device)
        self.text_graph, self.text_out = graph, out

    @torch.inference_mode()
    def full_step(self, ids: torch.Tensor, position: int) -> torch.Tensor:
        """The text-phase step (``FastLLM.full_step``, ``src/moss_tts/_runtime/llm.py:321-325``): ``ids``
        int64 ``[1, 1, 33]`` (or ``[1, 33]``) at cache row ``position``, K/V written there; returns the
        text logits bf16 ``[1, V]`` over the whole text head (a view of the graph's output buffer once
        ``capture_text`` has run, valid until the next text step)."""
        if not 0 <= position < self.max_length:
            raise ValueError("KV capacity exceeded")
        self.ids.copy_(ids.reshape(1, CODEBOOKS + 1))
        self.position.fill_(position)
        if self.text_graph is None:
            return self._text_forward()
        self.text_graph.replay()
        return self.text_out

    # ------------------------------------------------------------------ prefill
    def _prefill_body(self, ids: torch.Tensor, positions: torch.Tensor, start: torch.Tensor,
                      last: torch.Tensor, trace: list | None = None) -> torch.Tensor:
        """The prompt pass over ``n`` tokens (``src/moss_tts/_runtime/llm.py:204-207``; layer loop
        ``src/moss_tts/_runtime/prefill_pointwise.py:46-57``): embedding sum -> per layer the q||k||v
        GEMM -> q/k head-norm + RoPE with the K/V rows written at ``positions``
        (``prefill_qkv.py:31-53``) -> causal attention over cache rows ``0 .. position``
        (``llm.py:116-128``) -> O GEMM -> add-RMSNorm -> gate||up GEMM -> SiLU*mul -> down GEMM ->
        add-RMSNorm into the next layer; the last layer writes every token's K/V rows and runs its
        attention, O projection and MLP for the token ``last`` alone (only its logits are returned),
        then the final add-RMSNorm + heads on it.
        ``ids`` int64 ``[n, 33]``, ``positions`` int64 ``[n]`` (= start + arange(n)), ``start`` and
        ``last`` int64 ``[1]``, all on the device.  Returns the head logits as ``forward`` does and,
        when the step holds the text head, the text logits ``[1, V]`` (else None).
        ``trace`` (eager runs only): a list that receives, per layer, copies of the stream state it
        starts from (``residual_in``, its normalized form ``state_in``) and of its outputs: the
        RoPE'd queries ``q``, ``attn``, the residual and normalized state after the O projection
        (``residual_mid``, ``state_mid``), ``act`` and the state after the MLP (``residual_out``,
        ``state_out``, normalized with the next layer's input norm); the last layer's attention,
        O and MLP outputs are the last token's, and it records ``mlp`` instead of the state after it."""
        n, eps = ids.shape[0], self.eps
        x = attention.embedding_sum(ids, self.text_embedding, self.audio_embedding)
        residual = x
        state = pointwise.rmsnorm(x, self.layers[0].input_norm, eps)
        qbuf = torch.empty((n, QH, HD), device=self.device, dtype=torch.bfloat16)
        for i, layer in enumerate(self.layers):
            rec = dict(residual_in=residual.clone(), state_in=state.clone()) if trace is not None else None
            w4g32.gemm_qk_rope(state, layer.qkv.packed, layer.q_norm, layer.k_norm, self.cos, self.sin, self.keys[i],
                               self.values[i], positions, eps, out=qbuf)
            if rec is not None:
                rec["q"] = qbuf.clone()
                trace.append(rec)
            if i + 1 == len(self.layers):
                break
            attn = attention.prefill_attention(qbuf, self.keys[i], self.values[i], start)
            residual, state = w4g32.gemm_add_rmsnorm(attn, layer.o.packed, residual, layer.post_norm, eps)
            act = w4g32.gemm_silu(state, layer.gate_up.packed)
            if rec is not None:
                rec.update(attn=attn.clone(), residual_mid=residual.clone(), state_mid=state.clone(), act=act.clone())
            residual, state = w4g32.gemm_add_rmsnorm(act, layer.down.packed, residual, self.layers[i + 1].input_norm,
                                                     eps)
            if rec is not None:
                rec.update(residual_out=residual.clone(), state_out=state.clone())
        # Only the last token's hidden state reaches the logits, so after the last layer's K/V rows
        # are written for every token, its attention, O projection and MLP run for that token alone
        # (the decode step's kernels, exact dequant as the GEMMs): per-row math equal to the full
        # pass up to fp32 summation order.
        layer, i = self.layers[-1], len(self.layers) - 1
        attn = attention.decode_attention(qbuf.index_select(0, last), self.keys[i], self.values[i],
                                          positions.index_select(0, last), ws=self.ws)
        o = w4g32.gemv(attn.view(1, HIDDEN), layer.o.packed)
        residual, act = w4g32.norm_gateup_silu(o, layer.post_norm, eps, layer.gate_up.packed,
                                               residual=residual.index_select(0, last))
        mlp = w4g32.gemv(act, layer.down.packed)
        if trace is not None:
            trace[-1].update(attn=attn.clone().view(1, HIDDEN), o=o.clone(), residual_mid=residual.clone(),
                             act=act.clone(), mlp=mlp.clone())
        logits = self._heads(mlp, residual, CODEBOOKS)
        return logits, (self._text_logits(mlp, residual) if self.text_head is not None else None)

    def _prefill_inputs(self, ids: torch.Tensor, start: int, rows: int):
        n = ids.shape[0]
        static = torch.full((rows, CODEBOOKS + 1), SAMPLED_CODES, device=self.device, dtype=torch.int64)
        static[:, 0] = self.pad_id
        static[:n].copy_(ids)
        positions = torch.arange(start, start + rows, device=self.device, dtype=torch.int64)
        return (static, positions, torch.full((1,), start, device=self.device, dtype=torch.int64),
                torch.full((1,), n - 1, device=self.device, dtype=torch.int64))

    @torch.inference_mode()
    def capture_prefill(self, buckets=PREFILL_BUCKETS) -> None:
        """Capture the prompt pass for each bucket length as a graph (``llm.py:209-225``): a prompt of
        ``n`` tokens replays the smallest bucket ``>= n``, padded with the pad token and code 1024; the
        padded rows write K/V rows past the prompt, which the decode steps overwrite before they are
        read.  Install before the first request; the graphs share the engine's caches."""
        for b in sorted(set(int(x) for x in buckets)):
            if not 0 < b < self.max_length or b in self.prefill_graphs:
                continue
            inputs = self._prefill_inputs(torch.full((1, CODEBOOKS + 1), SAMPLED_CODES, device=self.device,
                                                     dtype=torch.int64), 0, b)
            side = torch.cuda.Stream(self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):
                for _ in range(2):
                    self._prefill_body(*inputs)
            torch.cuda.current_stream(self.device).wait_stream(side)
            torch.cuda.synchronize(self.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = self._prefill_body(*inputs)
            torch.cuda.synchronize(self.device)
            self.prefill_graphs[b] = (graph, inputs, out)

    @torch.inference_mode()
    def prefill(self, ids: torch.Tensor, start: int = 0) -> torch.Tensor:
        """The prompt pass (``src/moss_tts/_runtime/llm.py:303-318``) in the layout of ``step``: ``ids``
        int64 ``[1, n, 33]`` (or ``[n, 33]``) at cache rows ``start .. start + n - 1``; writes those K/V
        rows of every layer and returns the last token's head logits (32 audio heads, then the 2
        text-head rows).  ``prefill_logits`` returns the same pass in the reference's layout."""
        return self._prefill(ids, start)[0]

    @torch.inference_mode()
    def prefill_logits(self, ids: torch.Tensor, start: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
        """The prompt pass with ``FastLLM.prefill``'s result (``src/moss_tts/_runtime/llm.py:204-207,
        318``): the last token's text logits over the whole text head, bf16 ``[1, V]``, and its audio
        logits ``[32, 1024]`` (rows ``[:1024]`` of each codebook head).  Both are views of the bucket
        graph's output buffers when a bucket serves the prompt, valid until the next prompt."""
        _require(self.text_head is not None, "the text phase needs the model's text head (lm_heads[0])")
        logits, text = self._prefill(ids, start)
        audio = logits[:CODEBOOKS * self.audio_stride].view(CODEBOOKS, self.audio_stride)[:, :SAMPLED_CODES]
        return text, audio

    def _prefill(self, ids: torch.Tensor, start: int):
        """A captured bucket serves the prompt when one fits (the smallest bucket ``>= n``), else
        it runs eagerly."""
        ids = ids.reshape(-1, CODEBOOKS + 1)
        n = ids.shape[0]
        if n < 1 or start < 0 or start + n > self.max_length:
            raise ValueError("Batch must be one and prompt must fit the KV capacity")
        fits = [b for b in self.prefill_graphs if b >= n and start + b <= self.max_length]
        if fits:
            graph, (s_ids, s_pos, s_start, s_last), out = self.prefill_graphs[min(fits)]
            b = s_ids.shape[0]
            s_ids.fill_(SAMPLED_CODES)
            s_ids[:, 0] = self.pad_id
            s_ids[:n].copy_(ids)
            s_pos.copy_(torch.arange(start, start + b, dtype=torch.int64))
            s_start.fill_(start)
            s_last.fill_(n - 1)
            graph.replay()
            self.last_prefill_bucket = b
            return out
        self.last_prefill_bucket = None
        return self._prefill_body(*self._prefill_inputs(ids.to(self.device), start, n))

    @property
    def weight_bytes(self) -> int:
        heads = self.heads.nbytes if isinstance(self.heads, Bf16Linear) else self.heads.packed.nbytes
        return sum(layer.nbytes for layer in self.layers) + heads

    def step_bytes(self, position: int) -> int:
        """Algorithmic HBM bytes of one step at ``position``: packed weights and heads, the
        K/V rows ``0..position`` of every layer, the 33 embedding rows."""
        kv = len(self.layers) * 2 * KH * (position + 1) * HD * 2
        return self.weight_bytes + kv + (CODEBOOKS + 1) * HIDDEN * 2

    # ------------------------------------------------------------ installed model
    @classmethod
    @torch.no_grad()
    def from_model(cls, model, *, max_length: int, w4a8: bool = False) -> "DecodeStepG32":
        """The decode step of a MOSS-TTS model after ``install_gptq``: its quantized projections,
        norm weights and embeddings as they are (no copies); the 32 audio heads (rows ``[:1024]`` of
        ``lm_heads[1:]``) and the gen-slot / delay-slot rows of the text head concatenated into one
        bf16 matrix, as the reference keeps them (``src/moss_tts/_runtime/llm.py:188-191``), applied
        by the bf16 GEMV behind the fused final norm."""
        lm = model.language_model
        layers = []
        for i, layer in enumerate(lm.layers):
            a, m = layer.self_attn, layer.mlp
            if not (isinstance(getattr(a, "qkv_proj", None), QuantLinearG32)
                    and isinstance(getattr(m, "gate_up_proj", None), QuantGateUpG32)):
                raise ValueError(f"layer {i} has no installed quantized projections (run install_gptq first)")
            layers.append(DecoderLayerG32(a.qkv_proj, a.o_proj, m.gate_up_proj, m.down_proj,
                                          layer.input_layernorm.weight, layer.post_attention_layernorm.weight,
                                          a.q_norm.weight, a.k_norm.weight))
        cfg = getattr(model, "config", None)
        lc = getattr(cfg, "language_config", None)
        eps = float(getattr(lc, "rms_norm_eps", 1e-6)) if lc is not None else 1e-6
        theta = getattr(lc, "rope_theta", None) if lc is not None else None
        if theta is None and lc is not None:
            theta = (getattr(lc, "rope_parameters", None) or {}).get("rope_theta")
        cfg_ids = (getattr(cfg, "audio_assistant_gen_slot_token_id", GEN_SLOT_ID),
                   getattr(cfg, "audio_assistant_delay_slot_token_id", DELAY_SLOT_ID))
        text_head = model.lm_heads[0].weight
        if not all(0 <= int(t) < text_head.shape[0] for t in cfg_ids):
            raise ValueError("the gen-slot / delay-slot token ids are outside the text head")
        text_rows = text_head[torch.tensor([int(t) for t in cfg_ids], device=text_head.device)]
        heads = Bf16Linear(torch.cat([h.weight[:SAMPLED_CODES] for h in model.lm_heads[1:]] + [text_rows], 0)
                           .bfloat16().contiguous())
        # the whole text head for the text phase (prefill's text logits and full_step): held as given
        full_text = Bf16Linear(text_head) if text_head.dtype == torch.bfloat16 else None
        audio = torch.stack([e.weight for e in model.emb_ext]).contiguous()
        return cls(layers, lm.norm.weight, heads, lm.embed_tokens.weight.contiguous(), audio,
                   max_length=max_length, eps=eps, theta=float(theta) if theta is not None else 1e6, w4a8=w4a8,
                   audio_stride=SAMPLED_CODES, text_ids=cfg_ids,
                   audio_end_id=getattr(cfg, "audio_end_token_id", AUDIO_END_ID),
                   audio_start_id=getattr(cfg, "audio_start_token_id", AUDIO_START_ID), text_head=full_text)

    # -------------------------------------------------------------- synthetic model
    @classmethod
    @torch.inference_mode()
    def random(cls, n_layers: int, *, max_length: int, device, seed: int = 0, text_vocab: int = 151936,
               kv_fill: bool = True, dequant: int = w4g32.EXACT, w4a8: bool = False, greedy: bool = False,
               sample_seed: int = 0, bf16_heads: bool = False, text_head: bool = False) -> "DecodeStepG32":
        """Random-init Qwen3-8B-shaped weights (N(0, 0.02), min-max INT4-G32 quantized on the
        device), norm weights 1 + N(0, 0.01), embeddings N(0, 1), KV caches N(0, 1).  The heads are
        INT4-G32 (32 x 1025 + 2 rows), or with ``bf16_heads`` bf16 N(0, 0.02) as an installed model
        has them (32 x 1024 + 2 rows).  ``text_head`` adds a bf16 N(0, 0.02) text head of
        ``text_vocab`` rows for the text phase (``prefill_logits``, ``full_step``)."""
        dev = torch.device(device)
        gen = torch.Generator(device=dev).manual_seed(seed)

        def q(n, k, mod=QuantLinearG32):
            w = torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32).mul_(0.02)
            m = mod(w4g32.quantize_minmax(w), dequant=dequant)
            del w
            return m

        def norm(n):
            return (1 + 0.01 * torch.randn(n, generator=gen, device=dev)).bfloat16()

        layers = [DecoderLayerG32(q((QH + 2 * KH) * HD, HIDDEN), q(HIDDEN, QH * HD),
                                  q(2 * INTER, HIDDEN, QuantGateUpG32), q(HIDDEN, INTER),
                                  norm(HIDDEN), norm(HIDDEN), norm(HD), norm(HD)) for _ in range(n_layers)]
        if bf16_heads:
            stride = SAMPLED_CODES
            heads = Bf16Linear((torch.randn((CODEBOOKS * stride + 2, HIDDEN), generator=gen, device=dev) * 0.02)
                               .bfloat16())
        else:
            stride = AUDIO_VOCAB
            heads = q(CODEBOOKS * stride + 2, HIDDEN)  # 32 audio heads of 1025 rows, then the 2 text rows
        text = torch.randn((text_vocab, HIDDEN), generator=gen, device=dev).bfloat16()
        audio = torch.randn((CODEBOOKS, AUDIO_VOCAB, HIDDEN), generator=gen, device=dev).bfloat16()
        full_text = None
        if text_head:
            full_text = Bf16Linear((torch.randn((text_vocab, HIDDEN), generator=gen, device=dev) * 0.02).bfloat16())
        eng = cls(layers, norm(HIDDEN), heads, text, audio, max_length=max_length, w4a8=w4a8, greedy=greedy,
                  seed=sample_seed, audio_stride=stride, text_head=full_text)
        if kv_fill:
            for t in eng.keys + eng.values:
                t.copy_(torch.randn(t.shape, generator=gen, device=dev))
        return eng


class FirstAudioGraph:
    """``steps`` consecutive decode steps in one graph, for the steps right after the audio start
    (``src/moss_tts/_runtime/first_audio_graph.py:32-104``): each step samples its next ids on the
    device and ``advance_step`` turns them into the next step's inputs (position, audio length and
    delay counter as the host loop would, ``streaming.py:107-112``), recording them in ``history``.
    One graph serves every start position (attention work follows the device-side position), so
    there is no capacity list; ``run`` needs ``position + steps <= max_length``.  It shares the
    engine's KV cache and input buffers: it must not overlap another step of the same engine.
    ``warmup`` runs the body once at position 0, writing KV rows ``[0, steps)`` as the reference's
    warm-up does."""

    def __init__(self, engine: DecodeStepG32, steps: int = CODEBOOKS, *, head_prefixes: bool = True):
        _require(isinstance(engine, DecodeStepG32), "engine must be a DecodeStepG32")
        _require(0 < steps <= engine.max_length, "steps must be in [1, max_length]")
        self.engine = engine
        self.steps = int(steps)
        # step s runs with audio length s + 1 at most: the heads beyond the next multiple of 8
        # are masked by the composition and are not computed (first_audio_graph.py:45, llm.py:272)
        self.head_prefixes = bool(head_prefixes)
        dev = engine.device
        self.history = torch.empty((self.steps, CODEBOOKS + 1), device=dev, dtype=torch.int64)
        self.status = torch.empty(4, device=dev, dtype=torch.int64)
        self.graph = None

    def _body(self) -> None:
        e = self.engine
        for step in range(self.steps):
            e.forward(min((step // 8 + 1) * 8, CODEBOOKS) if self.head_prefixes else CODEBOOKS)
            sampling.advance_step(e.next_ids, e.ids.view(-1), e.position, e.audio_length, e.delay_length, step=step,
                                  history=self.history, status=self.status, audio_start_id=e.audio_start_id,
                                  gen_slot_id=e.text_ids_host[0], delay_slot_id=e.text_ids_host[1])

    def _initialize(self, ids: torch.Tensor, position: int, delay: int) -> None:
        e = self.engine
        e.ids.copy_(ids.reshape(1, CODEBOOKS + 1))
        e.position.fill_(position)
        e.audio_length.fill_(1)
        e.delay_length.fill_(delay)

    @torch.inference_mode()
    def warmup(self) -> None:
        if self.graph is not None:
            raise RuntimeError("First-audio graph already captured")
        e = self.engine
        saved = [t.clone() for t in (e.ids, e.position, e.audio_length, e.delay_length)]
        first = torch.full((1, CODEBOOKS + 1), SAMPLED_CODES, device=e.device, dtype=torch.int64)
        first[0, 0] = e.audio_start_id
        try:
            side = torch.cuda.Stream(e.device)
            side.wait_stream(torch.cuda.current_stream(e.device))
            with torch.cuda.stream(side):
                self._initialize(first, 0, -1)
                self._body()
            torch.cuda.current_stream(e.device).wait_stream(side)
            self._initialize(first, 0, -1)
            torch.cuda.synchronize(e.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._body()
            torch.cuda.synchronize(e.device)
            self.graph = graph
        finally:
            for dst, src in zip((e.ids, e.position, e.audio_length, e.delay_length), saved):
                dst.copy_(src)

    @torch.inference_mode()
    def run(self, ids: torch.Tensor, position: int, *, delay: int = -1,
            seed: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """The ``steps`` next-id rows ``[steps, 33]`` and the final (text token, audio length,
        delay, position), both device tensors overwritten by the next run.  ``seed`` sets the
        sampler's key for this run (``None`` keeps the engine's current one)."""
        if self.graph is None:
            raise RuntimeError("Warm the first-audio graph before use")
        e = self.engine
        if not 0 <= position or position + self.steps > e.max_length:
            raise ValueError("Initial interval exceeds captured context capacity")
        if tuple(ids.shape) != (1, 1, CODEBOOKS + 1) or ids.dtype != torch.long or ids.device != e.device:
            raise ValueError("Expected a CUDA int64 audio-start row with all 32 channels")
        if delay not in (-1, 0):
            raise ValueError("Only fresh audio or an immediate-delay validation probe is supported")
        if seed is not None:
            e.seed = seed
        self._initialize(ids, position, delay)
        self.graph.replay()
        return self.history, self.status
