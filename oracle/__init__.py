"""CPU oracle for the INT4-G32 quantized-linear path (TEST INFRASTRUCTURE ONLY).

This package restates, on the CPU, the reference algorithms that the HIP kernels in
``moss-tts-optimized_amd/csrc`` must reproduce.  It is what the kernels are
checked against, never the thing measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  Product code never imports it and
has no CPU fallback.

Modules
-------
``w4g32``      nibble formats, quantizers, bf16 dequant, dequant-then-matmul
               (reference: ``src/moss_tts/calibration.py:184-203``,
               ``src/moss_tts/_runtime/calibrated_quant.py:36-42``,
               ``src/moss_tts/_runtime/calibrated_backend.py:8-13``,
               ``src/moss_tts/_runtime/dp4a_packing.py:15-27``)
``pointwise``  RMSNorm / add-RMSNorm, SiLU*mul, q/k head-norm + RoPE + KV write
               (reference: ``src/moss_tts/_runtime/kernels.py:50-170``,
               ``src/moss_tts/_runtime/prefill_qkv.py:7-28``,
               ``src/moss_tts/_runtime/dp4a_scaled.py:65-68``)
``fp8``        OCP e4m3 weight-only linear (``src/moss_tts/_runtime/fused_mlp.py:7-23``)
``attention``  split-K GQA decode attention (``src/moss_tts/_runtime/kernels.py:173-208``)
               and the 33-row embedding sum (``src/moss_tts/_runtime/kernels.py:7-26``)
``decode``     one batch-1 decode step composed from the above
               (``src/moss_tts/_runtime/llm.py:227-279``)
``cref``       ctypes binding of ``oracle/w4g32_ref.c`` (an independent C restatement
               of the byte/integer work, used to cross-check the numpy restatement).

How each function is pinned (no reference golden vectors exist for this path) is
written in the docstring of its test in ``tests/test_oracle*.py``.
"""
