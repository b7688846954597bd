"""The C-ABI boundary without a GPU: ``libmoss_hip.so`` loads, exports every function that
``include/moss_hip.h`` declares, with the parameter count the ctypes binding declares, and
argument errors come back as ``hipErrorInvalidValue`` before anything is launched."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moss_hip.h")


def _declared() -> dict[str, int]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|long long|const char\s*\*)\s*(moss_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    from moss_tts import _build
    from moss_tts._runtime import native

    if not os.path.exists(native.LIB_PATH):
        _build.build()
    return native.lib()


def test_header_declares_the_binding():
    from moss_tts._runtime import native

    decl = _declared()
    assert len(decl) >= 20
    assert set(decl) == set(native.SIGNATURES), set(decl) ^ set(native.SIGNATURES)
    for name, n in decl.items():
        assert len(native.SIGNATURES[name]) == n, f"{name}: header has {n} parameters"


def test_library_exports_every_declared_symbol(lib):
    from moss_tts._runtime import native

    dyn = subprocess.run(["nm", "-D", "--defined-only", native.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in dyn.splitlines() if " T " in ln}
    missing = set(_declared()) - exported
    assert not missing, f"not exported: {sorted(missing)}"
    extra = {s for s in exported if s.startswith("moss_")} - set(_declared())
    assert not extra, f"exported but undeclared: {sorted(extra)}"
    for name in _declared():
        assert callable(getattr(lib, name))


def test_host_only_entry_points(lib):
    assert lib.moss_abi_version() == 1
    ws = lib.moss_gemm_workspace_bytes(64, 4096, 4096)                            # M=64: K split over workgroups
    assert ws > 0 and ws % (64 * 4096 * 4) == 0 and ws // (64 * 4096 * 4) in (2, 4, 8)
    assert lib.moss_gemm_workspace_bytes(512, 4096, 24576) == 0                   # prefill tiles fill the GPU
    # INT4 tiles of 128 tokens: the K split doubles while the workgroups fit one per CU
    assert lib.moss_gemm_workspace_bytes(512, 4096, 6144) == 0                    # 192 tiles: no split
    assert lib.moss_gemm_workspace_bytes(512, 4096, 4096) == 2 * 512 * 4096 * 4   # 128 tiles: K split in 2
    assert lib.moss_gemm_workspace_bytes(512, 12288, 4096) == 2 * 512 * 4096 * 4
    assert lib.moss_gemm_workspace_bytes(128, 12288, 4096) == 8 * 128 * 4096 * 4  # 32 tiles: K split in 8
    # M=16: 32 INT4 tiles of 32 tokens; the split doubles to 16 (512 workgroups) while the partials
    # stay under half the weight bytes
    assert lib.moss_gemm_workspace_bytes(16, 4096, 4096) == 16 * 16 * 4096 * 4
    # every GEMM plan's partial sums fit the allocation-free entry point's 32 MiB scratch array
    worst = max(lib.moss_gemm_workspace_bytes(m, k, n) for m in (1, 2, 5, 16, 33, 64, 65, 128, 200, 256, 300,
                                                                  512, 640, 1000, 1024, 2048, 4096)
                for k in (64, 1024, 4096, 4608, 12288, 16384) for n in (8, 100, 512, 1000, 2048, 4096, 6144,
                                                                         12288, 24576, 32800))
    assert 0 < worst <= 32 << 20
    assert lib.moss_error_string(0)
    assert lib.moss_decode_attention_splits(2048) == 32
    assert lib.moss_decode_attention_splits(128) == 2


def test_argument_errors_are_rejected_before_launch(lib):
    """Null pointers, bad sizes and misalignment return hipErrorInvalidValue (1) on the host;
    no kernel is launched, so this runs without a GPU."""
    null = None
    p = ctypes.c_void_p(4096)
    odd = ctypes.c_void_p(4097)
    assert lib.moss_w4g32_gemv(null, p, p, p, p, 1, 4096, 4096, 0, 0, null) == 1
    assert lib.moss_w4g32_gemv(p, p, p, p, p, 5, 4096, 4096, 0, 0, null) == 1          # M <= 4
    assert lib.moss_w4g32_gemv(p, p, p, p, p, 2, 4096, 4096, 0, 1, null) == 1          # M > 1: exact only
    assert lib.moss_w4g32_gemv(p, p, p, p, p, 2, 6144, 4096, 0, 0, null) == 1          # M > 1: K shape
    assert lib.moss_w4g32_gemv(p, p, p, p, p, 1, 4000, 4096, 0, 0, null) == 1          # K % 64
    assert lib.moss_w4g32_gemv(p, p, p, p, p, 1, 4096, 4096, 3, 0, null) == 1          # rows_per_wave
    assert lib.moss_w4g32_gemv(p, p, p, p, p, 1, 4096, 4096, 0, 7, null) == 1          # dequant mode
    assert lib.moss_w4g32_gemm(odd, p, p, p, p, 64, 4096, 4096, null, 0, null) == 1    # alignment
    assert lib.moss_w4g32_gemm_noalloc(odd, p, p, p, p, 64, 4096, 4096, null) == 1     # alignment
    assert lib.moss_w4g32_gemm_noalloc(p, p, p, p, p, 64, 4000, 4096, null) == 1       # K % 64
    assert lib.moss_fp8_linear(p, p, null, p, 1, 4100, 64, 0, null, 0, null) == 1      # K % 16
    assert lib.moss_fp8_linear(p, p, null, p, 2, 4112, 64, 0, null, 0, null) == 1      # GEMM K % 64
    assert lib.moss_fp8_gateup_silu(p, p, null, p, 2, 4096, 64, 0, null) == 1           # M must be 1
    assert lib.moss_fp8_to_bf16(p, p, 6, null) == 1                                     # count % 4
    assert lib.moss_stream_read(p, 24, p, null) == 1                                     # bytes % 16
    assert lib.moss_stream_read(odd, 32, p, null) == 1                                   # src alignment
    assert lib.moss_stream_read(null, 32, p, null) == 1
    assert lib.moss_stream_read_words(16385) == 8 and lib.moss_stream_read_words(0) == 0
    assert lib.moss_bf16_gemv(p, p, p, 4608, 64, 0, null) == 1                           # K / 512 = 9
    assert lib.moss_bf16_gemv(p, p, p, 4000, 64, 0, null) == 1                           # K % 512
    assert lib.moss_bf16_gemv(p, odd, p, 4096, 64, 0, null) == 1                         # weight alignment
    assert lib.moss_bf16_gemv(p, p, p, 4096, 64, 3, null) == 1                           # rows_per_wave
    assert lib.moss_bf16_norm_gemv(p, null, p, null, ctypes.c_float(1e-6), p, p, 4608, 64, 0, null) == 1  # K
    assert lib.moss_rmsnorm(p, null, p, null, p, 1, 8200, ctypes.c_float(1e-6), null) == 1   # n <= 8192
    assert lib.moss_int8_quantize_g32(p, p, p, p, 40, null) == 1                           # K % 32
    assert lib.moss_rmsnorm_quant_g32(p, null, p, null, null, p, p, p, 1, 4112, ctypes.c_float(1e-6), null) == 1
    assert lib.moss_w4a8_gemv(p, p, p, p, p, p, p, 4128, 64, 0, null) == 1                # K % 64
    assert lib.moss_w4a8_gemv(p, p, p, odd, p, p, p, 4096, 64, 0, null) == 1              # weight alignment
    assert lib.moss_w4a8_quant_gemv(p, p, p, p, p, 4128, 64, 0, null) == 1                 # K % 64
    assert lib.moss_w4a8_quant_gemv(p, p, p, p, p, 16448, 64, 0, null) == 1                # K <= 16384
    assert lib.moss_w4a8_quant_gemv(odd, p, p, p, p, 4096, 64, 0, null) == 1                # x alignment
    assert lib.moss_w4a8_quant_gemv(p, p, p, p, p, 4096, 64, 3, null) == 1                  # rows_per_wave
    assert lib.moss_w4a8_gateup_silu(p, p, p, p, p, p, p, p, null, p, 4096, 64, 0, null) == 1   # partial outputs
    assert lib.moss_w4a8_gateup_silu(p, p, p, p, p, p, p, p, p, p, 4096, 48, 0, null) == 1      # N_half % 32
    assert lib.moss_w4a8_gateup_silu(p, p, p, p, p, p, p, p, p, p, 4096, 64, 1, null) == 1      # fused rows 2|4
    f = ctypes.c_float
    assert lib.moss_sample_topk(p, 32, 1025, 1024, f(1.7), 0, f(0.8), p, p, 0, p, null) == 1      # top_k >= 1
    assert lib.moss_sample_topk(p, 32, 1025, 1024, f(1.7), 65, f(0.8), p, p, 0, p, null) == 1     # top_k <= 64
    assert lib.moss_sample_topk(p, 1, 4096, 4096, f(0.0), 1, f(0.8), p, p, 0, p, null) == 1      # vocab <= 2048
    assert lib.moss_sample_topk(p, 1, 100, 200, f(0.0), 1, f(0.8), p, p, 0, p, null) == 1        # stride >= vocab
    assert lib.moss_sample_topk(p, 1, 100, 100, f(1.0), 1, f(0.8), null, p, 0, p, null) == 1     # seed buffer
    assert lib.moss_sample_topk(p, 1, 100, 100, f(1.0), 1, f(0.8), ctypes.c_void_p(4100), p, 0, p,
                                null) == 1                                                        # seed alignment
    pair_ok = (p, 1, 2, 2, f(1.5), 2, f(1.0), 1, p, p, 32, 1025, 1024, f(1.7), 25, f(0.8), 0, p)
    bad_vocab = pair_ok[:10] + (32, 4096, 4096) + pair_ok[13:]
    assert lib.moss_sample_topk_pair(*bad_vocab, p, p, null) == 1                                 # vocab <= 2048
    bad_k = pair_ok[:5] + (3,) + pair_ok[6:]
    assert lib.moss_sample_topk_pair(*bad_k, p, p, null) == 1                                     # top_k <= vocab
    assert lib.moss_sample_topk_pair(*pair_ok, null, p, null) == 1                                # seed buffer
    assert lib.moss_compose_next_ids(p, p, p, p, p, 0, 0, 0, 1024, p, null) == 1                  # channels
    # the prefill fusions (every call below is refused before any launch)
    assert lib.moss_w4g32_gemm_silu(p, p, p, p, p, 512, 4096, 12290, null, 0, null) == 1          # N % 4
    assert lib.moss_w4g32_gemm_silu(odd, p, p, p, p, 512, 4096, 12288, null, 0, null) == 1        # alignment
    assert lib.moss_w4g32_gemm_silu(p, p, p, p, p, 16, 4096, 12288, null, 0, null) == 1           # unfused: workspace
    assert lib.moss_gemm_silu_workspace_bytes(512, 4096, 12288) == 512 * 2 * 12288 * 2             # upper bound: product
    assert lib.moss_gemm_silu_workspace_bytes(16, 4096, 12288) >= 16 * 2 * 12288 * 2               # [M, 2N] product
    qr = (p, p, p, p, p, p, p, p, p, p, p, p)
    assert lib.moss_w4g32_gemm_qk_rope(*qr[:4], null, *qr[5:], 512, 4096, 1024, f(1e-6), null, 0, null) == 1  # null
    assert lib.moss_w4g32_gemm_qk_rope(*qr, 512, 4000, 1024, f(1e-6), null, 0, null) == 1              # K % 64
    assert lib.moss_w4g32_gemm_qk_rope(*qr, 512, 4096, 1024, f(-1.0), null, 0, null) == 1              # eps
    assert lib.moss_w4g32_gemm_qk_rope(odd, *qr[1:], 512, 4096, 1024, f(1e-6), null, 0, null) == 1     # alignment
    assert lib.moss_w4g32_gemm_qk_rope(*qr, 128, 4096, 1024, f(1e-6), null, 0, null) == 1              # unfused: workspace
    assert lib.moss_gemm_qk_rope_workspace_bytes(512, 4096) == 512 * 6144 * 2                             # upper bound: product
    assert lib.moss_gemm_qk_rope_workspace_bytes(128, 4096) >= 128 * 6144 * 2 + 2 * 128 * 6144 * 4        # product + split
    assert lib.moss_w4g32_gemm_add_rmsnorm(p, p, p, p, p, p, f(1e-6), p, p, 512, 4096, 4100, null, 0,
                                           null) == 1                                              # N % 8
    assert lib.moss_w4g32_gemm_add_rmsnorm(p, p, p, p, p, p, f(1e-6), p, p, 512, 4096, 8200, null, 0,
                                           null) == 1                                              # N <= 8192
    assert lib.moss_w4g32_gemm_add_rmsnorm(p, p, p, p, odd, p, f(1e-6), p, p, 512, 4096, 4096, null, 0,
                                           null) == 1                                              # residual alignment
    q = ctypes.c_void_p(8192)
    assert lib.moss_w4a8_norm_gemv(p, null, p, null, f(1e-6), p, p, p, p, 12288, 64, 0, null) == 1   # K
    assert lib.moss_w4a8_norm_gemv(p, p, p, null, f(1e-6), p, p, p, p, 4096, 64, 0, null) == 1       # sum_out
    assert lib.moss_w4a8_norm_gateup_silu(p, null, p, null, f(1e-6), p, p, p, p, 4096, 64, 3, null) == 1  # rows
    # sum_out overlapping x or res (an in-place residual update) races with the other workgroups
    x0, r0 = ctypes.c_void_p(1 << 20), ctypes.c_void_p(2 << 20)
    for norm in (lib.moss_w4a8_norm_gemv, lib.moss_w4a8_norm_gateup_silu, lib.moss_w4g32_norm_gemv,
                 lib.moss_w4g32_norm_gateup_silu):
        extra = (0,) if norm in (lib.moss_w4g32_norm_gemv, lib.moss_w4g32_norm_gateup_silu) else ()
        assert norm(x0, r0, p, r0, f(1e-6), p, p, p, p, 4096, 64, 0, *extra, null) == 1         # sum_out == res
        assert norm(x0, r0, p, ctypes.c_void_p((1 << 20) + 4096), f(1e-6), p, p, p, p, 4096, 64, 0, *extra,
                    null) == 1                                                                    # overlaps x
        assert norm(x0, null, p, q, f(1e-6), p, p, p, p, 4096, 64, 0, *extra, null) == 1        # res NULL
    assert lib.moss_decode_attention_qkv_quant(p, p, p, p, p, p, p, p, p, p, p, null, p, p, 2048, f(1e-6),
                                               null) == 1                                         # out_qx
    assert lib.moss_decode_attention_qkv_quant(p, p, p, p, p, p, p, p, p, p, p, p, p, p, 2000, f(1e-6),
                                               null) == 1                                         # L % 64
    assert lib.moss_advance_step(p, p, q, q, q, null, null, 0, 33, 1, 2, 3, null) == 1             # next_ids == ids
    assert lib.moss_advance_step(p, q, q, q, q, null, null, 0, 65, 1, 2, 3, null) == 1             # width <= 64
    assert lib.moss_advance_step(p, q, q, q, q, null, null, -1, 33, 1, 2, 3, null) == 1            # step >= 0
    assert lib.moss_advance_step(p, q, null, q, q, null, null, 0, 33, 1, 2, 3, null) == 1          # position
