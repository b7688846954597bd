"""ctypes binding of ``libmoss_hip.so`` (the gfx950 C-ABI declared in ``include/moss_hip.h``).

Mirrors the reference's native convention (``src/moss_tts/_runtime/attention_native.py:11-44``):
the library is loaded once (``functools.lru_cache``), ``argtypes``/``restype`` are declared,
and a nonzero ``hipError_t`` raises ``RuntimeError``.  There is no fallback: a missing or
unloadable library is an error.

``torch`` is imported before the library so that its ``libamdhip64.so.7`` (same SONAME) is
the HIP runtime the library binds to; streams and pointers are then shared with torch.
"""
from __future__ import annotations

import ctypes
import functools
import os

import torch  # noqa: F401  (must load torch's HIP runtime first)

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_lib", "libmoss_hip.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes; every function returns int (hipError_t) unless listed in _RESTYPES.
SIGNATURES: dict[str, list] = {
    "moss_abi_version": [],
    "moss_error_string": [_I],
    "moss_check_device": [ctypes.c_char_p, _I],
    "moss_w4g32_repack_gptq": [_P, _P, _P, _P, _P, _P, _I, _I, _P],
    "moss_w4g32_import_signed": [_P, _P, _P, _I, _I, _P],
    "moss_w4g32_unpack_codes": [_P, _P, _I, _I, _P],
    "moss_w4g32_dequant_bf16": [_P, _P, _P, _P, _I, _I, _P],
    "moss_w4g32_quantize_minmax": [_P, _P, _P, _P, _I, _I, _P],
    "moss_w4g32_quantize_symmetric": [_P, _P, _P, _P, _I, _I, _P],
    "moss_w4g32_gemv": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "moss_w4g32_gateup_silu": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "moss_w4g32_gemm": [_P, _P, _P, _P, _P, _I, _I, _I, _P, ctypes.c_longlong, _P],
    "moss_gemm_workspace_bytes": [_I, _I, _I],
    "moss_w4g32_gemm_silu": [_P, _P, _P, _P, _P, _I, _I, _I, _P, ctypes.c_longlong, _P],
    "moss_gemm_silu_workspace_bytes": [_I, _I, _I],
    "moss_w4g32_gemm_qk_rope": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P,
                                ctypes.c_longlong, _P],
    "moss_gemm_qk_rope_workspace_bytes": [_I, _I],
    "moss_w4g32_gemm_add_rmsnorm": [_P, _P, _P, _P, _P, _P, _F, _P, _P, _I, _I, _I, _P, ctypes.c_longlong, _P],
    "moss_w4g32_gemm_noalloc": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "moss_w4g32_norm_gemv": [_P, _P, _P, _P, _F, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "moss_w4g32_norm_gateup_silu": [_P, _P, _P, _P, _F, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "moss_bf16_gemv": [_P, _P, _P, _I, _I, _I, _P],
    "moss_bf16_norm_gemv": [_P, _P, _P, _P, _F, _P, _P, _I, _I, _I, _P],
    "moss_rmsnorm": [_P, _P, _P, _P, _P, _I, _I, _F, _P],
    "moss_qk_norm_rope_kv": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _I, _P],
    "moss_silu_mul": [_P, _P, _I, _I, _P],
    "moss_decode_attention_splits": [_I],
    "moss_decode_attention": [_P, _P, _P, _P, _P, _P, _P, _I, _P],
    "moss_decode_attention_qkv": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _F, _P],
    "moss_decode_attention_qkv_quant": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _F, _P],
    "moss_embedding_sum": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "moss_prefill_attention": [_P, _P, _P, _P, _P, _I, _I, _P],
    "moss_fp8_linear": [_P, _P, _P, _P, _I, _I, _I, _I, _P, ctypes.c_longlong, _P],
    "moss_fp8_gateup_silu": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "moss_fp8_to_bf16": [_P, _P, ctypes.c_longlong, _P],
    "moss_int8_quantize_g32": [_P, _P, _P, _P, _I, _P],
    "moss_rmsnorm_quant_g32": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _P],
    "moss_w4a8_gemv": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "moss_w4a8_quant_gemv": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "moss_w4a8_gateup_silu": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "moss_w4a8_norm_gemv": [_P, _P, _P, _P, _F, _P, _P, _P, _P, _I, _I, _I, _P],
    "moss_w4a8_norm_gateup_silu": [_P, _P, _P, _P, _F, _P, _P, _P, _P, _I, _I, _I, _P],
    "moss_sample_topk": [_P, _I, _I, _I, _F, _I, _F, _P, _P, _I, _P, _P],
    "moss_sample_topk_pair": [_P, _I, _I, _I, _F, _I, _F, _I, _P, _P, _I, _I, _I, _F, _I, _F, _I, _P, _P, _P, _P],
    "moss_compose_next_ids": [_P, _P, _P, _P, _P, ctypes.c_longlong, ctypes.c_longlong, _I, ctypes.c_longlong, _P, _P],
    "moss_advance_step": [_P, _P, _P, _P, _P, _P, _P, _I, _I, ctypes.c_longlong, ctypes.c_longlong, ctypes.c_longlong,
                          _P],
    "moss_stream_read_words": [ctypes.c_longlong],
    "moss_stream_read": [_P, ctypes.c_longlong, _P, _P],
}
_RESTYPES = {"moss_error_string": ctypes.c_char_p, "moss_gemm_workspace_bytes": ctypes.c_longlong,
             "moss_gemm_silu_workspace_bytes": ctypes.c_longlong,
             "moss_gemm_qk_rope_workspace_bytes": ctypes.c_longlong,
             "moss_stream_read_words": ctypes.c_longlong}


class NativeLibraryMissing(RuntimeError):
    pass


@functools.lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryMissing(
            f"{LIB_PATH} is not built; build it with moss_tts._build.build() (hipcc, gfx950)")
    so = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
    for name, args in SIGNATURES.items():
        fn = getattr(so, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, _I)
    return so


def error_string(code: int) -> str:
    s = lib().moss_error_string(int(code))
    return s.decode() if s else f"hipError {code}"


def check(code: int, what: str) -> None:
    if code:
        raise RuntimeError(f"{what} failed: {error_string(code)} (hipError {code})")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def gemm_workspace(m: int, k: int, n: int, device) -> tuple:
    """(pointer, bytes, tensor) of a fresh fp32 workspace for an M x K x N GEMM, or (None, 0, None)
    when the GEMM needs none; the caller keeps the tensor alive until the launch has run."""
    nbytes = int(lib().moss_gemm_workspace_bytes(int(m), int(k), int(n)))
    if nbytes == 0:
        return None, 0, None
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=device)
    return ctypes.c_void_p(ws.data_ptr()), nbytes, ws


def workspace(nbytes: int, device) -> tuple:
    """(pointer, bytes, tensor) of a fresh 16-byte aligned device buffer of ``nbytes``, or
    (None, 0, None) for none; the caller keeps the tensor alive until the launch has run."""
    if nbytes == 0:
        return None, 0, None
    ws = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)
    return ctypes.c_void_p(ws.data_ptr()), int(nbytes), ws


def stream_of(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


@functools.lru_cache(maxsize=None)
def device_arch(index: int) -> str:
    """gcnArchName of a device; raises unless it is gfx950."""
    with torch.cuda.device(index):
        buf = ctypes.create_string_buffer(64)
        rc = lib().moss_check_device(buf, 64)
    arch = buf.value.decode()
    if rc:
        raise RuntimeError(f"libmoss_hip.so targets gfx950 (MI350/MI355); device {index} is {arch or 'unknown'}"
                           f" ({error_string(rc)})")
    return arch
