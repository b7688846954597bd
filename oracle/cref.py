"""ctypes binding of the oracle's C restatement (TEST INFRASTRUCTURE ONLY)."""
from __future__ import annotations

import ctypes
import functools
import os

import numpy as np
import torch

from . import build as _build

_P = ctypes.c_void_p
_I = ctypes.c_int


@functools.lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not os.path.exists(_build.LIB):
        _build.build()
    so = ctypes.CDLL(_build.LIB)
    so.oracle_bf16_rne.argtypes = [_P, _P, ctypes.c_size_t]
    so.oracle_unpack_gptq.argtypes = [_P, _I, _I, _P]
    so.oracle_unpack_gptq_zeros.argtypes = [_P, _I, _I, _P]
    so.oracle_dequant.argtypes = [_P, _P, _P, _I, _I, _P]
    so.oracle_unpack_signed.argtypes = [_P, _I, _I, _P]
    so.oracle_rowpack.argtypes = [_P, _P, _I, _I, _P, _P]
    so.oracle_linear_f64.argtypes = [_P, _P, _I, _I, _I, _P]
    for f in ("oracle_bf16_rne", "oracle_unpack_gptq", "oracle_unpack_gptq_zeros", "oracle_dequant",
              "oracle_unpack_signed", "oracle_rowpack", "oracle_linear_f64"):
        getattr(so, f).restype = None
    return so


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.contiguous().view(torch.int16).numpy().view(np.uint16))


def bf16_rne(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_bf16_rne(_ptr(a), _ptr(out), a.size)
    return out


def unpack_gptq(qweight: torch.Tensor, qzeros: torch.Tensor):
    qw = np.ascontiguousarray(qweight.numpy().view(np.uint32))
    qz = np.ascontiguousarray(qzeros.numpy().view(np.uint32))
    k8, n = qw.shape
    q = np.empty((n, k8 * 8), dtype=np.uint8)
    z = np.empty((n, qz.shape[0]), dtype=np.uint8)
    lib().oracle_unpack_gptq(_ptr(qw), k8 * 8, n, _ptr(q))
    lib().oracle_unpack_gptq_zeros(_ptr(qz), qz.shape[0], n, _ptr(z))
    return torch.from_numpy(q), torch.from_numpy(z)


def dequant(q: torch.Tensor, z: torch.Tensor, s: torch.Tensor) -> np.ndarray:
    qn = np.ascontiguousarray(q.numpy(), dtype=np.uint8)
    zn = np.ascontiguousarray(z.numpy(), dtype=np.uint8)
    sn = _u16(s)
    n, k = qn.shape
    w = np.empty((n, k), dtype=np.uint16)
    lib().oracle_dequant(_ptr(qn), _ptr(zn), _ptr(sn), n, k, _ptr(w))
    return w


def unpack_signed(packed: torch.Tensor) -> torch.Tensor:
    p = np.ascontiguousarray(packed.numpy(), dtype=np.uint8)
    n, k2 = p.shape
    c = np.empty((n, 2 * k2), dtype=np.int8)
    lib().oracle_unpack_signed(_ptr(p), n, 2 * k2, _ptr(c))
    return torch.from_numpy(c)


def rowpack(q: torch.Tensor, z: torch.Tensor):
    qn = np.ascontiguousarray(q.numpy(), dtype=np.uint8)
    zn = np.ascontiguousarray(z.numpy(), dtype=np.uint8)
    n, k = qn.shape
    qw = np.empty((n, k // 8), dtype=np.uint32)
    zp = np.empty((n, k // 64), dtype=np.uint8)
    lib().oracle_rowpack(_ptr(qn), _ptr(zn), n, k, _ptr(qw), _ptr(zp))
    return qw, zp


def linear_f64(x_bf16: torch.Tensor, w_bf16: torch.Tensor) -> np.ndarray:
    xn = _u16(x_bf16)
    wn = _u16(w_bf16)
    m, k = xn.shape
    n = wn.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    lib().oracle_linear_f64(_ptr(xn), _ptr(wn), m, n, k, _ptr(y))
    return y
