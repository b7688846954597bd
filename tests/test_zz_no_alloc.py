"""GPU: the allocation-free INT4 GEMM entry point (``moss_w4g32_gemm_noalloc``) against the GEMM with
a caller workspace (``moss_w4g32_gemm``), through the C-ABI.

Both take the same plan (the scratch array holds every plan's partials), so the outputs must be equal
bit for bit.  Two K-split calls in a row, the second smaller (4 MiB of partials against the first's
16 MiB, written over the first call's), show that the scratch contents left by one call do not leak
into the next; a shape with no K split runs too, and the Python wrapper gives the same result into a
caller-owned output."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20


def _fn():
    from moss_tts._runtime import native

    return native.lib().moss_w4g32_gemm_noalloc


def test_gemm_noalloc_matches_workspace_entry(dev):
    from moss_tts._runtime import native, w4g32

    fn = _fn()
    g = torch.Generator(device=dev).manual_seed(31)
    for (m, k, n), split in (((512, 12288, 4096), True), ((64, 4096, 4096), True), ((512, 4096, 24576), False)):
        print(f"gemm noalloc M={m} K={k} N={n}", flush=True)
        need = native.lib().moss_gemm_workspace_bytes(m, k, n)
        assert need <= SCRATCH and (need > 0) == split
        pw = w4g32.quantize_minmax((torch.randn((n, k), device=dev, generator=g) * 0.02).contiguous())
        x = torch.randn((m, k), device=dev, generator=g).bfloat16()
        ref = w4g32.gemm(x, pw)
        y = torch.full_like(ref, float("nan"))
        rc = fn(native.ptr(x), native.ptr(pw.qw), native.ptr(pw.scales), native.ptr(pw.zeros), native.ptr(y), m, k, n,
                native.stream_of(x))
        torch.cuda.synchronize()
        assert rc == 0, native.error_string(rc)
        assert torch.equal(y, ref), f"M={m} K={k} N={n} (workspace plan {need} B)"
        out = torch.empty_like(ref)
        assert torch.equal(w4g32.gemm_noalloc(x, pw, out), ref)


def test_gemm_noalloc_rejects_bad_arguments(dev):
    from moss_tts._runtime import native

    fn = _fn()
    p = ctypes.c_void_p(4096)
    assert fn(None, p, p, p, p, 64, 4096, 4096, None) == 1
    assert fn(p, p, p, p, p, 64, 4000, 4096, None) == 1                      # K % 64
    assert fn(ctypes.c_void_p(4097), p, p, p, p, 64, 4096, 4096, None) == 1  # alignment
