"""The 128-token INT4 GEMM tile copies activations from global memory into LDS with
global_load_lds_dwordx4 and waits for those copies with explicit vmcnt counts before each barrier
(the compiler only orders a copy before this wave's own reads of it).  Those counts hold only if
the generated code issues exactly the loads they count after each copy.  This test compiles
csrc/w4g32_gemm.hip for gfx950 with the library's flags and checks, in the generated assembly of
every w4g32_gemm_tdma_kernel instance, that no s_barrier and no s_endpgm is reached while a copy
of this wave may still be in flight: after the last copy, some s_waitcnt must have a vmcnt no
larger than the number of vector-memory instructions issued after that copy.
"""
import os
import re
import shutil
import subprocess

import pytest

from moss_tts import _build

# loads only: vector-memory loads complete in order, so a wait that leaves at most N ops
# outstanding, N = the loads issued after a copy, implies the copy has landed; a store issued after
# it may complete first and must not be counted
_VMEM_LOAD = re.compile(r"^(global_load|buffer_load|scratch_load|flat_load)")


def _device_asm(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    src = os.path.join(_build.CSRC, "w4g32_gemm.hip")
    out = tmp_path / "w4g32_gemm.s"
    flags = [f for f in _build.CFLAGS if f not in ("-fPIC", "-fvisibility=hidden")]
    r = subprocess.run([hipcc, *flags, "-I", _build.CSRC, "-S", "--cuda-device-only", src, "-o", str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text().split("\n")


def _kernel_bodies(lines, needle):
    bodies = {}
    for i, line in enumerate(lines):
        if line.startswith("_Z") and needle in line.split(":")[0] and ":" in line:
            body = []
            for ln in lines[i + 1:]:
                t = ln.strip()
                body.append(t)
                if t.startswith("s_endpgm"):
                    break
            bodies[line.split(":")[0]] = body
    return bodies


def check_copy_waits(body):
    """Returns the number of barriers checked; raises AssertionError on a barrier (or the end)
    that a copy of this wave may still be in flight for.  Straight-line scan: the kernel's loop
    bodies are unrolled and every step ends at a barrier."""
    pending = None  # vector-memory loads issued since the last uncovered copy
    barriers = 0
    for k, t in enumerate(body):
        if t.startswith("global_load_lds"):
            pending = 0
        elif _VMEM_LOAD.match(t):
            if pending is not None:
                pending += 1
        elif t.startswith("s_waitcnt") and "vmcnt" in t:
            n = int(re.search(r"vmcnt\((\d+)\)", t).group(1))
            if pending is not None and n <= pending:
                pending = None
        elif t.startswith("s_barrier") or t.startswith("s_endpgm"):
            assert pending is None, f"line {k}: {t} with a copy in flight ({pending} loads after it)"
            barriers += t.startswith("s_barrier")
    return barriers


def test_check_rejects_a_lax_wait():
    """The checker itself: a wait that leaves the copy outstanding is caught."""
    body = ["global_load_lds_dwordx4 v[0:1], off", "global_load_dwordx4 v[2:5], v[6:7], off",
            "s_waitcnt vmcnt(2)", "s_barrier", "s_endpgm"]
    with pytest.raises(AssertionError):
        check_copy_waits(body)
    body[2] = "s_waitcnt vmcnt(1)"
    assert check_copy_waits(body) == 1
    # a store after the copy does not count: vmcnt(1) could pass with the copy still in flight
    body = ["global_load_lds_dwordx4 v[0:1], off", "scratch_store_dword off, v9, off", "s_waitcnt vmcnt(1)",
            "s_barrier", "s_endpgm"]
    with pytest.raises(AssertionError):
        check_copy_waits(body)


def test_copy_tile_waits_cover_every_copy(tmp_path):
    bodies = _kernel_bodies(_device_asm(tmp_path), "w4g32_gemm_tdma_kernel")
    assert len(bodies) == 4, sorted(bodies)  # split, unsplit, unsplit with the SiLU or the q/k-norm + RoPE epilogue
    for name, body in bodies.items():
        assert any(t.startswith("global_load_lds_dwordx4") for t in body), name
        # prologue + 8 steps of the paired-block loop + 4 steps of the last block
        assert check_copy_waits(body) >= 13, name
