"""Build recipe for the oracle's C restatement (TEST INFRASTRUCTURE ONLY).

``python oracle/build.py`` compiles ``oracle/w4g32_ref.c`` with gcc into
``oracle/_build/liboracle_w4g32.so``.  The reference itself is Python/Triton plus
nvcc-only CUDA, so there is no ``oracle/_ref`` build of it.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "liboracle_w4g32.so")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    src = os.path.join(HERE, "w4g32_ref.c")
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-fno-fast-math", "-ffp-contract=off",
           src, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
