"""Build oracle/lib/liboracle.so from oracle/csrc/oracle.c (gcc, OpenMP, AVX2+F16C).

    python -m oracle.build

The reference itself (Metal shaders + a Swift host) cannot be compiled here:
there is no Metal toolchain or swiftc, so there is no oracle/_ref build.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "csrc" / "oracle.c"
LIB = HERE / "lib" / "liboracle.so"
FLAGS = ["-O3", "-fPIC", "-shared", "-fopenmp", "-mavx2", "-mfma", "-mf16c", "-std=c11", "-Wall", "-Wno-unused-function"]


def build() -> Path:
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    res = subprocess.run(["gcc", *FLAGS, str(SRC), "-o", str(tmp), "-lm"], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed\n{res.stdout}{res.stderr}")
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    print(build())
    sys.exit(0)
