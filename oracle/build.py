"""TEST INFRASTRUCTURE: build recipe for the parity oracle (oracle/xt_oracle.c).

Produces oracle/lib/libxt_oracle.so (gcc, OpenMP, no fast-math, FP contraction
off so f32 ops round exactly as written).

The reference itself (sjjeong94/xtile) cannot be compiled here: its C++
needs MLIR/LLVM 20.1.8, TableGen and nanobind, none of which are in the image,
and it computes no numbers anyway.  So there is no oracle/_ref build.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "lib" / "libxt_oracle.so"


def build() -> Path:
    LIB.parent.mkdir(parents=True, exist_ok=True)
    cc = shutil.which("gcc") or "gcc"
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [
        cc,
        "-O3",
        "-march=x86-64-v3",
        "-fopenmp",
        "-ffp-contract=off",
        "-fno-fast-math",
        "-fPIC",
        "-shared",
        "-Wall",
        str(HERE / "xt_oracle.c"),
        "-lm",
        "-o",
        str(tmp),
    ]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
