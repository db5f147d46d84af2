"""Build the CPU oracle (test infrastructure only) with gcc.

-ffp-contract=off and no fast-math keep every fp32 operation in ks_oracle.c a
single IEEE-754 operation, which the bit-exact parity checks rely on.

The reference implementation itself (cklxx/kernel-set, CUDA sources needing
nvcc, <cuda_fp8.h> and a CMake build) cannot be compiled in this image, so no
oracle/_ref build exists; see DESIGN.md.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "ks_oracle.c")
LIB = os.path.join(HERE, "libks_oracle.so")


def build() -> str:
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-std=c11",
           "-shared", "-fPIC", "-o", tmp, SRC, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
