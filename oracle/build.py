"""Compile the CPU restatement (oracle/oa_oracle.c) into oracle/_build/liboa_oracle.so.

Test infrastructure only: the library is loaded by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker, never by the product path.

gcc flags: -O2 -ffp-contract=off (no implicit fused multiply-adds: the restatement replays the
device's arithmetic order, and every fma it performs is an explicit fma()/fmaf() call) and no
-march, so float/double arithmetic is plain IEEE SSE2.

The reference itself (/root/reference) is Python + Triton: there is no C/C++ source to build
into oracle/_ref, so this file builds only the restatement.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(OUT, "liboa_oracle.so")
SRC = os.path.join(HERE, "oa_oracle.c")
CFLAGS = ["-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
          "-Wall", "-Wextra", "-Wno-unused-parameter"]


def build(verbose: bool = False) -> str:
    os.makedirs(OUT, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = ["gcc", *CFLAGS, SRC, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
