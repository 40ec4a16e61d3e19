"""Build the oracle (test infrastructure) with gcc.

Produces oracle/_build/libneedle_oracle.so from needle_oracle.c,
cpu_baseline.c, cpu_simd.c, decoder.c and needle3_model.c.  Flags keep every float operation an IEEE binary32 operation
in source order (-ffp-contract=off, no -ffast-math); -O2 -mavx2 only lets gcc
vectorise the integer group dots and the row loops.  cpu_simd.c's SIMD tier
(the timed baseline) takes its AVX2 / AVX-VNNI instructions from function
target attributes and is picked at run time from CPUID.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(OUT, "libneedle_oracle.so")
SOURCES = ["needle_oracle.c", "cpu_baseline.c", "cpu_simd.c", "decoder.c", "needle3_model.c"]
FLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-mavx2",
         "-Wall", "-Wextra", "-pthread", "-fopenmp"]


def build() -> str:
    os.makedirs(OUT, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = ["gcc", *FLAGS, *[os.path.join(HERE, s) for s in SOURCES], "-o", tmp, "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(), file=sys.stdout)
