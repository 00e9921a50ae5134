"""Builds the CPU oracle (test infrastructure only) into oracle/liboracle_attn.so with gcc.

The reference implementation itself (csrc/*.cpp) is not built: it includes ggml headers
(csrc/gt_internal.h:4-8) from a llama.cpp checkout that its build downloads, which this
environment does not have, so oracle/_ref/ stays empty.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "oracle_attn.c"
LIB = HERE / "liboracle_attn.so"

# x86-64-v3 (AVX2/FMA) instead of -march=native: the library is built here and run on another
# host; -fopenmp as the reference build (build_native.py:564-575).
CFLAGS = ["-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-std=c11", "-Wall"]


def build() -> Path:
    cc = os.environ.get("CC", "gcc")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, *CFLAGS, str(SRC), "-o", str(tmp), "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
