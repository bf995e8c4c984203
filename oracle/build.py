"""Build the oracle's C restatement (TEST INFRASTRUCTURE ONLY).

``oracle/attn_ref.c`` -> ``oracle/_build/liboracle_ref.so`` with gcc and
OpenMP. x86-64-v3 (AVX2 + FMA) keeps the binary portable to the GPU boxes'
host CPUs.

The reference itself (Rust on candle 0.11.1) cannot be compiled here: there
is no Rust toolchain and candle is not vendored, so there is no
``oracle/_ref`` build.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "liboracle_ref.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared",
           "-std=c11", "-Wall", str(HERE / "attn_ref.c"), "-o", str(tmp), "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
