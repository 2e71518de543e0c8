"""Build recipe of the CPU oracle (plain C, gcc): oracle/liboracle.so.

The reference itself (Rust + CUDA) cannot be compiled in this image (no cargo,
rustc or nvcc), so there is no oracle/_ref build."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

DIR = Path(__file__).resolve().parent
LIB = DIR / "liboracle.so"


def build() -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter", "-o", str(tmp),
           str(DIR / "oracle.c")]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
