"""Build recipe for the native libraries of xlog_amd.

    python xlog_amd/_build.py         # builds libxlog_hip.so and libxlog_datagen.so in-tree

libxlog_hip.so   : the gfx950 HIP kernels + C ABI (include/xlog_hip.h), hipcc.
libxlog_datagen.so: host-only seeded input generators (plain C, gcc).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build" / "xlog_amd"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_SOURCES = ["sort.hip", "select.hip", "join.hip", "tc_bitmap.hip", "chain_bitmap.hip", "hash_set.hip", "arrow_ipc.cpp",
               "abi.hip", "fixpoint.hip"]
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-munsafe-fp-atomics",
    # no packed-FP32 instruction forms in any code object
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]

LIB_HIP = PKG / "libxlog_hip.so"
LIB_DATAGEN = PKG / "libxlog_datagen.so"


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}")
    out = r.stdout.strip()
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected
    lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l and "not a recognized feature" not in l]
    if lines:
        print("\n".join(lines), file=sys.stderr)


def build_datagen() -> Path:
    tmp = LIB_DATAGEN.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-fPIC", "-shared", "-Wall", "-o", str(tmp), str(CSRC / "datagen.c"), "-lm"])
    os.replace(tmp, LIB_DATAGEN)
    return LIB_DATAGEN


def build_hip(jobs: int = 8) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)

    def compile_one(src: str) -> Path:
        obj = BUILD / (src.rsplit(".", 1)[0] + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(HIP_SOURCES)))) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    tmp = LIB_HIP.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_HIP)
    return LIB_HIP


def build(jobs: int = 8) -> None:
    build_datagen()
    build_hip(jobs)


if __name__ == "__main__":
    build()
    print(f"built {LIB_HIP} and {LIB_DATAGEN}")
