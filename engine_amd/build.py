"""Builds engine_amd/libribn_amd.so (HIP kernels + C ABI) for gfx950 with hipcc.

    python -m engine_amd.build

Compiles every translation unit under engine_amd/csrc in parallel and links one
shared library in-tree, next to this file, so it travels with the repository.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libribn_amd.so")
ARCH = os.environ.get("RIBN_AMD_ARCH", "gfx950")

# Packed-FP32 instructions are disabled for all device code on this platform.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Products and sums round separately unless a kernel asks for an FMA
    # (__builtin_fmaf): keeps the exact-order kernels bit-identical to the host.
    "-ffp-contract=off",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Wall", "-Wno-unused-function",
]

SOURCES = ["kquant_kernels.hip", "gemv_wave.hip", "gemv_f32.hip", "gemv_mfma.hip", "gemv_f32mma.hip", "q8_1.hip", "qgemm.hip", "decode_kernels.hip", "ribn_amd.cpp", "qwen3_decode.cpp", "gguf.cpp", "serving.cpp"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build engine_amd")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
