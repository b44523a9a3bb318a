"""Builds libstrata_moe.so (HIP kernels for gfx950 + C++ host runtime) in-tree.

Every HIP translation unit is compiled for gfx950 only, without floating-point
contraction (fusion happens only where the code writes fma), and with packed-FP32
instruction selection disabled.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libstrata_moe.so"
INCLUDE = HERE.parent / "include"

HIP_SOURCES = ["sm_route_group.hip", "sm_gemm.hip", "sm_wide.hip", "sm_post.hip", "sm_decode.hip", "sm_runtime.cpp"]
HOST_SOURCES = ["sm_synth.cpp", "sm_gguf.cpp", "sm_tiered.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libstrata_moe.so")


def _compile(src: str, hipcc: str) -> Path:
    obj = BUILD / (src + ".o")
    path = CSRC / src
    if src in HIP_SOURCES:
        cmd = [hipcc, "-x", "hip", *HIPCC_FLAGS, "-c", str(path), "-o", str(obj)]
    else:
        cmd = [hipcc, "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", "-c", str(path), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every source and links libstrata_moe.so; returns its path."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    srcs = HIP_SOURCES + HOST_SOURCES
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
