"""Ahead-of-time build of libcpq.so for gfx950 (hipcc; no JIT, no torch extension).

Usage: ``python -m cider_press_amd._build`` (or ``__graft_entry__.build()``).
Always recompiles every source; objects go to ``cider_press_amd/_build/``,
the shared library to ``cider_press_amd/libcpq.so``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcpq.so")

SOURCES = [
    "runtime.cpp",
    "ops.cpp",
    "graph.cpp",
    "safetensors.cpp",
    "noalloc.hip",
    "kernels/dequantize.hip",
    "kernels/embed.hip",
    "kernels/qmv.hip",
    "kernels/skinny.hip",
    "kernels/qmm.hip",
    "kernels/qmm_wide.hip",
    "kernels/qmm_dma.hip", "kernels/qmm_small.hip",
    "kernels/qmm_n.hip",
    "kernels/gather.hip",
    "kernels/gather_decode.hip", "kernels/qmm_rows.hip",
    "kernels/moe.hip",
    "kernels/stream_read.hip",
]

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    f"--offload-arch={ARCH}",
    # Packed FP32 VALU ops stay off: the compiler must not form v_pk_*_f32.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Kernel arguments arrive in SGPRs before the wave starts (gfx950
    # kernarg preloading), so a wave's first loads need no scalar round trip.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-I", os.path.join(ROOT, "include"),
]


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, src.replace("/", "_") + ".o")
    lang = ["-x", "hip"]
    cmd = [HIPCC, *lang, *COMMON, "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    workers = min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
