"""Build the two native libraries in-tree:

    libdsa_amd.so  (include/dsa_amd.h)  the gfx950 kernels, hipcc, from csrc/*.hip + capi.cpp
    libdsa_cpu.so  (include/dsa_cpu.h)  the host k-th largest of the CPU-offload path, g++ + OpenMP

    python dsa-cpu-topk_amd/build_native.py          # build both (always recompiles)

Both are plain C-ABI shared objects; nothing here depends on torch.
Translation units compile in parallel, then link.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libdsa_amd.so")
OUT_CPU = os.path.join(HERE, "libdsa_cpu.so")
CPU_SOURCES = ["topk_cpu.cpp"]
# No -march=native (the library runs on the GPU box's host, whatever it is:
# AVX-512 code is compiled per function and picked at run time) and no
# -ffast-math (score rows hold -inf and NaN must order as torch.topk orders it).
CXXFLAGS = ["-O3", "-std=c++17", "-fPIC", "-fopenmp", "-Wall", "-Wextra"]
SOURCES = ["capi.cpp", "topk.hip", "indexer.hip", "sparse_attn.hip", "tile_attn.hip",
           "staged_attn.hip", "fused.hip"]

HIPFLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # No packed-fp32 instructions anywhere (they have produced silent wrong
    # results on these boxes); the host pass warns that it does not know the
    # feature, which is harmless.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(src: str, objdir: str) -> str:
    obj = os.path.join(objdir, os.path.basename(src) + ".o")
    cmd = [hipcc(), *HIPFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def build_cpu(verbose: bool = True) -> str:
    """libdsa_cpu.so with the host C++ compiler (no GPU code)."""
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    tmp = OUT_CPU + ".tmp"
    cmd = [cxx, *CXXFLAGS, "-shared", "-o", tmp, *(os.path.join(CSRC, s) for s in CPU_SOURCES)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{cxx} failed for {CPU_SOURCES}:\n{r.stderr[-6000:]}")
    os.replace(tmp, OUT_CPU)
    if verbose:
        print(f"built {OUT_CPU}")
    return OUT_CPU


def build(verbose: bool = True) -> str:
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        cpu = ex.submit(build_cpu, verbose)
        objs = list(ex.map(lambda s: _compile(s, objdir), SOURCES))
        cpu.result()
    tmp = OUT + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
