"""Build recipe for the oracle's native pieces -- TEST INFRASTRUCTURE ONLY.

    python oracle/build.py

1. oracle/liboracle_topk.so  <- oracle/topk_cpu.cpp (this repo's C++ port of
   the reference's AVX-512 k-th-largest; the CPU baseline, kind "port").
2. oracle/_ref/topk_avx512_ref*.so  <- the reference's own topk_avx512.cpp,
   compiled where it lies under /root/reference (kind "reference").  Only
   when that file exists (this build container, not the GPU box: the built
   .so travels there).  It is compiled directly with g++ against the torch
   headers and libraries already installed in this image -- the same
   libtorch the reference's JIT load() links -- with no stand-ins.  Flags
   follow the reference's load() (dsa_hybrid.py:23-33) minus -march=native
   (the .so must run on the GPU box's host) and minus -ffast-math (its rows
   hold -inf).
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REF_SRC = os.environ.get("DSA_REFERENCE_DIR", "/root/reference")
REF_NAME = "topk_avx512_ref"

AVX512 = ["-mavx512f", "-mavx512bw", "-mavx512dq", "-mavx512vl", "-mavx512vbmi",
          "-mavx512vbmi2"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed: {' '.join(cmd)}\n{r.stderr[-4000:]}")


def build_port() -> str:
    out = os.path.join(HERE, "liboracle_topk.so")
    _run(["g++", "-O3", "-std=c++17", "-fopenmp", "-fPIC", "-shared", "-funroll-loops",
          os.path.join(HERE, "topk_cpu.cpp"), "-o", out])
    return out


def ref_available() -> bool:
    return os.path.isfile(os.path.join(REF_SRC, "topk_avx512.cpp"))


def build_ref() -> str | None:
    src = os.path.join(REF_SRC, "topk_avx512.cpp")
    if not os.path.isfile(src):
        return None
    import torch
    from torch.utils.cpp_extension import include_paths, library_paths

    outdir = os.path.join(HERE, "_ref")
    os.makedirs(outdir, exist_ok=True)
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(outdir, REF_NAME + suffix)
    libdir = library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O3", "-std=c++17", "-fopenmp", "-fPIC", "-shared", "-funroll-loops", *AVX512,
           f"-DTORCH_EXTENSION_NAME={REF_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{p}" for p in include_paths()], f"-I{sysconfig.get_paths()['include']}",
           src, "-o", out, f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           f"-Wl,-rpath,{libdir}"]
    _run(cmd)
    return out


def build(verbose: bool = True) -> None:
    p = build_port()
    if verbose:
        print(f"built {p}")
    r = build_ref()
    if verbose:
        print(f"built {r}" if r else "reference sources absent: oracle/_ref not built")


if __name__ == "__main__":
    build()
    sys.exit(0)
