"""Loaders for the oracle's native builds -- TEST INFRASTRUCTURE ONLY.

port():  ctypes handle of oracle/liboracle_topk.so (this repo's C++ port of
         the reference's AVX-512 k-th-largest).
ref():    the reference's own topk_avx512.cpp compiled into oracle/_ref, as a
         Python extension module exposing topk_threshold(scores, k) and
         topk_threshold_batch_merge(scores, k); None when it was not built or
         the host CPU lacks the AVX-512 subsets it was compiled for.
"""
from __future__ import annotations

import ctypes
import glob
import importlib.machinery
import importlib.util
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_port = None
_ref = None
_REF_FLAGS = ("avx512f", "avx512bw", "avx512dq", "avx512vl", "avx512vbmi", "avx512_vbmi2")


def cpu_flags() -> set[str]:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def port():
    global _port
    if _port is None:
        path = os.path.join(HERE, "liboracle_topk.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle/liboracle_topk.so not built: run python oracle/build.py")
        lib = ctypes.CDLL(path)
        lib.oracle_topk_has_avx512.restype = ctypes.c_int
        lib.oracle_topk_threshold.restype = ctypes.c_int
        lib.oracle_topk_threshold.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                              ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int]
        _port = lib
    return _port


def port_topk_threshold(scores, k, nthreads=None, use_avx512=True):
    """k-th largest per row via the C++ port; scores: array-like [..., n] fp32."""
    x = np.ascontiguousarray(np.asarray(scores, dtype=np.float32))
    n = x.shape[-1]
    rows = x.size // n if n else 0
    out = np.empty(x.shape[:-1] + (1,), dtype=np.float32)
    nt = nthreads or len(os.sched_getaffinity(0))
    rc = port().oracle_topk_threshold(x.ctypes.data, out.ctypes.data, rows, n, int(k), int(nt),
                                      1 if use_avx512 else 0)
    if rc != 0:
        raise ValueError(f"oracle_topk_threshold rejected k={k} n={n}")
    return out


def ref_available() -> bool:
    return bool(glob.glob(os.path.join(HERE, "_ref", "topk_avx512_ref*.so")))


def ref():
    """The reference's compiled extension, or None."""
    global _ref
    if _ref is None:
        hits = glob.glob(os.path.join(HERE, "_ref", "topk_avx512_ref*.so"))
        if not hits or not set(_REF_FLAGS) <= cpu_flags():
            return None
        import torch  # noqa: F401  (the extension links libtorch)
        loader = importlib.machinery.ExtensionFileLoader("topk_avx512_ref", hits[0])
        spec = importlib.util.spec_from_file_location("topk_avx512_ref", hits[0], loader=loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
        _ref = mod
    return _ref
