"""ctypes bindings of libdsa_amd.so (the gfx950 kernels, include/dsa_amd.h)
and libdsa_cpu.so (the host k-th largest of the CPU-offload path,
include/dsa_cpu.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already loaded (one runtime per process: streams and device pointers are
shared).  There is no fallback: if the library is missing the first call
raises, naming the build command.

Status mapping (same error classes as the reference): negative status
(invalid argument / unsupported shape) -> AssertionError, as the reference's
Python asserts raise; positive status (HIP runtime failure) -> RuntimeError.
"""
from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdsa_amd.so")
CPU_LIB_PATH = os.path.join(HERE, "libdsa_cpu.so")

DSA_F32, DSA_BF16, DSA_F16, DSA_FP8 = 0, 1, 2, 3
DSA_OK, DSA_EINVAL, DSA_EUNSUPPORTED, DSA_EHIP = 0, -1, -2, 1

_lib = None
_cpu_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

_SIGNATURES = {
    "dsa_last_error": ([], ctypes.c_char_p),
    "dsa_version": ([], ctypes.c_char_p),
    "dsa_fused_max_T": ([], _I64),
    "dsa_indexer_scores": ([_P, _P, _P, _I, _I64, _I64, _I, _I, _P, _I64, _I, _P], _I),
    "dsa_indexer_scores_strided": ([_P, _P, _P, _I, _I64, _I64, _I, _I, _I64, _I64, _I64, _P,
                                    _I64, _I, _P], _I),
    "dsa_indexer_scores_fp8_scaled": ([_P, _P, _P, _P, _P, _I64, _I64, _I, _I, _P, _I64, _I, _P],
                                      _I),
    "dsa_topk_threshold": ([_P, _I64, _I64, _I64, _I, _I64, _P, _P, _P], _I),
    "dsa_sparse_attn_threshold": ([_P, _I64, _P, _P, _P, _P, _I, _I64, _I64, _I, _I, _I, _F,
                                   _P, _P], _I),
    "dsa_sparse_attn_threshold_tiled": ([_P, _I64, _P, _P, _P, _P, _I, _I64, _I64, _I, _I, _I,
                                         _F, _P, _P], _I),
    "dsa_sparse_attn_threshold_staged": ([_P, _I64, _P, _P, _P, _P, _I, _I64, _I64, _I, _I, _I,
                                          _F, _P, _P], _I),
    "dsa_sparse_attn_threshold_ws": ([_P, _I64, _P, _P, _P, _P, _I, _I64, _I64, _I, _I, _I, _F,
                                      _P, _P, _I64, _P], _I),
    "dsa_sparse_attn_threshold_staged_ws": ([_P, _I64, _P, _P, _P, _P, _I, _I64, _I64, _I, _I,
                                             _I, _F, _P, _P, _I64, _P], _I),
    "dsa_sparse_attn_workspace_bytes": ([_I, _I, _I64, _I64, _I, _I, _I, _I64], _I64),
    "dsa_fused_forward": ([_P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I, _I, _I, _I, _I, _I, _F,
                           _P, _P], _I),
    "dsa_selection_mask": ([_P, _I64, _P, _I64, _I64, _P, _I64, _P], _I),
    "dsa_topk_threshold_mask": ([_P, _I64, _I64, _I64, _I, _P, _P, _I64, _P], _I),
    "dsa_sparse_attn_mask": ([_P, _I64, _P, _P, _P, _I, _I64, _I64, _I, _I, _I, _F, _P, _P], _I),
    "dsa_sparse_attn_uses_mask": ([_I, _I64, _I, _I, _I], _I),
    "dsa_sparse_attn_mask_noalloc": ([_P, _I64, _P, _P, _P, _P, _I, _I64, _I64, _I, _I, _I, _F,
                                      _P, _P], _I),
}


_CPU_SIGNATURES = {
    "dsa_cpu_last_error": ([], ctypes.c_char_p),
    "dsa_cpu_isa": ([], _I),
    "dsa_cpu_topk_threshold": ([_P, _I64, _I64, _I64, _I, _I64, _I64, _P, _I], _I),
}


class DSAUnsupported(AssertionError):
    """A shape the library has no kernel instance for (status DSA_EUNSUPPORTED)."""


def lib():
    """The loaded library (raises RuntimeError if it was never built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python dsa-cpu-topk_amd/build_native.py` "
                "(or __graft_entry__.build()). There is no CPU fallback.")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def cpu_lib():
    """The loaded host library (raises RuntimeError if it was never built)."""
    global _cpu_lib
    if _cpu_lib is None:
        if not os.path.exists(CPU_LIB_PATH):
            raise RuntimeError(
                f"{CPU_LIB_PATH} is not built; run `python dsa-cpu-topk_amd/build_native.py` "
                "(or __graft_entry__.build()).")
        handle = ctypes.CDLL(CPU_LIB_PATH)
        for name, (args, res) in _CPU_SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _cpu_lib = handle
    return _cpu_lib


def check(rc: int, what: str) -> None:
    if rc == DSA_OK:
        return
    msg = lib().dsa_last_error().decode(errors="replace")
    if rc == DSA_EUNSUPPORTED:
        raise DSAUnsupported(f"{what}: {msg}")
    if rc < 0:
        raise AssertionError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def dtype_code(t: torch.dtype) -> int:
    if t == torch.float32:
        return DSA_F32
    if t == torch.bfloat16:
        return DSA_BF16
    if t == torch.float16:
        return DSA_F16
    if t == torch.float8_e4m3fn:
        return DSA_FP8
    raise AssertionError(f"unsupported dtype {t}")


def common_dtype(*xs: torch.Tensor) -> torch.dtype:
    """The one element type a group of inputs is handed to the kernels in:
    their shared dtype if it is fp32/bf16/fp16, otherwise fp32 (the reference
    upcasts every load to fp32: dsa_attention.py:125-129)."""
    d = xs[0].dtype
    if all(x.dtype == d for x in xs) and d in (torch.float32, torch.bfloat16, torch.float16):
        return d
    return torch.float32


def prep(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Contiguous, 16-byte aligned, in `dtype` (copies only when needed)."""
    if x.dtype != dtype:
        x = x.to(dtype)
    x = x.contiguous()
    if x.data_ptr() % 16 != 0:
        x = x.clone()
    return x


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*xs: torch.Tensor) -> None:
    for x in xs:
        if not x.is_cuda:
            raise AssertionError("inputs must be GPU tensors (this is the MI355X HIP path)")
