"""k-th largest per row ("top-K threshold") -- drop-in for the reference's
AVX-512 extension API (topk_avx512.cpp:226-264: topk_threshold and
topk_threshold_batch_merge).

Same contract: scores fp32, contiguous, k > 0, k <= N; returns the k-th
largest of each row of the last dimension (ties counted) as a tensor of
shape sizes[:-1] + [1] -- bit-identical to torch.topk(x, k).values[..., -1:].
Same error class: RuntimeError (the extension's TORCH_CHECK).

Where it runs is where the tensor lives, and nothing crosses over:
  * GPU tensors: the MI355X radix-select (libdsa_amd.so);
  * CPU tensors: the host library of the CPU-offload path (libdsa_cpu.so,
    AVX-512 scan + vector quickselect on OpenMP threads) -- the reference's
    extension takes CPU tensors, and its callers (dsa_hybrid.py:61) pass the
    pinned host copy of the scores.
A GPU tensor never runs on the host, and a missing library raises.

Extras the reference lacks: `topk_indices` (the exactly-k index set, lowest
index winning ties; GPU) and a `causal` mode for [B,T,T] indexer matrices
that reads only the s <= t entries of each row (both devices).
"""
from __future__ import annotations

import torch

import _dsa_lib as L


def _check(scores: torch.Tensor, k: int) -> int:
    if not scores.is_contiguous():
        raise RuntimeError("scores must be contiguous")
    if scores.dtype != torch.float32:
        raise RuntimeError("fp32 only")
    if k <= 0:
        raise RuntimeError("k must be > 0")
    if scores.dim() == 0:
        raise RuntimeError("scores must have at least one dimension")
    N = scores.shape[-1]
    if k > N:
        raise RuntimeError("k must be <= N")
    return N


def _select(scores: torch.Tensor, k: int, causal: bool, want_idx: bool,
            thr: torch.Tensor | None = None, nthreads: int = 0):
    N = _check(scores, k)
    rows = scores.numel() // N if N else 0
    causal_T = 0
    if causal:
        if scores.dim() < 2 or scores.shape[-2] != N:
            raise RuntimeError("causal select needs [..., T, T] scores")
        causal_T = N
    if thr is None:
        thr = torch.empty(scores.shape[:-1] + (1,), device=scores.device, dtype=torch.float32)
    elif (thr.dtype != torch.float32 or not thr.is_contiguous() or thr.numel() != rows
          or thr.device != scores.device):
        raise RuntimeError("thr must be a contiguous fp32 tensor of one value per row")
    if not scores.is_cuda:
        if want_idx:
            raise RuntimeError("topk_indices: GPU tensors only")
        if rows:
            lib = L.cpu_lib()
            rc = lib.dsa_cpu_topk_threshold(scores.data_ptr(), rows, N, N, int(k), causal_T, 0,
                                            thr.data_ptr(), int(nthreads))
            if rc != 0:
                msg = lib.dsa_cpu_last_error().decode(errors="replace")
                raise RuntimeError(f"topk_threshold: {msg}")
        return thr, None
    idx = None
    if want_idx:
        idx = torch.empty(scores.shape[:-1] + (k,), device=scores.device, dtype=torch.int32)
    if rows:
        rc = L.lib().dsa_topk_threshold(scores.data_ptr(), rows, N, N, int(k), causal_T,
                                        thr.data_ptr(), idx.data_ptr() if want_idx else None,
                                        L.stream_ptr(scores.device))
        if rc != L.DSA_OK:
            msg = L.lib().dsa_last_error().decode(errors="replace")
            raise RuntimeError(f"topk_threshold: {msg}")
    return thr, idx


def topk_threshold(scores: torch.Tensor, k: int, causal: bool = False,
                   nthreads: int = 0) -> torch.Tensor:
    """k-th largest of every row of the last dim -> shape [..., 1] fp32.

    causal=True treats a [..., T, T] matrix as causal indexer scores: row t
    reads only entries s <= t and counts the rest as -inf (what the
    reference's masked full row holds), halving the bytes read.
    nthreads: host threads for a CPU tensor (0 = OMP_NUM_THREADS / all).
    """
    return _select(scores, k, causal, False, nthreads=nthreads)[0]


def topk_threshold_into(scores: torch.Tensor, k: int, thr: torch.Tensor,
                        causal: bool = False, nthreads: int = 0) -> torch.Tensor:
    """topk_threshold writing into a preallocated fp32 tensor of one value
    per row, on the scores' device (no allocation: for pipelines that reuse
    their buffers, e.g. the pinned thr_cpu of the CPU-offload path)."""
    return _select(scores, k, causal, False, thr, nthreads)[0]


def topk_threshold_batch_merge(scores: torch.Tensor, k: int) -> torch.Tensor:
    """The reference's batch-merge variant has the same contract and result
    (topk_avx512.cpp:255-257); each device here has one select."""
    return _select(scores, k, False, False)[0]


def topk_threshold_mask(scores: torch.Tensor, k: int, thr: torch.Tensor | None = None,
                        mask: torch.Tensor | None = None):
    """Causal thresholds of [B, T, T] GPU scores plus the selection bitmask
    of those thresholds -- (thr [B, T, 1] fp32, mask [B, T, ceil(T/64)]
    int64), the same as topk_threshold(scores, k, causal=True) followed by
    dsa_attention.selection_mask(scores, thr), bit for bit, with the mask
    written by the select's own pass over the scores where it can.
    thr / mask: preallocated outputs (optional)."""
    if scores.dim() != 3 or scores.shape[-2] != scores.shape[-1]:
        raise RuntimeError("topk_threshold_mask needs [B, T, T] scores")
    _check(scores, k)
    L.require_gpu(scores)
    B, T, _ = scores.shape
    W = (T + 63) // 64
    if thr is None:
        thr = torch.empty(B, T, 1, device=scores.device, dtype=torch.float32)
    if mask is None:
        mask = torch.empty(B, T, W, device=scores.device, dtype=torch.int64)
    if (thr.dtype != torch.float32 or not thr.is_contiguous() or thr.numel() != B * T
            or thr.device != scores.device):
        raise RuntimeError("thr must be a contiguous fp32 tensor of one value per row")
    if (mask.dtype != torch.int64 or not mask.is_contiguous() or mask.shape != (B, T, W)
            or mask.device != scores.device):
        raise RuntimeError("mask must be a contiguous int64 [B, T, ceil(T/64)] tensor")
    if B * T:
        rc = L.lib().dsa_topk_threshold_mask(scores.data_ptr(), B, T, T, int(k), thr.data_ptr(),
                                             mask.data_ptr(), W, L.stream_ptr(scores.device))
        if rc != L.DSA_OK:
            msg = L.lib().dsa_last_error().decode(errors="replace")
            raise RuntimeError(f"topk_threshold_mask: {msg}")
    return thr, mask


def topk_indices(scores: torch.Tensor, k: int, causal: bool = False):
    """(threshold [...,1] fp32, indices [...,k] int32).

    indices = the k positions a stable descending sort puts first: every
    entry above the threshold plus the lowest-index entries equal to it, in
    ascending index order.
    """
    return _select(scores, k, causal, True)
