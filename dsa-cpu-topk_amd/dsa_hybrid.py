"""Precomputed-threshold DSA path -- drop-in for the reference's dsa_hybrid.py
(HybridContext, dsa_hybrid_cpu_topk; reference dsa_hybrid.py:36-66).

Reference pipeline: GPU indexer -> pinned d2h of the [B,T,T] scores -> CPU
AVX-512 k-th largest -> h2d threshold -> GPU sparse attention that takes the
threshold as an input.  On MI355X the middle of that pipeline is the
radix-select of topk_threshold.py, which keeps the extension's contract
(k-th largest per row, [B,T,1], same checks) but runs on the GPU, so the
scores never cross PCIe.  The boundary call the reference makes at
dsa_hybrid.py:66 -- sparse attention with an externally supplied threshold
tensor -- is unchanged and accepts any [B,T,1] threshold.
"""
from __future__ import annotations

import torch

from dsa_attention import sparse_attention_with_threshold_triton
from lightning_indexer import indexer_scores_hip
from topk_threshold import topk_threshold


class HybridContext:
    """Reusable per-shape buffers (reference dsa_hybrid.py:36-43)."""

    def __init__(self, B, T, device="cuda"):
        self.B, self.T = B, T
        self.thr_gpu = torch.empty((B, T, 1), dtype=torch.float32, device=device)
        self.scores_gpu = torch.empty((B, T, T), dtype=torch.float32, device=device)


def dsa_hybrid_cpu_topk(q_idx, k_idx, w_idx, Q, K, V, top_k: int,
                        ctx: HybridContext | None = None) -> torch.Tensor:
    """Indexer -> k-th-largest threshold -> sparse attention with the
    threshold as an input (reference dsa_hybrid.py:46-66).  top_k must be
    <= T, as the extension's k <= N check requires (RuntimeError)."""
    B, T = Q.shape[0], Q.shape[1]
    if ctx is None:
        ctx = HybridContext(B, T, device=Q.device)
    assert ctx.B == B and ctx.T == T

    # 1. indexer, full matrix as in the reference (dsa_hybrid.py:54)
    scores = indexer_scores_hip(q_idx, k_idx, w_idx, write_upper=True, out=ctx.scores_gpu)
    # 2-4. k-th largest of every full row -> [B,T,1] (dsa_hybrid.py:57-63)
    ctx.thr_gpu.copy_(topk_threshold(scores, top_k))
    # 5. sparse attention with the precomputed threshold (dsa_hybrid.py:66)
    return sparse_attention_with_threshold_triton(scores, ctx.thr_gpu, Q, K, V)
