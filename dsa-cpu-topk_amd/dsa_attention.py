"""DeepSeek Sparse Attention forward on MI355X -- drop-in for the reference's
dsa_attention.py (same names, arguments, asserts and fp32 outputs).

Pipeline:
  1. lightning indexer   I[t,s] = sum_j w[t,j] * ReLU(<q_idx[t,j], k_idx[s]>), causal
  2. threshold           thr[t] = min(top_k, T)-th largest of row t (ties counted)
  3. sparse attention    softmax over {s <= t : I[t,s] >= thr[t]} of <Q,K>/sqrt(DQ), times V

Inputs (GPU tensors; fp32, bf16 or fp16):
  q_idx [B,T,HI,DI]  k_idx [B,T,DI]  w_idx [B,T,HI]  Q,K [B,T,HQ,DQ]  V [B,T,HQ,DV]
Output: O [B,T,HQ,DV] fp32.

The *_triton names are kept so the reference's callers switch without edits;
every one of them runs hand-written gfx950 kernels from libdsa_amd.so:
  dsa_attention_triton                    -> one fused kernel (T <= 2048)
  dsa_attention_split_triton              -> indexer, radix-select, sparse attention
  sparse_attention_with_threshold_triton  -> sparse attention given any threshold
`dsa_attention_torch` / `dsa_attention_naive` are the reference's plain-torch
functions, kept as API; no *_triton path calls them.
"""
from __future__ import annotations

import math

import torch

import _dsa_lib as L
from lightning_indexer import indexer_scores_hip, indexer_scores_torch
from topk_threshold import topk_threshold, topk_threshold_mask


# ---------------------------------------------------------------------------
# Plain-torch functions of the reference API (dsa_attention.py:35-89)
# ---------------------------------------------------------------------------
def dsa_attention_torch(q_idx, k_idx, w_idx, Q, K, V, top_k: int) -> torch.Tensor:
    B, T, HQ, DQ = Q.shape
    scale = 1.0 / math.sqrt(DQ)
    scores = indexer_scores_torch(q_idx, k_idx, w_idx)
    k_eff = min(top_k, T)
    topv, _ = scores.topk(k_eff, dim=-1)
    threshold = topv[..., -1:]
    causal = torch.ones(T, T, device=Q.device, dtype=torch.bool).tril()
    sel = (scores >= threshold) & causal
    logits = torch.einsum("bthd,bshd->bths", Q, K) * scale
    logits = logits.masked_fill(~sel.unsqueeze(2), float("-inf"))
    attn = torch.softmax(logits, dim=-1)
    return torch.einsum("bths,bshd->bthd", attn, V)


def dsa_attention_naive(q_idx, k_idx, w_idx, Q, K, V, top_k: int) -> torch.Tensor:
    B, T, HQ, DQ = Q.shape
    DV = V.shape[-1]
    scale = 1.0 / math.sqrt(DQ)
    out = torch.zeros(B, T, HQ, DV, device=Q.device, dtype=torch.float32)
    for b in range(B):
        for t in range(T):
            scores = torch.full((T,), float("-inf"), device=Q.device)
            for s in range(t + 1):
                dots = (q_idx[b, t] * k_idx[b, s].unsqueeze(0)).sum(-1)
                scores[s] = (w_idx[b, t] * torch.relu(dots)).sum()
            thresh = scores.topk(min(top_k, T)).values[-1]
            keep = (scores >= thresh) & (torch.arange(T, device=Q.device) <= t)
            sel = torch.nonzero(keep, as_tuple=False).squeeze(-1)
            logits = torch.einsum("hd,khd->kh", Q[b, t], K[b, sel]) * scale
            out[b, t] = torch.einsum("kh,khd->hd", torch.softmax(logits, dim=0), V[b, sel])
    return out


# ---------------------------------------------------------------------------
# MI355X kernels
# ---------------------------------------------------------------------------
def _attn_inputs(Q, K, V):
    dt = L.common_dtype(Q, K, V)
    return dt, L.prep(Q, dt), L.prep(K, dt), L.prep(V, dt)


def sparse_attention_hip(scores: torch.Tensor, threshold: torch.Tensor, Q, K, V,
                         out: torch.Tensor | None = None, tiled: bool = False,
                         kernel: str | None = None) -> torch.Tensor:
    """Sparse attention for any T given scores [B,T,T] fp32 and threshold
    [B,T,1] (or [B,T]); only entries s <= t of each score row are read.

    The library picks the kernel: per-query gathers; dense-masked MFMA tiles
    for T >= 4096 with 16-bit Q/K/V and DQ = DV in {64, 128}; K/V staged
    through LDS for fp32 rows of HQ*DQ = 512 at T >= 3072 when the batch
    gives at least one 64-query tile per compute unit (with a workspace
    from the caching allocator, so that long key ranges split over several
    blocks; dsa_sparse_attn_workspace_bytes gives its size).  Where it would
    take the tiles, the selection is first reduced to a bitmask
    (dsa_selection_mask, 1 bit per (query, key) instead of a 4-byte score
    read once per head) and the tile kernel reads that (dsa_sparse_attn_mask):
    the same output, bit for bit.
    kernel="tiled" (or tiled=True) / "staged" / "mask" runs that kernel at
    any T (AssertionError for shapes it does not cover)."""
    L.require_gpu(scores, threshold, Q, K, V)
    B, T, _ = scores.shape
    HQ, DQ = Q.shape[-2], Q.shape[-1]
    DV = V.shape[-1]
    assert Q.shape == (B, T, HQ, DQ) and K.shape == (B, T, HQ, DQ), "Q/K shape"
    assert V.shape == (B, T, HQ, DV), "V shape"
    assert threshold.numel() == B * T, "threshold must hold one value per query"
    scores = L.prep(scores, torch.float32)
    thr = L.prep(threshold, torch.float32)
    dt, Q, K, V = _attn_inputs(Q, K, V)
    if out is None:
        out = torch.empty(B, T, HQ, DV, device=Q.device, dtype=torch.float32)
    if tiled:
        kernel = "tiled"
    assert kernel in (None, "tiled", "staged", "mask"), f"unknown kernel {kernel!r}"
    if kernel is None and L.lib().dsa_sparse_attn_uses_mask(L.dtype_code(dt), T, HQ, DQ, DV):
        kernel = "mask"
    if kernel == "mask":
        return _sparse_attention_mask(scores, thr, Q, K, V, out)
    args = (scores.data_ptr(), T, thr.data_ptr(), Q.data_ptr(), K.data_ptr(), V.data_ptr(),
            L.dtype_code(dt), B, T, HQ, DQ, DV, 1.0 / math.sqrt(DQ), out.data_ptr())
    if kernel == "tiled":
        rc = L.lib().dsa_sparse_attn_threshold_tiled(*args, L.stream_ptr(Q.device))
    else:
        staged = kernel == "staged"
        with torch.cuda.device(Q.device):
            nws = L.lib().dsa_sparse_attn_workspace_bytes(int(staged), L.dtype_code(dt), B, T, HQ,
                                                          DQ, DV, T)
        ws = torch.empty(max(nws, 0), device=Q.device, dtype=torch.uint8) if nws > 0 else None
        fn = (L.lib().dsa_sparse_attn_threshold_staged_ws if staged
              else L.lib().dsa_sparse_attn_threshold_ws)
        rc = fn(*args, ws.data_ptr() if ws is not None else None, nws if ws is not None else 0,
                L.stream_ptr(Q.device))
    L.check(rc, "sparse_attention")
    return out


def selection_mask(scores: torch.Tensor, threshold: torch.Tensor) -> torch.Tensor:
    """Bitmask of the causal threshold selection: int64 [B, T, ceil(T/64)],
    bit i of word w of row (b, t) set iff 64w + i <= t and
    scores[b, t, 64w + i] >= threshold[b, t] (words past a row's causal
    range up to its 128-query block are 0, later ones are not written)."""
    L.require_gpu(scores, threshold)
    B, T, _ = scores.shape
    assert threshold.numel() == B * T, "threshold must hold one value per query"
    scores = L.prep(scores, torch.float32)
    thr = L.prep(threshold, torch.float32)
    W = (T + 63) // 64
    mask = torch.empty(B, T, W, device=scores.device, dtype=torch.int64)
    rc = L.lib().dsa_selection_mask(scores.data_ptr(), T, thr.data_ptr(), B, T, mask.data_ptr(), W,
                                    L.stream_ptr(scores.device))
    L.check(rc, "selection_mask")
    return mask


def sparse_attention_from_mask(mask: torch.Tensor, Q, K, V,
                               out: torch.Tensor | None = None) -> torch.Tensor:
    """Sparse attention on the dense-masked tiles with the selection given as
    a bitmask (selection_mask or topk_threshold_mask): 16-bit Q/K/V, DQ = DV
    in {64, 128} (DSAUnsupported otherwise)."""
    L.require_gpu(mask, Q, K, V)
    B, T, HQ, DQ = Q.shape
    DV = V.shape[-1]
    assert K.shape == (B, T, HQ, DQ) and V.shape == (B, T, HQ, DV), "K/V shapes"
    W = (T + 63) // 64
    assert (mask.dtype == torch.int64 and mask.is_contiguous() and mask.dim() == 3
            and mask.shape[:2] == (B, T) and mask.shape[-1] >= W), "mask: int64 [B, T, >= ceil(T/64)]"
    dt, Q, K, V = _attn_inputs(Q, K, V)
    if out is None:
        out = torch.empty(B, T, HQ, DV, device=Q.device, dtype=torch.float32)
    rc = L.lib().dsa_sparse_attn_mask(
        mask.data_ptr(), mask.shape[-1], Q.data_ptr(), K.data_ptr(), V.data_ptr(), L.dtype_code(dt),
        B, T, HQ, DQ, DV, 1.0 / math.sqrt(DQ), out.data_ptr(), L.stream_ptr(Q.device))
    L.check(rc, "sparse_attention")
    return out


def _sparse_attention_mask(scores, thr, Q, K, V, out):
    return sparse_attention_from_mask(selection_mask(scores, thr), Q, K, V, out=out)


def dsa_split_hip(q_idx, k_idx, w_idx, Q, K, V, top_k: int) -> torch.Tensor:
    """Split forward for any T: indexer (causal half only) -> causal
    radix-select of the min(top_k,T)-th largest -> sparse attention.  Where
    the attention runs on tiles from a selection bitmask, the select writes
    that bitmask in its own pass over the scores (topk_threshold_mask): the
    same output as the three steps apart, bit for bit."""
    B, T, HQ, DQ = Q.shape
    DV = V.shape[-1]
    scores = indexer_scores_hip(q_idx, k_idx, w_idx, write_upper=False)
    k = min(top_k, T)
    L.require_gpu(Q, K, V)
    dt = L.common_dtype(Q, K, V)
    if L.lib().dsa_sparse_attn_uses_mask(L.dtype_code(dt), T, HQ, DQ, DV):
        _, mask = topk_threshold_mask(scores, k)
        return sparse_attention_from_mask(mask, Q, K, V)
    thr = topk_threshold(scores, k, causal=True)
    return sparse_attention_hip(scores, thr, Q, K, V)


def dsa_fused_hip(q_idx, k_idx, w_idx, Q, K, V, top_k: int) -> torch.Tensor:
    """One-kernel forward (T <= 2048); raises _dsa_lib.DSAUnsupported for a
    shape without a fused kernel instance."""
    L.require_gpu(q_idx, k_idx, w_idx, Q, K, V)
    B, T, HQ, DQ = Q.shape
    HI, DI = q_idx.shape[2], q_idx.shape[3]
    DV = V.shape[-1]
    assert k_idx.shape == (B, T, DI) and w_idx.shape == (B, T, HI), "indexer input shapes"
    assert K.shape == (B, T, HQ, DQ) and V.shape == (B, T, HQ, DV), "K/V shapes"
    dt = L.common_dtype(q_idx, k_idx, w_idx, Q, K, V)
    q_idx, k_idx, w_idx, Q, K, V = (L.prep(x, dt) for x in (q_idx, k_idx, w_idx, Q, K, V))
    out = torch.empty(B, T, HQ, DV, device=Q.device, dtype=torch.float32)
    rc = L.lib().dsa_fused_forward(
        q_idx.data_ptr(), k_idx.data_ptr(), w_idx.data_ptr(), Q.data_ptr(), K.data_ptr(),
        V.data_ptr(), L.dtype_code(dt), B, T, HI, DI, HQ, DQ, DV, int(top_k),
        1.0 / math.sqrt(DQ), out.data_ptr(), L.stream_ptr(Q.device))
    L.check(rc, "dsa_fused")
    return out


def dsa_forward_hip(q_idx, k_idx, w_idx, Q, K, V, top_k: int) -> torch.Tensor:
    """Forward for any shape: the fused kernel where one exists (T <= 2048),
    else the split kernels.  Both are gfx950 HIP; nothing runs on the CPU."""
    if Q.shape[1] <= L.lib().dsa_fused_max_T():
        try:
            return dsa_fused_hip(q_idx, k_idx, w_idx, Q, K, V, top_k)
        except L.DSAUnsupported:
            pass
    return dsa_split_hip(q_idx, k_idx, w_idx, Q, K, V, top_k)


def _assert_pow2(pairs):
    for n, v in pairs:
        assert v & (v - 1) == 0 and v > 0, f"{n}={v} must be a power of 2"


def dsa_attention_triton(q_idx, k_idx, w_idx, Q, K, V, top_k: int,
                         BLOCK_S: int = 32) -> torch.Tensor:
    """Drop-in for the fused reference forward (dsa_attention.py:196-227):
    same asserts; BLOCK_S is accepted and only checked, as there."""
    B, T, HQ, DQ = Q.shape
    DV = V.shape[-1]
    HI, DI = q_idx.shape[2], q_idx.shape[3]
    _assert_pow2([("T", T), ("HI", HI), ("DI", DI), ("HQ", HQ), ("DQ", DQ), ("DV", DV),
                  ("BLOCK_S", BLOCK_S), ("top_k", top_k)])
    assert T % BLOCK_S == 0, "T must be divisible by BLOCK_S"
    assert top_k <= T
    return dsa_forward_hip(q_idx, k_idx, w_idx, Q, K, V, top_k)


def sparse_attention_with_threshold_triton(scores, threshold, Q, K, V) -> torch.Tensor:
    """Drop-in for the reference (dsa_attention.py:298-324): same asserts,
    threshold [B,T,1] from anywhere (e.g. a CPU select, dsa_hybrid.py:66)."""
    B, T, _ = scores.shape
    HQ, DQ = Q.shape[-2], Q.shape[-1]
    DV = V.shape[-1]
    _assert_pow2([("T", T), ("HQ", HQ), ("DQ", DQ), ("DV", DV)])
    return sparse_attention_hip(scores, threshold, Q, K, V)


def dsa_attention_split_triton(q_idx, k_idx, w_idx, Q, K, V, top_k: int,
                               BLOCK_T: int = 32, BLOCK_S: int = 32) -> torch.Tensor:
    """Drop-in for the split reference forward (dsa_attention.py:327-345)."""
    B, T, HQ, DQ = Q.shape
    DV = V.shape[-1]
    HI, DI = q_idx.shape[2], q_idx.shape[3]
    _assert_pow2([("T", T), ("HI", HI), ("DI", DI), ("HQ", HQ), ("DQ", DQ), ("DV", DV),
                  ("BLOCK_T", BLOCK_T), ("BLOCK_S", BLOCK_S), ("top_k", top_k)])
    assert T % BLOCK_T == 0, "T must be divisible by BLOCK_T"
    assert T % BLOCK_S == 0, "T must be divisible by BLOCK_S"
    assert top_k <= T
    return dsa_split_hip(q_idx, k_idx, w_idx, Q, K, V, top_k)
