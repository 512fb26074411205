"""CPU restatement of the reference DSA forward -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker (and, for the CPU baseline, as the thing timed on
the host cores).  The product never routes through it.

What each function restates (reference files under Infatoshi/dsa-cpu-topk):
  indexer_scores         lightning_indexer.py:26-33  (einsum, ReLU, w-sum, causal -inf)
  indexer_scores_naive   dsa_attention.py:67-74      (per-(t,s) loop)
  topk_threshold         dsa_attention.py:41-44, topk_avx512.cpp:226-249
                         (k-th largest of the full row, ties counted)
  select_indices         no reference counterpart: the exactly-k set a stable
                         descending sort puts first (lowest index wins ties);
                         the reference's topk_mask (lightning_indexer.py:137-144)
                         takes torch.topk's indices, whose tie order is unspecified
  sparse_attn_threshold  dsa_attention.py:45-51 and :256-290 (keep = s<=t & score>=thr)
  dsa_forward            dsa_attention.py:35-52      (dsa_attention_torch)
  dsa_forward_naive      dsa_attention.py:59-89      (dsa_attention_naive)

How each is pinned (tests/test_oracle.py): indexer by the per-(t,s) loop and
closed forms (w=0, anti-aligned keys, single head self-dot); threshold by
numpy sorting, the C++ port (oracle/topk_cpu.cpp), the reference's own
compiled extension (oracle/_ref, when built) and the -inf closed form for
short rows; select_indices by an explicit key-by-key brute force and its
defining properties; attention by the naive loop and closed forms (one
selected key gives V[s]; equal logits give the mean of the selected V rows);
the forward by dsa_forward_naive and the committed golden fixtures.

All arithmetic runs in `acc` precision (float64 by default: the truth the
GPU's fp32 result is compared against with rtol 1e-4 / 2e-2).  With
acc=torch.float32 it is the reference's torch-vectorised CPU path, which is
what bench.py times as the CPU baseline.
"""
from __future__ import annotations

import math

import numpy as np
import torch

NEG_INF = float("-inf")


# ---------------------------------------------------------------------------
# Inputs
# ---------------------------------------------------------------------------
def make_inputs(B, T, HI, DI, HQ, DQ, DV, *, dtype=torch.float32, seed0=0, w_scale=None,
                scale=1.0, v_scale=1.0):
    """Seeded CPU inputs: seeds seed0+0..5 for q_idx, k_idx, w, Q, K, V.

    Default distribution is the one BASELINE.json states: q_idx, k_idx, Q, K,
    V ~ N(0,1), w ~ N(0,1)/sqrt(HI).  The reference's own tests scale
    everything but V by 0.3 (test_dsa.py:17-24): pass scale=0.3, w_scale=0.3.
    Generated on the CPU generator so they do not depend on any GPU's RNG.
    """
    def rn(shape, seed):
        g = torch.Generator().manual_seed(seed)
        return torch.randn(shape, generator=g, dtype=torch.float32)

    ws = (1.0 / math.sqrt(HI)) if w_scale is None else w_scale
    q_idx = rn((B, T, HI, DI), seed0 + 0) * scale
    k_idx = rn((B, T, DI), seed0 + 1) * scale
    w_idx = rn((B, T, HI), seed0 + 2) * ws
    Q = rn((B, T, HQ, DQ), seed0 + 3) * scale
    K = rn((B, T, HQ, DQ), seed0 + 4) * scale
    V = rn((B, T, HQ, DV), seed0 + 5) * v_scale
    return tuple(x.to(dtype) for x in (q_idx, k_idx, w_idx, Q, K, V))


def _chunk_rows(T, per_row_elems, budget=1 << 25):
    return max(1, min(T, budget // max(1, per_row_elems)))


# ---------------------------------------------------------------------------
# Indexer
# ---------------------------------------------------------------------------
def indexer_scores(q, k, w, *, acc=torch.float64, rows=None, chunk=None):
    """I[b,t,s] = sum_j w[b,t,j] * relu(<q[b,t,j], k[b,s]>), -inf for s > t.

    q [B,T,HI,DI], k [B,T,DI], w [B,T,HI] -> [B,T,T] (or [B,len(rows),T] for
    the query positions in `rows`).  Chunked over queries so the [.,HI,T]
    intermediate stays bounded (the reference materialises all of it).
    """
    B, T, HI, DI = q.shape
    qf, kf, wf = q.to(acc), k.to(acc), w.to(acc)
    ts = torch.arange(T) if rows is None else torch.as_tensor(rows, dtype=torch.long)
    out = torch.empty((B, len(ts), T), dtype=acc)
    step = chunk or _chunk_rows(len(ts), B * HI * T)
    for i0 in range(0, len(ts), step):
        tt = ts[i0:i0 + step]
        dots = torch.einsum("bthd,bsd->bths", qf[:, tt], kf)           # [B,c,HI,T]
        sc = (wf[:, tt].unsqueeze(-1) * torch.relu(dots)).sum(dim=2)     # [B,c,T]
        upper = torch.arange(T)[None, :] > tt[:, None]
        out[:, i0:i0 + step] = sc.masked_fill(upper.unsqueeze(0), NEG_INF)
    return out


def indexer_scores_naive(q, k, w):
    """Per-(b,t,s) loop in float64 (dsa_attention.py:67-74).  Tiny shapes only."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    B, T, HI, _ = q.shape
    out = np.full((B, T, T), NEG_INF)
    for b in range(B):
        for t in range(T):
            for s in range(t + 1):
                dots = q[b, t] @ k[b, s]                 # [HI]
                out[b, t, s] = float(np.sum(w[b, t] * np.maximum(dots, 0.0)))
    return out


# ---------------------------------------------------------------------------
# Select
# ---------------------------------------------------------------------------
def topk_threshold(scores, k):
    """k-th largest of every row of the last dim (ties counted), shape [...,1].

    Exactly torch.topk(x, k).values[..., -1:], which is what the reference
    computes (dsa_attention.py:43-44) and what its extension is tested to
    equal bit-for-bit (test_topk_avx512.py:20-26).
    """
    x = torch.as_tensor(scores)
    n = x.shape[-1]
    if not (0 < k <= n):
        raise ValueError(f"k={k} outside [1, {n}]")
    return torch.topk(x, k, dim=-1).values[..., -1:]


def radix_key(x):
    """Order-preserving int64 key: numeric order, -0.0 == +0.0, every NaN
    equal and above +inf (torch.topk's NaN order)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.int64)
    u = np.where(u == 0x80000000, 0, u)
    u = np.where((u & 0x7FFFFFFF) > 0x7F800000, 0x7FC00000, u)
    neg = (u & 0x80000000) != 0
    return np.where(neg, (~u) & 0xFFFFFFFF, u | 0x80000000)


def select_indices(scores, k):
    """Exactly-k index set: the first k positions of a stable descending sort
    of each row (every entry above the k-th largest plus the lowest-index
    entries equal to it), returned in ascending index order, int32."""
    key = radix_key(scores)
    order = np.argsort(-key, axis=-1, kind="stable")[..., :k]
    return np.sort(order, axis=-1).astype(np.int32)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
def sparse_attn_threshold(scores, thr, Q, K, V, *, acc=torch.float64, rows=None, chunk=None):
    """O[b,t] = softmax over {s <= t : scores[b,t,s] >= thr[b,t]} of
    <Q[b,t,h], K[b,s,h]>/sqrt(DQ), applied to V (dsa_attention.py:45-51).

    scores [B,T,T] (or [B,len(rows),T]), thr [B,T,1] (or [B,len(rows),1]).
    """
    B, T, HQ, DQ = Q.shape
    DV = V.shape[-1]
    scale = 1.0 / math.sqrt(DQ)
    Qf, Kf, Vf = Q.to(acc), K.to(acc), V.to(acc)
    sc = torch.as_tensor(scores).to(acc)
    th = torch.as_tensor(thr).to(acc)
    ts = torch.arange(T) if rows is None else torch.as_tensor(rows, dtype=torch.long)
    out = torch.empty((B, len(ts), HQ, DV), dtype=acc)
    step = chunk or _chunk_rows(len(ts), B * HQ * T)
    for i0 in range(0, len(ts), step):
        tt = ts[i0:i0 + step]
        causal = torch.arange(T)[None, :] <= tt[:, None]                   # [c,T]
        sel = (sc[:, i0:i0 + step] >= th[:, i0:i0 + step]) & causal        # [B,c,T]
        logits = torch.einsum("bthd,bshd->bths", Qf[:, tt], Kf) * scale    # [B,c,HQ,T]
        logits = logits.masked_fill(~sel.unsqueeze(2), NEG_INF)
        attn = torch.softmax(logits, dim=-1)
        out[:, i0:i0 + step] = torch.einsum("bths,bshd->bthd", attn, Vf)
    return out


# ---------------------------------------------------------------------------
# Forward
# ---------------------------------------------------------------------------
def dsa_forward(q_idx, k_idx, w_idx, Q, K, V, top_k, *, acc=torch.float64, rows=None,
                return_parts=False):
    """dsa_attention_torch restated (dsa_attention.py:35-52): k_eff =
    min(top_k, T); threshold = k_eff-th largest of the full (-inf masked) row;
    keep scores >= threshold and s <= t; softmax attention over the kept keys.
    """
    T = Q.shape[1]
    scores = indexer_scores(q_idx, k_idx, w_idx, acc=acc, rows=rows)
    thr = topk_threshold(scores, min(top_k, T))
    out = sparse_attn_threshold(scores, thr, Q, K, V, acc=acc, rows=rows)
    if return_parts:
        return out, scores, thr
    return out


def dsa_forward_naive(q_idx, k_idx, w_idx, Q, K, V, top_k):
    """dsa_attention_naive restated (dsa_attention.py:59-89) in float64 loops."""
    qi, ki, wi = (np.asarray(x, dtype=np.float64) for x in (q_idx, k_idx, w_idx))
    Qn, Kn, Vn = (np.asarray(x, dtype=np.float64) for x in (Q, K, V))
    B, T, HQ, DQ = Qn.shape
    DV = Vn.shape[-1]
    scale = 1.0 / math.sqrt(DQ)
    out = np.zeros((B, T, HQ, DV))
    scores_all = indexer_scores_naive(qi, ki, wi)
    k_eff = min(top_k, T)
    for b in range(B):
        for t in range(T):
            row = scores_all[b, t]
            thresh = np.sort(row)[::-1][k_eff - 1]
            sel = [s for s in range(t + 1) if row[s] >= thresh]
            for h in range(HQ):
                lg = np.array([float(Qn[b, t, h] @ Kn[b, s, h]) * scale for s in sel])
                p = np.exp(lg - lg.max())
                p /= p.sum()
                out[b, t, h] = sum(p[i] * Vn[b, s, h] for i, s in enumerate(sel))
    return out
