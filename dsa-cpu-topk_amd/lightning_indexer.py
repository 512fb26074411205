"""DeepSeek-V3.2 lightning indexer on MI355X -- drop-in for the reference's
lightning_indexer.py (same names, arguments, return shapes and error classes).

    I[b,t,s] = sum_j w[b,t,j] * ReLU(<q[b,t,j,:], k[b,s,:]>)   for s <= t, -inf otherwise

    h   [B,T,D]   W_Q [D,H*d]   W_K [D,d]   W_W [D,H]   ->  scores [B,T,T] fp32

`indexer_scores_triton` / `indexer_triton` keep the reference's names so
callers switch without edits; they run the gfx950 MFMA kernel in
libdsa_amd.so (no Triton).  `indexer_scores_torch`, `project`,
`indexer_torch` are the reference's plain-torch functions, kept as API.
"""
from __future__ import annotations

import weakref
from collections import OrderedDict

import torch

import _dsa_lib as L


# ---------------------------------------------------------------------------
# Plain-torch functions of the reference API (lightning_indexer.py:26-47)
# ---------------------------------------------------------------------------
def indexer_scores_torch(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """q: [B,T,H,d]  k: [B,T,d]  w: [B,T,H] -> scores [B,T,T] (reference :26-33)."""
    B, T, H, d = q.shape
    dots = torch.einsum("bthd,bsd->bths", q, k)
    scores = (w.unsqueeze(-1) * torch.relu(dots)).sum(dim=2)
    causal = torch.ones(T, T, device=q.device, dtype=torch.bool).tril()
    return scores.masked_fill(~causal, float("-inf"))


def project(h: torch.Tensor, W_Q: torch.Tensor, W_K: torch.Tensor, W_W: torch.Tensor,
            num_heads: int, head_dim: int):
    """h@W projections to (q [B,T,H,d], k [B,T,d], w [B,T,H]) (reference :36-42)."""
    B, T, _ = h.shape
    q = (h @ W_Q).view(B, T, num_heads, head_dim)
    k = h @ W_K
    w = h @ W_W
    return q, k, w


def indexer_torch(h, W_Q, W_K, W_W, num_heads, head_dim):
    q, k, w = project(h, W_Q, W_K, W_W, num_heads, head_dim)
    return indexer_scores_torch(q, k, w)


# ---------------------------------------------------------------------------
# MI355X kernel (replaces _indexer_score_kernel + indexer_scores_triton, :54-125)
# ---------------------------------------------------------------------------
def indexer_scores_hip(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, *,
                       write_upper: bool = True, out: torch.Tensor | None = None,
                       q_scale: torch.Tensor | None = None,
                       k_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Indexer scores [B,T,T] fp32 from the gfx950 MFMA kernel.

    write_upper=False leaves the s > t triangle untouched (the split pipeline
    never reads it).  `out` may be a preallocated [B,T,T] fp32 buffer.

    q and k both torch.float8_e4m3fn select the fp8 MFMA kernel (E4M3
    operands, exact products, fp32 accumulation; w is taken as fp32), with
    optional positive quantisation scales q_scale [B,T,H] (per token and
    head) and k_scale [B,T] (per token): the scores are then those of the
    dequantised q_scale*q and k_scale*k (dsa_indexer_scores_fp8_scaled).
    The reference has no fp8 path: its kernel upcasts every load to fp32
    (lightning_indexer.py:81-91), which fp8 inputs match to fp32 rounding.
    """
    L.require_gpu(q, k, w)
    B, T, H, d = q.shape
    assert k.shape == (B, T, d), f"k shape {tuple(k.shape)} != {(B, T, d)}"
    assert w.shape == (B, T, H), f"w shape {tuple(w.shape)} != {(B, T, H)}"
    if q_scale is not None or k_scale is not None:
        assert q.dtype == torch.float8_e4m3fn and k.dtype == torch.float8_e4m3fn, \
            "quantisation scales go with fp8 (e4m3) q and k"
        if q_scale is not None:
            L.require_gpu(q_scale)
            assert q_scale.shape == (B, T, H), f"q_scale shape {tuple(q_scale.shape)} != {(B, T, H)}"
            q_scale = L.prep(q_scale, torch.float32)
        if k_scale is not None:
            L.require_gpu(k_scale)
            assert k_scale.numel() == B * T, f"k_scale must hold B*T = {B * T} values"
            k_scale = L.prep(k_scale.reshape(B, T), torch.float32)
        dt = torch.float8_e4m3fn
        q, k = L.prep(q, dt), L.prep(k, dt)
        w = L.prep(w, torch.float32)
        if out is None:
            out = torch.empty((B, T, T), device=q.device, dtype=torch.float32)
        else:
            assert out.shape == (B, T, T) and out.dtype == torch.float32 and out.is_contiguous()
        rc = L.lib().dsa_indexer_scores_fp8_scaled(
            q.data_ptr(), k.data_ptr(), w.data_ptr(),
            q_scale.data_ptr() if q_scale is not None else None,
            k_scale.data_ptr() if k_scale is not None else None,
            B, T, H, d, out.data_ptr(), T, 1 if write_upper else 0, L.stream_ptr(q.device))
        L.check(rc, "indexer_scores_fp8_scaled")
        return out
    if q.dtype == torch.float8_e4m3fn and k.dtype == torch.float8_e4m3fn:
        dt = torch.float8_e4m3fn
        q, k = L.prep(q, dt), L.prep(k, dt)
        w = L.prep(w, torch.float32)
    else:
        dt = L.common_dtype(q, k, w)
        q, k, w = (L.prep(x, dt) for x in (q, k, w))
    if out is None:
        out = torch.empty((B, T, T), device=q.device, dtype=torch.float32)
    else:
        assert out.shape == (B, T, T) and out.dtype == torch.float32 and out.is_contiguous()
    rc = L.lib().dsa_indexer_scores(q.data_ptr(), k.data_ptr(), w.data_ptr(), L.dtype_code(dt),
                                    B, T, H, d, out.data_ptr(), T, 1 if write_upper else 0,
                                    L.stream_ptr(q.device))
    L.check(rc, "indexer_scores")
    return out


def indexer_scores_triton(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor,
                          BLOCK_T: int = 64, BLOCK_S: int = 64) -> torch.Tensor:
    """Drop-in for the reference's indexer_scores_triton (:100-125).

    Same checks (GPU tensors, shapes, power-of-two head_dim) and output:
    fp32 [B,T,T], causal scores, -inf above the diagonal.  BLOCK_T/BLOCK_S
    are accepted for compatibility; the gfx950 kernel picks its own tiles.
    """
    assert q.is_cuda and k.is_cuda and w.is_cuda
    B, T, H, d = q.shape
    assert k.shape == (B, T, d)
    assert w.shape == (B, T, H)
    assert d > 0 and d & (d - 1) == 0, f"head_dim {d} must be power of 2"
    return indexer_scores_hip(q, k, w, write_upper=True)


class _ProjectionWeightCache:
    """Concatenated projection weights [W_Q | W_K | W_W | 0-pad], one entry
    per set of weight tensors.

    An entry is keyed on the identity of the three tensor objects and is
    valid only while all three are alive (weak references), still hold the
    same storage (data_ptr, shape, strides) and have not been modified in
    place (`_version`).  A freed tensor's address can be handed to a new
    tensor, so an address alone never identifies a weight: a new tensor is a
    miss even when it lands where an old one lived.  An entry is dropped as
    soon as one of its weights is garbage collected; at most `capacity`
    entries (least recently used first out) are kept, e.g. one per layer.
    """

    def __init__(self, capacity: int = 64):
        self.capacity = capacity
        self._entries: "OrderedDict[tuple, tuple]" = OrderedDict()

    @staticmethod
    def _state(W: torch.Tensor) -> tuple:
        return (W.data_ptr(), W._version, tuple(W.shape), W.stride(), W.dtype, W.device)

    def get(self, W_Q, W_K, W_W, dtype) -> torch.Tensor:
        ws = (W_Q, W_K, W_W)
        key = (id(W_Q), id(W_K), id(W_W), dtype)
        hit = self._entries.get(key)
        if hit is not None:
            refs, states, wc = hit
            if all(r() is W for r, W in zip(refs, ws)) and \
                    states == tuple(self._state(W) for W in ws):
                self._entries.move_to_end(key)
                return wc
            del self._entries[key]
        wc = fuse_projection_weights(W_Q, W_K, W_W, dtype)
        entries = self._entries

        def _drop(dead, key=key):
            # a weight of this entry was collected: the entry can never hit again
            e = entries.get(key)
            if e is not None and any(r is dead for r in e[0]):
                del entries[key]

        refs = tuple(weakref.ref(W, _drop) for W in ws)
        self._entries[key] = (refs, tuple(self._state(W) for W in ws), wc)
        while len(self._entries) > self.capacity:
            self._entries.popitem(last=False)
        return wc

    def clear(self) -> None:
        self._entries.clear()

    def __len__(self) -> int:
        return len(self._entries)


def fuse_projection_weights(W_Q, W_K, W_W, dtype=None) -> torch.Tensor:
    """[W_Q | W_K | W_W | 0-pad] as one [D, n_pad] matrix in `dtype` (default:
    the weights' common dtype).  The zero columns pad each row of the
    projection output to a 16-byte multiple, and 16-bit weights to a multiple
    of 256 columns (measured on MI355X at D=2048, HI=64, DI=128 bf16: the
    GEMM with 8448 columns takes 125.9 us against 133.4 us with 8384; fp32
    at D=1024, HI=4, DI=32 is faster unpadded, 31.7 against 35.1 us).  Pass
    the result as `W_cat` to indexer_from_hidden to skip the per-call cache
    lookup."""
    if dtype is None:
        dtype = L.common_dtype(W_Q, W_K, W_W)
    D = W_Q.shape[0]
    n = W_Q.shape[1] + W_K.shape[1] + W_W.shape[1]
    es = torch.tensor([], dtype=dtype).element_size()
    per = 256 if es == 2 else 16 // es
    n_pad = (n + per - 1) // per * per
    wc = torch.zeros(D, n_pad, device=W_Q.device, dtype=dtype)
    wc[:, :n].copy_(torch.cat([W_Q, W_K, W_W], dim=1))
    return wc


_WCAT_CACHE = _ProjectionWeightCache()


def _fused_weights(W_Q, W_K, W_W, dtype):
    """The cached concatenation of one set of projection weights."""
    return _WCAT_CACHE.get(W_Q, W_K, W_W, dtype)


def indexer_from_hidden(h, W_Q, W_K, W_W, num_heads, head_dim, *,
                        write_upper: bool = True,
                        W_cat: torch.Tensor | None = None) -> torch.Tensor:
    """Projection front end fused into the indexer's input stage: ONE GEMM
    h @ [W_Q | W_K | W_W] (hipBLASLt via torch) writes every token's q, k and
    w side by side, and the MFMA indexer reads them in place through row
    strides (dsa_indexer_scores_strided) -- no split, no copies.  Same result
    as project() + indexer_scores_hip (reference lightning_indexer.py:36-47,
    128-130).

    W_cat: the concatenated weights from fuse_projection_weights (optional;
    without it the concatenation is looked up in, or added to, a cache keyed
    on the weight tensors' identity and in-place version)."""
    L.require_gpu(h, W_Q, W_K, W_W)
    B, T, D = h.shape
    H, d = num_heads, head_dim
    assert W_Q.shape == (D, H * d) and W_K.shape == (D, d) and W_W.shape == (D, H), \
        "projection weight shapes"
    dt = L.common_dtype(h, W_Q, W_K, W_W)
    if W_cat is None:
        wc = _fused_weights(W_Q, W_K, W_W, dt)
    else:
        n = H * d + d + H
        assert W_cat.shape[0] == D and W_cat.shape[1] >= n and W_cat.dtype == dt \
            and W_cat.is_contiguous() and (W_cat.shape[1] * W_cat.element_size()) % 16 == 0, \
            "W_cat must be fuse_projection_weights(W_Q, W_K, W_W) in the inputs' dtype"
        wc = W_cat
    y = L.prep(h, dt).reshape(B * T, D) @ wc          # [B*T, n_pad]
    ldr = y.shape[1]
    out = torch.empty((B, T, T), device=h.device, dtype=torch.float32)
    base = y.data_ptr()
    es = y.element_size()
    rc = L.lib().dsa_indexer_scores_strided(
        base, base + H * d * es, base + (H * d + d) * es, L.dtype_code(dt), B, T, H, d,
        ldr, ldr, ldr, out.data_ptr(), T, 1 if write_upper else 0, L.stream_ptr(h.device))
    L.check(rc, "indexer_from_hidden")
    return out


def indexer_triton(h, W_Q, W_K, W_W, num_heads, head_dim, **kw):
    """Drop-in for the reference's indexer_triton (:128-130): the projection
    as one fused GEMM read in place by the MFMA indexer (indexer_from_hidden).
    BLOCK_T/BLOCK_S keywords are accepted for compatibility."""
    assert head_dim > 0 and head_dim & (head_dim - 1) == 0, f"head_dim {head_dim} must be power of 2"
    return indexer_from_hidden(h, W_Q, W_K, W_W, num_heads, head_dim)


# ---------------------------------------------------------------------------
# Top-k mask helper (reference :137-144)
# ---------------------------------------------------------------------------
def topk_mask(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Boolean [B,T,T] mask of the top-k key positions of every query row.

    Built from the radix-select's exactly-k index set: the lowest index wins
    ties, so the mask is deterministic (the reference took torch.topk's
    indices, whose tie order is unspecified).  GPU tensors only.
    """
    from topk_threshold import topk_indices

    L.require_gpu(scores)
    B, T, _ = scores.shape
    _, idx = topk_indices(scores, min(k, T))
    mask = torch.zeros_like(scores, dtype=torch.bool)
    mask.scatter_(-1, idx.long(), True)
    return mask
