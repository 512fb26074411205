"""DSA forward with the top-K threshold offloaded to the host CPU -- drop-in
for the reference's dsa_hybrid.py (HybridContext, dsa_hybrid_cpu_topk;
reference dsa_hybrid.py:36-66), the experiment the reference was built for.

Pipeline, as the reference runs it:
  1. GPU: lightning indexer -> scores [B,T,T] fp32 (-inf above the diagonal)
  2. d2h into pinned host memory, then wait for it
  3. CPU: k-th largest of every row -> threshold [B,T,1], written into the
     pinned thr_cpu buffer (the reference allocates a new tensor each call
     and never uses its thr_cpu)
  4. h2d of the thresholds
  5. GPU: sparse attention with the threshold as an input
The GPU stages are the gfx950 kernels of libdsa_amd.so; the CPU stage is
libdsa_cpu.so (AVX-512 scan + vector quickselect on OpenMP threads), the
same contract as the reference's topk_avx512 extension.

Beyond the reference:
  * chunks > 1 splits the d2h into row blocks with an event after each, and
    the host selects each block as soon as it lands, so the copy of block
    j+1 overlaps the select of block j;
  * causal=True has the host read only the s <= t entries of each row (the
    result is the full-row one: the indexer writes -inf above the diagonal);
  * dsa_hybrid_stream overlaps the host select of batch i with the GPU
    indexer and d2h of batch i+1 (the batch-streaming case the reference
    notes in DEVLOG.md:207-210).

On MI355X the GPU radix-select of the same rows is tens of times faster than
the PCIe round trip alone; this path exists to run the reference's
experiment on this hardware, not as the default forward.
"""
from __future__ import annotations

import torch

import _dsa_lib as L
from dsa_attention import sparse_attention_hip
from lightning_indexer import indexer_scores_hip


def _check_like_reference(q_idx, Q, V, top_k):
    """The checks the reference's path makes before any work: power-of-two
    DI (indexer_scores_triton, lightning_indexer.py:107-108) and T, HQ, DQ,
    DV (sparse_attention_with_threshold_triton, dsa_attention.py:303-304) as
    AssertionError; k <= N (the extension's TORCH_CHECK) as RuntimeError."""
    T = Q.shape[1]
    for n, v in (("DI", q_idx.shape[3]), ("T", T), ("HQ", Q.shape[2]), ("DQ", Q.shape[3]),
                 ("DV", V.shape[3])):
        assert v > 0 and v & (v - 1) == 0, f"{n}={v} must be a power of 2"
    if not 0 < top_k <= T:
        raise RuntimeError(f"topk_threshold: k must be > 0 and <= N (k={top_k}, N={T})")


class HybridContext:
    """Reusable buffers of one batch shape (reference dsa_hybrid.py:36-43):
    pinned host scores_cpu [B,T,T] and thr_cpu [B,T,1], and on the GPU
    thr_gpu [B,T,1] and scores_gpu [B,T,T] (the indexer's output)."""

    def __init__(self, B, T, device="cuda"):
        self.B, self.T = B, T
        dev = torch.device(device)
        self.device = dev
        self.scores_cpu = torch.empty((B, T, T), dtype=torch.float32, pin_memory=True)
        self.thr_cpu = torch.empty((B, T, 1), dtype=torch.float32, pin_memory=True)
        self.thr_gpu = torch.empty((B, T, 1), dtype=torch.float32, device=dev)
        self.scores_gpu = torch.empty((B, T, T), dtype=torch.float32, device=dev)


def _row_blocks(rows: int, chunks: int):
    chunks = max(1, min(int(chunks), rows))
    step = -(-rows // chunks)
    return [(r0, min(rows, r0 + step)) for r0 in range(0, rows, step)]


def _host_select(ctx: HybridContext, r0: int, r1: int, k: int, causal: bool,
                 nthreads: int) -> None:
    """k-th largest of host rows r0..r1 of ctx.scores_cpu into ctx.thr_cpu."""
    T = ctx.T
    lib = L.cpu_lib()
    base = ctx.scores_cpu.data_ptr() + r0 * T * 4
    rc = lib.dsa_cpu_topk_threshold(base, r1 - r0, T, T, int(k), T if causal else 0, r0,
                                    ctx.thr_cpu.data_ptr() + r0 * 4, int(nthreads))
    if rc != 0:
        raise RuntimeError(f"topk_threshold: {lib.dsa_cpu_last_error().decode(errors='replace')}")


def _enqueue_scores_d2h(ctx: HybridContext, q_idx, k_idx, w_idx, chunks: int, stream):
    """Indexer into ctx.scores_gpu, then the d2h of its row blocks, one event
    after each block (all on `stream`)."""
    B, T = ctx.B, ctx.T
    indexer_scores_hip(q_idx, k_idx, w_idx, write_upper=True, out=ctx.scores_gpu)
    src = ctx.scores_gpu.view(B * T, T)
    dst = ctx.scores_cpu.view(B * T, T)
    blocks = []
    for r0, r1 in _row_blocks(B * T, chunks):
        dst[r0:r1].copy_(src[r0:r1], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        blocks.append((r0, r1, ev))
    return blocks


def _finish(ctx: HybridContext, blocks, k: int, causal: bool, nthreads: int, Q, K, V,
            out=None):
    """Host select of each block once its copy has landed, h2d of the
    thresholds, and the GPU attention (enqueued on the current stream)."""
    for r0, r1, ev in blocks:
        ev.synchronize()
        _host_select(ctx, r0, r1, k, causal, nthreads)
    ctx.thr_gpu.copy_(ctx.thr_cpu, non_blocking=True)
    return sparse_attention_hip(ctx.scores_gpu, ctx.thr_gpu, Q, K, V, out=out)


def dsa_hybrid_cpu_topk(q_idx, k_idx, w_idx, Q, K, V, top_k: int,
                        ctx: HybridContext | None = None, *, chunks: int = 1,
                        causal: bool = False, nthreads: int = 0) -> torch.Tensor:
    """Indexer (GPU) -> pinned d2h -> k-th largest of every row (host CPU) ->
    h2d -> sparse attention with the threshold as an input (GPU); reference
    dsa_hybrid.py:46-66.  Returns O [B,T,HQ,DV] fp32, equal to the split
    forward's (the host and GPU selects give bit-identical thresholds).

    top_k must be <= T (the extension's k <= N check, RuntimeError).
    chunks / causal / nthreads: see the module docstring; the defaults run
    the reference's pipeline step for step (full rows, one copy, then wait).
    """
    L.require_gpu(q_idx, k_idx, w_idx, Q, K, V)
    B, T = Q.shape[0], Q.shape[1]
    _check_like_reference(q_idx, Q, V, top_k)
    if ctx is None:
        ctx = HybridContext(B, T, device=Q.device)
    assert ctx.B == B and ctx.T == T
    stream = torch.cuda.current_stream(Q.device)
    blocks = _enqueue_scores_d2h(ctx, q_idx, k_idx, w_idx, chunks, stream)
    return _finish(ctx, blocks, top_k, causal, nthreads, Q, K, V)


def dsa_hybrid_stream(batches, top_k: int, *, chunks: int = 1, causal: bool = True,
                      nthreads: int = 0):
    """The CPU-offload forward over an iterable of (q_idx, k_idx, w_idx, Q, K,
    V) batches of one shape, with the host select of batch i running while
    the GPU computes the indexer scores of batch i+1 and copies them out.

    Two contexts alternate.  Order on the one stream: indexer(i+1), d2h(i+1),
    then h2d(i), attention(i); the host selects batch i between enqueueing
    batch i+1's copies and batch i's attention.  Buffer reuse is safe by that
    order: batch i+2's d2h into a context is enqueued after the host has
    finished reading it, and the host writes a context's thr_cpu only after
    waiting for a copy enqueued after that context's previous h2d.
    Returns the outputs (the stream is synchronised at the end).
    """
    outs = []
    ctxs = []
    pending = None  # (ctx, blocks, Q, K, V, out)
    stream = None
    for i, bt in enumerate(batches):
        q_idx, k_idx, w_idx, Q, K, V = bt
        L.require_gpu(q_idx, k_idx, w_idx, Q, K, V)
        B, T = Q.shape[0], Q.shape[1]
        if not ctxs:
            _check_like_reference(q_idx, Q, V, top_k)
            ctxs = [HybridContext(B, T, device=Q.device) for _ in range(2)]
            stream = torch.cuda.current_stream(Q.device)
        ctx = ctxs[i % 2]
        assert (ctx.B, ctx.T) == (B, T), "dsa_hybrid_stream: batches must share one shape"
        blocks = _enqueue_scores_d2h(ctx, q_idx, k_idx, w_idx, chunks, stream)
        out = torch.empty(B, T, Q.shape[2], V.shape[3], device=Q.device, dtype=torch.float32)
        if pending is not None:
            _finish(*pending[:2], top_k, causal, nthreads, *pending[2:5], out=pending[5])
        pending = (ctx, blocks, Q, K, V, out)
        outs.append(out)
    if pending is not None:
        _finish(*pending[:2], top_k, causal, nthreads, *pending[2:5], out=pending[5])
        stream.synchronize()
    return outs
