"""Batch streaming: the split DSA forward over a sequence of batches.

The reference sketches this for its hybrid path (DEVLOG.md:207-210: overlap
the CPU top-K of batch i with the GPU indexer of batch i+1; "only matters in
batch-streaming inference").  That overlap, with the host select, is
dsa_hybrid.dsa_hybrid_stream.  With the whole forward on the GPU there is no
host stage to hide, and each kernel fills the MI355X by itself, so:

  * dsa_attention_stream (the default form) runs the batches one after
    another on the caller's stream with one reused score/threshold buffer;
  * DSAStreamGraph captures N batches into one HIP graph (no per-launch host
    cost: the form for serving loops of small batches);
  * DSAStreamPipeline overlaps batch i+1's indexer with batch i's select and
    attention on two streams.  Measured on MI355X it is slower than running
    the batches one after another (config 2: ~3x, from its per-batch host
    work; configs 3-4: no gain), so nothing here uses it by default.

DSAStreamPipeline: two HIP streams (default priority) and `depth`
score/threshold slots:
  indexer stream:    indexer(i) -> scores[i % depth]; event ready[i]
  attention stream:  wait ready[i]; select(i) -> thr[i % depth];
                     attention(i) -> out[i]; event done[i]
  indexer(i + depth) waits done[i] before it rewrites the slot.
Each batch's output is the split forward's (`dsa_split_hip`), bit for bit:
same kernels, same inputs, only the launch order across streams differs.
"""
from __future__ import annotations

import math

import torch

import _dsa_lib as L
from dsa_attention import sparse_attention_hip
from lightning_indexer import indexer_scores_hip
from topk_threshold import topk_threshold_into


def _refuse_capture(what: str) -> None:
    """The two-stream pipeline is eager only.  Capturing it into one graph
    crashed the host process inside the runtime's end of capture (cause not
    established), so a call made while the current stream is capturing is
    refused before it enqueues anything; DSAStreamGraph is the captured form
    (one stream)."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"DSAStreamPipeline.{what}: the two-stream pipeline cannot be "
                           "captured into a graph; use DSAStreamGraph (one stream)")


class DSAStreamPipeline:
    """Streams batches of one shape [B,T,...] through the split forward.

    submit(q_idx, k_idx, w_idx, Q, K, V) enqueues one batch and returns its
    output tensor [B,T,HQ,DV] fp32, valid once `synchronize()` (or an event
    recorded on `attention_stream` after it) has completed.  Inputs must
    stay alive and unchanged until then; the pipeline keeps a reference.
    submit() and join() raise RuntimeError while the current stream is
    being captured: the pipeline is not capturable.
    """

    def __init__(self, B: int, T: int, top_k: int, device="cuda", depth: int = 2):
        assert depth >= 1, "depth must be >= 1"
        assert top_k >= 1, "top_k must be >= 1"
        self.B, self.T, self.k = B, T, min(top_k, T)
        self.device = torch.device(device)
        self.depth = depth
        self.indexer_stream = torch.cuda.Stream(device=self.device)
        self.attention_stream = torch.cuda.Stream(device=self.device)
        self.scores = [torch.empty(B, T, T, device=self.device) for _ in range(depth)]
        self.thr = [torch.empty(B, T, 1, device=self.device) for _ in range(depth)]
        self._done = [None] * depth      # event: slot's last reader finished
        self._keep = []                  # inputs/outputs in flight
        self._n = 0

    def submit(self, q_idx, k_idx, w_idx, Q, K, V) -> torch.Tensor:
        _refuse_capture("submit")
        L.require_gpu(q_idx, k_idx, w_idx, Q, K, V)
        B, T = Q.shape[0], Q.shape[1]
        assert (B, T) == (self.B, self.T), f"batch shape {(B, T)} != pipeline {(self.B, self.T)}"
        slot = self._n % self.depth
        caller = torch.cuda.current_stream(self.device)
        ready = torch.cuda.Event()
        # inputs were produced on the caller's stream
        self.indexer_stream.wait_stream(caller)
        self.attention_stream.wait_stream(caller)
        with torch.cuda.stream(self.indexer_stream):
            if self._done[slot] is not None:
                self.indexer_stream.wait_event(self._done[slot])
            indexer_scores_hip(q_idx, k_idx, w_idx, write_upper=False, out=self.scores[slot])
            ready.record(self.indexer_stream)
        with torch.cuda.stream(self.attention_stream):
            self.attention_stream.wait_event(ready)
            topk_threshold_into(self.scores[slot], self.k, self.thr[slot], causal=True)
            out = torch.empty(B, T, Q.shape[2], V.shape[3], device=self.device)
            sparse_attention_hip(self.scores[slot], self.thr[slot], Q, K, V, out=out)
            done = torch.cuda.Event()
            done.record(self.attention_stream)
        self._done[slot] = done
        self._keep.append((q_idx, k_idx, w_idx, Q, K, V, out))
        self._n += 1
        return out

    def join(self) -> None:
        """Order the caller's stream after every submitted batch (no host
        wait).  Not valid under graph capture (see `_refuse_capture`)."""
        _refuse_capture("join")
        caller = torch.cuda.current_stream(self.device)
        caller.wait_stream(self.attention_stream)
        caller.wait_stream(self.indexer_stream)

    def synchronize(self) -> None:
        """Wait for every submitted batch; the caller's stream is ordered
        after them."""
        self.join()
        torch.cuda.synchronize(self.device)
        self._keep.clear()

    def reset(self) -> None:
        """Forget slot-reuse events of earlier submissions (after a
        synchronize)."""
        self._done = [None] * self.depth
        self._keep.clear()
        self._n = 0


class DSAStreamGraph:
    """The split forward of `nbatch` batches of one shape, captured once into
    a HIP graph over static buffers; `replay()` relaunches every kernel with
    no host work per launch.  For serving loops of small batches, where
    launching from Python costs more than the kernels (config 2: a split
    forward's three kernels take ~36 us eagerly).

    The batches are captured one after another on the capture stream.
    (Capturing the two-stream DSAStreamPipeline instead crashed the host
    process inside the runtime's end-of-capture, cause not established; that
    form is not offered.)

    Fill `inputs[i]` (q_idx, k_idx, w_idx, Q, K, V) in place, call
    `replay()`, read `outputs[i]` after the caller's stream has reached it.
    """

    def __init__(self, B: int, T: int, HI: int, DI: int, HQ: int, DQ: int, DV: int,
                 top_k: int, nbatch: int, dtype=torch.float32, device="cuda"):
        dev = torch.device(device)
        self.k = min(top_k, T)
        self.inputs = [
            (torch.zeros(B, T, HI, DI, device=dev, dtype=dtype),
             torch.zeros(B, T, DI, device=dev, dtype=dtype),
             torch.zeros(B, T, HI, device=dev, dtype=dtype),
             torch.zeros(B, T, HQ, DQ, device=dev, dtype=dtype),
             torch.zeros(B, T, HQ, DQ, device=dev, dtype=dtype),
             torch.zeros(B, T, HQ, DV, device=dev, dtype=dtype))
            for _ in range(nbatch)]
        self.scores = torch.empty(B, T, T, device=dev)
        self.thr = torch.empty(B, T, 1, device=dev)
        self.outputs = [torch.empty(B, T, HQ, DV, device=dev) for _ in range(nbatch)]
        # one eager pass first: library load and kernel attributes happen
        # outside the capture
        self._run()
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._run()

    def _run(self) -> None:
        for bt, out in zip(self.inputs, self.outputs):
            q_idx, k_idx, w_idx, Q, K, V = bt
            indexer_scores_hip(q_idx, k_idx, w_idx, write_upper=False, out=self.scores)
            topk_threshold_into(self.scores, self.k, self.thr, causal=True)
            sparse_attention_hip(self.scores, self.thr, Q, K, V, out=out)

    def replay(self) -> None:
        self.graph.replay()


def dsa_attention_stream(batches, top_k: int, depth: int | None = None):
    """Split forward over an iterable of (q_idx, k_idx, w_idx, Q, K, V)
    batches of one shape; returns the list of outputs (synchronised).

    Default: the batches one after another on the caller's stream, the score
    and threshold buffers allocated once and reused.  depth=N runs them on
    the two-stream DSAStreamPipeline with N slots instead (same outputs, bit
    for bit; slower on MI355X as measured, kept for experiments)."""
    outs = []
    if depth is not None:
        pipe = None
        for bt in batches:
            if pipe is None:
                pipe = DSAStreamPipeline(bt[3].shape[0], bt[3].shape[1], top_k,
                                         device=bt[3].device, depth=depth)
            outs.append(pipe.submit(*bt))
        if pipe is not None:
            pipe.synchronize()
        return outs
    scores = thr = None
    dev = None
    for bt in batches:
        q_idx, k_idx, w_idx, Q, K, V = bt
        L.require_gpu(q_idx, k_idx, w_idx, Q, K, V)
        B, T = Q.shape[0], Q.shape[1]
        if scores is None:
            dev = Q.device
            scores = torch.empty(B, T, T, device=dev)
            thr = torch.empty(B, T, 1, device=dev)
            k = min(top_k, T)
        assert scores.shape == (B, T, T), "dsa_attention_stream: batches must share one shape"
        indexer_scores_hip(q_idx, k_idx, w_idx, write_upper=False, out=scores)
        topk_threshold_into(scores, k, thr, causal=True)
        outs.append(sparse_attention_hip(scores, thr, Q, K, V))
    if dev is not None:
        torch.cuda.synchronize(dev)
    return outs
