"""Benchmark: DSA forward on one MI355X at BASELINE.json's headline config.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--mode graph|eager]

Workload: B=16, T=512, k=32, HI=4, DI=32, HQ=4, DQ=DV=32, fp32,
synthetic N(0,1) inputs (w ~ N(0,1)/sqrt(HI)) resident in HBM before timing.
A step is one fused DSA forward (indexer -> radix-select -> sparse attention,
one kernel).  Prints ONE JSON line:

  value        query tokens/s over the K timed steps (B*T*K / seconds)
  roofline     the fused kernel: algorithmic fp32 FLOPs per launch / its
               average duration (HIP events on the stream it runs on, around
               the K back-to-back launches of the graph), against the fp32
               MFMA peak (157.3 TFLOP/s)
  topk_select  the radix-select at config 4's shape (T=16384, k=2048, causal
               rows of real config-4 indexer scores): algorithmic bytes
               4*sum(t+1) (+ outputs) / duration, against 8 TB/s
  split        the split forward (indexer, select, attention) at config 1
  sweep_c2     fused and split forwards over config 2's (B, k) sweep at T=512,
               beside the reference's published fused Triton times there
  split_c3/c4  the split forward at configs 3 (fp32) and 4 (bf16), per stage
  projection   the indexer's projection front end (one GEMM + strided entry
               vs three GEMMs)
  stream       batches of configs 2-4 one after another, two-stream
               pipelined, and captured in one HIP graph
  cpu_baseline the reference's CPU path restated (oracle/, torch-vectorised
               fp32 forward) on the host cores, plus the AVX-512 k-th-largest
               (the reference's own topk_avx512.cpp from oracle/_ref when it
               was built and the host has AVX-512, else this repo's port)

--mode graph (default) replays the K steps from one HIP graph, so the Python
launch path is out of the timed region; every kernel still runs every step.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "dsa-cpu-topk_amd")]

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, vendor figure
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix, vendor figure
BASELINE_MS = 5.62             # reference fused Triton forward, README.md:49 (RTX PRO 6000)

C1 = dict(B=16, T=512, k=32, HI=4, DI=32, HQ=4, DQ=32, DV=32)
C4 = dict(B=1, T=16384, k=2048, HI=64, DI=128, HQ=16, DQ=128, DV=128)
C2 = dict(B=4, T=512, k=64, HI=4, DI=32, HQ=4, DQ=32, DV=32)  # smallest config-2 batch


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def indexer_flops(B, T, HI, DI):
    return B * T * (T + 1) / 2 * HI * (2 * DI + 2)


def attention_flops(B, T, k, HQ, DQ, DV):
    sel = sum(min(k, t + 1) for t in range(T))
    return B * sel * HQ * (2 * DQ + 2 * DV)


def gpu_inputs(cfg, dtype, dev, seed=0):
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    B, T, HI, DI, HQ, DQ, DV = (cfg[x] for x in ("B", "T", "HI", "DI", "HQ", "DQ", "DV"))

    def rn(*shape, s=1.0):
        return (torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * s).to(dtype)

    return (rn(B, T, HI, DI), rn(B, T, DI), rn(B, T, HI, s=1.0 / math.sqrt(HI)),
            rn(B, T, HQ, DQ), rn(B, T, HQ, DQ), rn(B, T, HQ, DV))


def warm(fn, seconds=0.25):
    """Run fn() back to back for about `seconds` of wall time before a timed
    region: the GPU's clocks settle under sustained load (the first tens of
    milliseconds of a burst run measurably slower)."""
    import time

    import torch

    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def time_events(fn, reps, stream):
    """Mean duration (s) of fn() over reps back-to-back calls: HIP events on
    `stream` (the stream the kernels are launched on) around the batch, so
    the host-side launch path overlaps the GPU work and the figure is the
    kernels' average duration."""
    import torch

    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps / 1e3


def bench_fused(args, dev):
    import torch

    import dsa_attention as D

    ins = gpu_inputs(C1, torch.float32, dev)
    k = C1["k"]
    fwd = lambda: D.dsa_fused_hip(*ins, k)  # noqa: E731
    for _ in range(args.warmup):
        fwd()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)

    if args.mode == "graph":
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(args.steps):
                fwd()
        graph.replay()                 # warm the graph once (untimed)
        torch.cuda.synchronize()
        # HIP events on the stream the graph's kernels run on: K back-to-back
        # launches, so elapsed / K is the kernel's average launch duration.
        stream = torch.cuda.current_stream(dev)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        graph.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
        kern_s = ev0.elapsed_time(ev1) / 1e3 / args.steps
        t0 = time.perf_counter()
        graph.replay()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    else:
        kern_s = time_events(fwd, max(20, min(args.steps, 200)), stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fwd()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    return elapsed, kern_s


def bench_split(dev, reps=50):
    import torch

    import dsa_attention as D

    ins = gpu_inputs(C1, torch.float32, dev, seed=1)
    fwd = lambda: D.dsa_split_hip(*ins, C1["k"])  # noqa: E731
    for _ in range(5):
        fwd()
    return time_events(fwd, reps, torch.cuda.current_stream(dev))


# Config 2 sweep at T=512 with the reference's published fused Triton times
# on its own GPU (README.md:50-54; RTX PRO 6000 Blackwell).
C2_SWEEP = ((4, 64, 1.34), (16, 64, 5.66), (16, 128, 5.67), (32, 64, 11.98), (64, 64, 25.96))


def bench_sweep_c2(dev, reps=50):
    """Fused and split forwards over the config-2 (B, k) sweep."""
    import torch

    import dsa_attention as D

    stream = torch.cuda.current_stream(dev)
    res = []
    for B, k, ref_ms in C2_SWEEP:
        cfg = dict(C1, B=B, k=k)
        ins = gpu_inputs(cfg, torch.float32, dev, seed=B + k)
        fused = lambda: D.dsa_fused_hip(*ins, k)  # noqa: E731
        split = lambda: D.dsa_split_hip(*ins, k)  # noqa: E731
        warm(fused, 0.1)
        tf = time_events(fused, reps, stream)
        warm(split, 0.1)
        ts = time_events(split, reps, stream)
        res.append({"B": B, "T": cfg["T"], "k": k,
                    "fused_ms": round(tf * 1e3, 4), "split_ms": round(ts * 1e3, 4),
                    "fused_query_tokens_per_s": round(B * cfg["T"] / tf, 1),
                    "reference_fused_ms": ref_ms, "speedup_vs_reference": round(ref_ms / (tf * 1e3), 1)})
        del ins
    return res


C3 = dict(B=4, T=4096, k=256, HI=8, DI=64, HQ=8, DQ=64, DV=64)


def bench_split_long(dev, cfg, dtype, name, reps, fp8_indexer=False):
    """Split forward at a long-row config: indexer (causal half), causal
    radix-select, attention (the tile kernel where it applies), each stage
    timed with HIP events on the stream it runs on."""
    import torch

    import _dsa_lib as L
    from dsa_attention import sparse_attention_from_mask, sparse_attention_hip
    from lightning_indexer import indexer_scores_hip
    from topk_threshold import topk_threshold_into, topk_threshold_mask

    B, T, k = cfg["B"], cfg["T"], cfg["k"]
    ins = gpu_inputs(cfg, dtype, dev, seed=3)
    stream = torch.cuda.current_stream(dev)
    scores = torch.empty(B, T, T, device=dev)
    thr = torch.empty(B, T, 1, device=dev)
    out = torch.empty(B, T, cfg["HQ"], cfg["DV"], device=dev)
    ix = lambda: indexer_scores_hip(*ins[:3], write_upper=False, out=scores)  # noqa: E731
    # The stages as dsa_split_hip runs them: where the attention runs on
    # tiles from a bitmask, the select writes that bitmask in its own pass.
    uses_mask = bool(L.lib().dsa_sparse_attn_uses_mask(L.dtype_code(dtype), T, cfg["HQ"],
                                                       cfg["DQ"], cfg["DV"]))
    if uses_mask:
        mask = torch.empty(B, T, (T + 63) // 64, device=dev, dtype=torch.int64)
        sel = lambda: topk_threshold_mask(scores, min(k, T), thr=thr, mask=mask)  # noqa: E731
        att = lambda: sparse_attention_from_mask(mask, *ins[3:], out=out)  # noqa: E731
    else:
        sel = lambda: topk_threshold_into(scores, min(k, T), thr, causal=True)  # noqa: E731
        att = lambda: sparse_attention_hip(scores, thr, *ins[3:], out=out)  # noqa: E731

    def fwd():
        ix()
        sel()
        att()

    warm(fwd)
    t_ix = time_events(ix, reps, stream)
    t_sel = time_events(sel, reps, stream)
    t_att = time_events(att, reps, stream)
    t_fwd = time_events(fwd, reps, stream)
    idx_fl = indexer_flops(B, T, cfg["HI"], cfg["DI"])
    res = {"workload": f"{name}: split forward B={B},T={T},k={k},HI={cfg['HI']},DI={cfg['DI']},"
                       f"HQ={cfg['HQ']},DQ=DV={cfg['DQ']} {str(dtype).replace('torch.', '')}",
           "ms_per_forward": round(t_fwd * 1e3, 4),
           "query_tokens_per_s": round(B * T / t_fwd, 1),
           "indexer_ms": round(t_ix * 1e3, 4),
           "indexer_TFLOP_per_s": round(idx_fl / t_ix / 1e12, 1),
           "select_ms": round(t_sel * 1e3, 4),
           "select_GB_per_s": round((4.0 * B * T * (T + 1) / 2 + 4.0 * B * T) / t_sel / 1e9, 1),
           "attention_ms": round(t_att * 1e3, 4),
           "select_writes_selection_bitmask": uses_mask}
    if fp8_indexer:
        # the same indexer on e4m3 q_idx/k_idx (w fp32): informational, the
        # split forward above runs the input dtype
        q8, k8 = (x.to(torch.float8_e4m3fn) for x in ins[:2])
        w32 = ins[2].float()
        ix8 = lambda: indexer_scores_hip(q8, k8, w32, write_upper=False, out=scores)  # noqa: E731
        warm(ix8)
        t_ix8 = time_events(ix8, reps, stream)
        res["indexer_fp8_ms"] = round(t_ix8 * 1e3, 4)
        res["indexer_fp8_TFLOP_per_s"] = round(idx_fl / t_ix8 / 1e12, 1)
        # with per-(token, head) q scales and per-token k scales
        qs = torch.rand(B, T, cfg["HI"], device=dev) + 0.5
        ks = torch.rand(B, T, device=dev) + 0.5
        ix8s = lambda: indexer_scores_hip(q8, k8, w32, write_upper=False, out=scores,  # noqa: E731
                                          q_scale=qs, k_scale=ks)
        warm(ix8s)
        t_ix8s = time_events(ix8s, reps, stream)
        res["indexer_fp8_scaled_ms"] = round(t_ix8s * 1e3, 4)
        del q8, k8, w32, qs, ks
    del ins, scores, thr, out
    return res


def bench_stream(dev, cfg, dtype, name, nbatch=4, reps=3):
    """Batch streaming (dsa_stream.py): nbatch batches through the split
    forward one after another, and through the two-stream pipeline that
    overlaps each batch's indexer with the previous batch's select and
    attention.  Informational: query tokens/s of each."""
    import torch

    from dsa_attention import dsa_split_hip
    from dsa_stream import DSAStreamPipeline

    B, T, k = cfg["B"], cfg["T"], cfg["k"]
    batches = [gpu_inputs(cfg, dtype, dev, seed=20 + i) for i in range(nbatch)]
    pipe = DSAStreamPipeline(B, T, k, device=dev)

    def sequential():
        for bt in batches:
            dsa_split_hip(*bt, k)

    def streamed():
        for bt in batches:
            pipe.submit(*bt)
        pipe.synchronize()

    import time

    res = {}
    for leg, fn in (("sequential", sequential), ("streamed", streamed)):
        warm(fn)
        best = float("inf")
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
        res[leg + "_ms"] = round(best * 1e3, 3)
        res[leg + "_query_tokens_per_s"] = round(nbatch * B * T / best, 1)
    # the batches captured once into a HIP graph over static buffers (one stream)
    from dsa_stream import DSAStreamGraph

    sg = DSAStreamGraph(B, T, cfg["HI"], cfg["DI"], cfg["HQ"], cfg["DQ"], cfg["DV"], k, nbatch,
                        dtype=dtype, device=dev)
    for dst, src in zip(sg.inputs, batches):
        for d_, s_ in zip(dst, src):
            d_.copy_(s_)
    warm(sg.replay)
    stream = torch.cuda.current_stream(dev)
    t_g = time_events(sg.replay, max(reps, 5), stream)
    res["graph_ms"] = round(t_g * 1e3, 3)
    res["graph_query_tokens_per_s"] = round(nbatch * B * T / t_g, 1)
    res["workload"] = (f"{name} x {nbatch} batches, split forward: one after another (eager), "
                       "two-stream pipeline (indexer of batch i+1 during select+attention of i), "
                       "and the batches captured in one HIP graph on one stream")
    del batches, pipe, sg
    return res


def time_reference_style(fn, stream, warmup=5, iters=20):
    """The reference's timing (bench_hybrid.py:26-37): warm-up calls, then
    HIP events on the stream around `iters` Python calls; ms per call.  Host
    work inside fn (launch path, host waits) is inside the figure."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(iters):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


# The reference's published end-to-end table (README.md:49-55): GPU fused
# and CPU hybrid ms on its RTX PRO 6000 + Ryzen 9 9950X3D.
REF_HYBRID = {(16, 512, 32): (5.62, 4.68), (16, 512, 64): (5.66, 5.47), (32, 512, 64): (11.98, 11.72),
              (64, 512, 64): (25.96, 24.97), (16, 512, 128): (5.67, 8.39), (4, 512, 64): (1.34, 1.56),
              (16, 128, 16): (0.10, 0.20)}


def bench_hybrid(dev):
    """The reference's experiment (bench_hybrid.py:40-53, dsa_hybrid.py:46-66)
    on this box: the whole CPU-offload forward -- GPU indexer, pinned d2h, host
    k-th largest (libdsa_cpu.so), h2d, GPU attention -- against the all-GPU
    fused and split forwards, each timed the reference's way (events around
    Python calls).  `hybrid` is the reference's pipeline step for step;
    `hybrid_pipelined` copies in 4 row blocks and selects each block as it
    lands, reading only the causal half of each row."""
    import torch

    import dsa_attention as D
    from dsa_hybrid import HybridContext, dsa_hybrid_cpu_topk, dsa_hybrid_stream

    stream = torch.cuda.current_stream(dev)
    rows = []
    # config 1, the config-2 sweep, and the reference's T=128 row (README.md:55)
    for B, T, k in ([(C1["B"], C1["T"], C1["k"])] + [(b, C1["T"], kk) for b, kk, _ in C2_SWEEP]
                    + [(16, 128, 16)]):
        cfg = dict(C1, B=B, T=T, k=k)
        ins = gpu_inputs(cfg, torch.float32, dev, seed=B + k)
        ctx = HybridContext(B, cfg["T"], device=dev)
        hyb = dsa_hybrid_cpu_topk(*ins, k, ctx=ctx)
        equal = bool(torch.equal(hyb, D.dsa_split_hip(*ins, k)))
        legs = {
            "fused_ms": lambda: D.dsa_attention_triton(*ins, top_k=k),
            "split_ms": lambda: D.dsa_attention_split_triton(*ins, top_k=k),
            "hybrid_ms": lambda: dsa_hybrid_cpu_topk(*ins, k, ctx=ctx),
            "hybrid_pipelined_ms": lambda: dsa_hybrid_cpu_topk(*ins, k, ctx=ctx, chunks=4,
                                                               causal=True),
        }
        row = {"B": B, "T": cfg["T"], "k": k, "hybrid_equals_split": equal}
        if (B, T, k) in REF_HYBRID:
            row["reference_fused_ms"], row["reference_hybrid_ms"] = REF_HYBRID[(B, T, k)]
        for name, fn in legs.items():
            row[name] = round(time_reference_style(fn, stream), 4)
        rows.append(row)
        del ins, ctx, hyb
    # batch streaming of the hybrid path: config 2 (B=4, k=64) x 16 batches
    nb = 16
    batches = [gpu_inputs(C2, torch.float32, dev, seed=40 + i) for i in range(nb)]
    ctx = HybridContext(C2["B"], C2["T"], device=dev)

    def one_by_one():
        for bt in batches:
            dsa_hybrid_cpu_topk(*bt, C2["k"], ctx=ctx, causal=True)
        torch.cuda.synchronize()

    streamed = lambda: dsa_hybrid_stream(batches, C2["k"], causal=True)  # noqa: E731
    res = {"workload": "CPU-offload DSA forward (host k-th largest) vs all-GPU, config 1 and "
                       "the config-2 sweep (T=512, fp32); ms per forward, events around "
                       "Python calls as bench_hybrid.py times them",
           "host_isa": "avx512" if __import__("_dsa_lib").cpu_lib().dsa_cpu_isa() else "scalar",
           "host_threads": int(os.environ.get("OMP_NUM_THREADS", "0")) or
           len(os.sched_getaffinity(0)),
           "rows": rows}
    t_seq = time_reference_style(one_by_one, stream, warmup=1, iters=3)
    t_str = time_reference_style(streamed, stream, warmup=1, iters=3)
    res["stream_c2x16"] = {"one_by_one_ms": round(t_seq, 3), "streamed_ms": round(t_str, 3),
                           "note": "host select of batch i during the GPU indexer + d2h of "
                                   "batch i+1 (dsa_hybrid_stream)"}
    return res


def bench_eager_latency(dev):
    """Per-call latency of the drop-ins at config 1 as the reference measures
    its own (bench_hybrid.py:26-37: 5 warm-up calls, events around 20 Python
    calls), launch path included."""
    import torch

    import dsa_attention as D

    ins = gpu_inputs(C1, torch.float32, dev)
    stream = torch.cuda.current_stream(dev)
    k = C1["k"]
    return {"dsa_attention_triton_ms": round(time_reference_style(
                lambda: D.dsa_attention_triton(*ins, top_k=k), stream), 4),
            "dsa_attention_split_triton_ms": round(time_reference_style(
                lambda: D.dsa_attention_split_triton(*ins, top_k=k), stream), 4),
            "method": "5 warm-up calls, HIP events around 20 Python calls (bench_hybrid.py:26-37)"}


def bench_projection(dev, reps=20):
    """Projection front end (informational): three projection GEMMs + the
    indexer (the reference's indexer_triton structure) against one fused
    GEMM read in place by the strided indexer (indexer_from_hidden)."""
    import torch

    from lightning_indexer import indexer_from_hidden, indexer_scores_hip, project

    res = []
    for (B, T, D, H, d, dt) in [(2, 96, 128, 4, 64, torch.float32),
                                (16, 512, 1024, 4, 32, torch.float32),
                                (1, 4096, 2048, 64, 128, torch.bfloat16)]:
        g = torch.Generator(device=dev).manual_seed(0)
        h = torch.randn(B, T, D, generator=g, device=dev).to(dt)
        Ws = [(torch.randn(D, n, generator=g, device=dev) * 0.03).to(dt) for n in (H * d, d, H)]
        sep = lambda: indexer_scores_hip(*project(h, *Ws, H, d), write_upper=False)  # noqa: E731
        fus = lambda: indexer_from_hidden(h, *Ws, H, d, write_upper=False)  # noqa: E731
        stream = torch.cuda.current_stream(dev)
        warm(sep, 0.1)
        warm(fus, 0.1)
        # the two forms alternate over 5 rounds and each reports its median
        # round, so neither gains from running first or on settled clocks
        ts, tf = [], []
        for _ in range(5):
            ts.append(time_events(sep, reps, stream))
            tf.append(time_events(fus, reps, stream))
        t_sep, t_fus = sorted(ts)[2], sorted(tf)[2]
        res.append({"shape": f"B={B},T={T},D={D},HI={H},DI={d},{str(dt).replace('torch.', '')}",
                    "three_gemms_us": round(t_sep * 1e6, 1), "fused_us": round(t_fus * 1e6, 1)})
    return res


def bench_select_c4(dev, reps=20):
    """Radix-select on config-4 causal rows (real indexer scores)."""
    import torch

    from lightning_indexer import indexer_scores_hip
    from topk_threshold import topk_indices, topk_threshold, topk_threshold_mask

    T, k = C4["T"], C4["k"]
    ins = gpu_inputs(C4, torch.bfloat16, dev, seed=4)
    scores = indexer_scores_hip(*ins[:3], write_upper=False)
    del ins
    stream = torch.cuda.current_stream(dev)
    warm(lambda: topk_threshold(scores, k, causal=True))
    t_thr = time_events(lambda: topk_threshold(scores, k, causal=True), reps, stream)
    warm(lambda: topk_indices(scores, k, causal=True))
    t_idx = time_events(lambda: topk_indices(scores, k, causal=True), reps, stream)
    thr_buf = torch.empty(1, T, 1, device=dev)
    W = (T + 63) // 64
    mask = torch.empty(1, T, W, device=dev, dtype=torch.int64)
    sel_mask = lambda: topk_threshold_mask(scores, k, thr=thr_buf, mask=mask)  # noqa: E731
    warm(sel_mask)
    t_mask = time_events(sel_mask, reps, stream)
    read = 4.0 * T * (T + 1) / 2
    out_thr = 4.0 * T
    out_idx = out_thr + 4.0 * T * k
    # bitmask words written: row t writes words 0 .. min(W, (t|127)/64 + 1) - 1
    out_mask = out_thr + 8.0 * sum(min(W, ((t | 127) >> 6) + 1) for t in range(T))
    res = {
        "workload": "causal radix-select, config-4 indexer scores [1,16384,16384] fp32, k=2048",
        "ms": round(t_thr * 1e3, 4),
        "GB_per_s": round((read + out_thr) / t_thr / 1e9, 1),
        "frac": round((read + out_thr) / t_thr / 1e9 / PEAK_HBM_GBS, 4),
        "algorithmic_bytes": read + out_thr,
        "with_indices_ms": round(t_idx * 1e3, 4),
        "with_indices_GB_per_s": round((read + out_idx) / t_idx / 1e9, 1),
        "with_indices_frac": round((read + out_idx) / t_idx / 1e9 / PEAK_HBM_GBS, 4),
        "with_mask_ms": round(t_mask * 1e3, 4),
        "with_mask_GB_per_s": round((read + out_mask) / t_mask / 1e9, 1),
        "with_mask_frac": round((read + out_mask) / t_mask / 1e9 / PEAK_HBM_GBS, 4),
        "with_mask_note": "thresholds plus the selection bitmask in one pass "
                          "(topk_threshold_mask, the select the config-4 split forward runs); "
                          f"{out_mask - out_thr:.0f} bytes of bitmask words written",
        "peak_GB_per_s": PEAK_HBM_GBS,
    }
    del scores
    # config-2 standalone top-K: [64,2048,2048] N(0,1), k=128
    x = torch.randn((64, 2048, 2048), device=dev, dtype=torch.float32)
    warm(lambda: topk_threshold(x, 128))
    t2 = time_events(lambda: topk_threshold(x, 128), reps, stream)
    b2 = 4.0 * x.numel() + 4.0 * 64 * 2048
    res["c2_standalone"] = {"workload": "[64,2048,2048] N(0,1) fp32, k=128",
                            "ms": round(t2 * 1e3, 4),
                            "GB_per_s": round(b2 / t2 / 1e9, 1),
                            "frac": round(b2 / t2 / 1e9 / PEAK_HBM_GBS, 4)}
    return res


def cpu_baseline(dev=None, budget_s=12.0):
    """The reference's CPU path, restated: torch-vectorised fp32 DSA forward
    (oracle.dsa_forward, acc=float32) on config 1, plus the AVX-512
    k-th-largest on config 1's score matrix."""
    import numpy as np
    import torch

    from oracle import dsa_oracle as O
    from oracle import native

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    ins = O.make_inputs(C1["B"], C1["T"], C1["HI"], C1["DI"], C1["HQ"], C1["DQ"], C1["DV"])
    k = C1["k"]
    O.dsa_forward(*ins, k, acc=torch.float32)          # warm-up
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n < 2:
        O.dsa_forward(*ins, k, acc=torch.float32)
        n += 1
    dt = (time.perf_counter() - t0) / n
    tokens = C1["B"] * C1["T"]
    res = {"value": round(tokens / dt, 1), "unit": "query tokens/s", "cores": cores,
           "kind": "port",
           "sample": f"config 1 (B=16,T=512,k=32) torch-vectorised fp32 forward x{n}, "
                     f"{dt * 1e3:.1f} ms each",
           "ms_per_step": round(dt * 1e3, 3), "cpu": native.cpu_model()}
    # AVX-512 k-th largest on the config-1 score matrix [16,512,512], k=32
    scores = O.indexer_scores(*ins[:3], acc=torch.float32).contiguous()
    ref = native.ref()
    if ref is not None:
        fn = lambda: ref.topk_threshold(scores, k)  # noqa: E731
        kind = "reference"
    else:
        s_np = scores.numpy()
        fn = lambda: native.port_topk_threshold(s_np, k)  # noqa: E731
        kind = "port"
    for _ in range(5):
        fn()
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 3.0 or reps < 30:
        fn()
        reps += 1
    topk_ms = (time.perf_counter() - t0) / reps * 1e3
    res["topk_avx512"] = {"kind": kind, "ms": round(topk_ms, 4),
                          "sample": "config-1 scores [16,512,512], k=32", "cores": cores,
                          "avx512": "avx512f" in native.cpu_flags()}
    res.update(cpu_baseline_wide(cores))
    res.update(cpu_baseline_small(cores))
    if dev is not None:
        # The reference's hybrid path (dsa_hybrid.py:46-66) on this host: the
        # score matrix crosses PCIe to pinned memory, the CPU selects, the
        # thresholds come back.  Timed here with HIP events around the copies.
        B, T = C1["B"], C1["T"]
        s_gpu = scores.to(dev)
        s_pin = torch.empty(B, T, T, dtype=torch.float32, pin_memory=True)
        t_pin = torch.empty(B, T, 1, dtype=torch.float32, pin_memory=True)
        t_gpu = torch.empty(B, T, 1, device=dev)
        stream = torch.cuda.current_stream(dev)
        d2h = time_events(lambda: s_pin.copy_(s_gpu, non_blocking=True), 20, stream)
        h2d = time_events(lambda: t_gpu.copy_(t_pin, non_blocking=True), 20, stream)
        res["hybrid_pcie"] = {
            "workload": "config 1: scores [16,512,512] fp32 d2h, CPU k-th largest, thresholds "
                        "[16,512,1] h2d (the reference's CPU-offload step)",
            "d2h_ms": round(d2h * 1e3, 4), "cpu_topk_ms": round(topk_ms, 4),
            "h2d_ms": round(h2d * 1e3, 4),
            "offload_ms": round(d2h * 1e3 + topk_ms + h2d * 1e3, 4)}
    return res


def _evenly(T, n):
    """n query rows spread evenly over 0..T-1 (the causal cost of a row grows
    with t, so their mean cost is the mean cost of all T rows)."""
    return [int((i + 0.5) * T / n) for i in range(n)]


def cpu_baseline_wide(cores, budget_s=4.0):
    """The reference's CPU path beyond config 1 (bounded samples, each named):
      * the AVX-512 k-th largest on the standalone [64,2048,2048] k=128 rows
        (the reference publishes 143.9 ms there, README.md:67; method
        bench_avx512.py:25-52): the reference's own source (oracle/_ref) and
        this repo's host library (libdsa_cpu.so, the CPU-offload select);
      * the torch-vectorised fp32 forward (oracle restatement of
        dsa_attention_torch) at configs 3 and 4 on evenly spread query rows,
        chunked over rows, scaled to a whole forward;
      * the k-th largest on config-4 score rows (real indexer scores, -inf
        past the diagonal) for the same sampled rows."""
    import torch

    from oracle import dsa_oracle as O
    from oracle import native
    from topk_threshold import topk_threshold

    out = {}
    ref = native.ref()

    def timed(fn, min_reps=3):
        fn()
        n, t0 = 0, time.perf_counter()
        while n < min_reps or time.perf_counter() - t0 < budget_s / 4:
            fn()
            n += 1
        return (time.perf_counter() - t0) / n * 1e3

    x = torch.randn((64, 2048, 2048), generator=torch.Generator().manual_seed(0))
    row = {"workload": "[64,2048,2048] N(0,1) fp32, k=128 (config 2 standalone)",
           "cores": cores, "reference_published_ms": 143.9,
           "reference_published_on": "Ryzen 9 9950X3D, 16 threads (README.md:67)",
           "host_lib_ms": round(timed(lambda: topk_threshold(x, 128)), 3)}
    if ref is not None:
        row["reference_build_ms"] = round(timed(lambda: ref.topk_threshold(x, 128)), 3)
        row["equal"] = bool(torch.equal(ref.topk_threshold(x, 128), topk_threshold(x, 128)))
    out["topk_c2_standalone"] = row
    del x

    for name, cfg, dt, nrows in (("c3", C3, torch.float32, 256), ("c4", C4, torch.bfloat16, 128)):
        B, T, k = cfg["B"], cfg["T"], cfg["k"]
        ins = O.make_inputs(B, T, cfg["HI"], cfg["DI"], cfg["HQ"], cfg["DQ"], cfg["DV"],
                            dtype=dt, w_scale=(1 / 8 if name == "c4" else None))
        rows = _evenly(T, nrows)
        chunk = O._chunk_rows(len(rows), B * max(cfg["HI"], cfg["HQ"]) * T)
        t0 = time.perf_counter()
        _, sc, _ = O.dsa_forward(*ins, k, acc=torch.float32, rows=rows, return_parts=True)
        dt_s = time.perf_counter() - t0
        est_ms = dt_s * (T / nrows) * 1e3
        out[f"forward_{name}"] = {
            "workload": f"config {name[1]}: torch-vectorised fp32 forward (oracle restatement of "
                        f"dsa_attention_torch; {str(dt).replace('torch.', '')} inputs upcast)",
            "sample": f"{B}x{nrows} query rows spread evenly over T={T} (t = (i+0.5)*T/{nrows}), "
                      f"{chunk} rows per chunk; {dt_s:.2f} s, scaled by T/{nrows}",
            "est_ms_per_forward": round(est_ms, 1),
            "query_tokens_per_s": round(B * T / (est_ms / 1e3), 1), "cores": cores}
        if name == "c4":
            scf = sc.float().contiguous()              # [1, nrows, T], -inf past each t
            r4 = {"workload": f"k-th largest (k={k}) of {nrows} config-4 score rows "
                              f"[1,{nrows},{T}] (real indexer scores, full rows)",
                  "host_lib_ms": round(timed(lambda: topk_threshold(scf, k)), 4)}
            if ref is not None:
                r4["reference_build_ms"] = round(timed(lambda: ref.topk_threshold(scf, k)), 4)
                r4["equal"] = bool(torch.equal(ref.topk_threshold(scf, k),
                                               topk_threshold(scf, k)))
            r4["host_lib_est_ms_all_rows"] = round(r4["host_lib_ms"] * T / nrows, 2)
            out["topk_c4_rows"] = r4
        del ins, sc
    return out


# The reference's published standalone CPU top-K table (README.md:63-67;
# shapes from bench_avx512.py:55-70, rows N(0,1)), on its Ryzen 9 9950X3D:
# (B, T, k, torch.topk ms, avx512 ms).
README_TOPK = ((1, 128, 8, 0.026, 0.005), (4, 128, 8, 0.251, 0.007), (1, 256, 16, 0.189, 0.008),
               (16, 1024, 64, 8.395, 6.771), (64, 2048, 128, 150.5, 143.9))


def time_reference_cpu(fn, budget_s=1.5, warmup=5, iters=30):
    """bench_avx512.py:25-31's method (5 warm-up calls, then the mean over 30
    timed calls, perf_counter), with the timed calls capped to about
    budget_s of work for the slow shapes (at least 3); ms per call."""
    t0 = time.perf_counter()
    fn()
    one = time.perf_counter() - t0
    for _ in range(min(warmup, max(1, int(budget_s / 4 / max(one, 1e-9))))):
        fn()
    n = max(3, min(iters, int(budget_s / max(one, 1e-9))))
    t0 = time.perf_counter()
    for _ in range(n):
        fn()
    return (time.perf_counter() - t0) / n * 1e3, n


def cpu_baseline_small(cores):
    """The reference's CPU path at its own small shapes:
      * the torch-vectorised fp32 forward (oracle restatement of
        dsa_attention_torch, dsa_attention.py:35-52) at configs[0] and at the
        five config-2 (B, k) shapes, whole forwards;
      * the standalone k-th largest at the five shapes of the reference's
        published table: torch.topk's k-th value, the reference's own
        topk_avx512.cpp (oracle/_ref, when built here) and this repo's host
        library, beside the published figures."""
    import torch

    from oracle import dsa_oracle as O
    from oracle import native
    from topk_threshold import topk_threshold

    out = {}
    c0 = dict(B=1, T=128, k=8, HI=4, DI=32, HQ=4, DQ=32, DV=32)
    rows = []
    for name, cfg in [("c0", c0)] + [(f"c2_b{B}_k{k}", dict(C1, B=B, k=k)) for B, k, _ in C2_SWEEP]:
        ins = O.make_inputs(cfg["B"], cfg["T"], cfg["HI"], cfg["DI"], cfg["HQ"], cfg["DQ"], cfg["DV"])
        ms, n = time_reference_cpu(lambda: O.dsa_forward(*ins, cfg["k"], acc=torch.float32))
        rows.append({"config": name, "B": cfg["B"], "T": cfg["T"], "k": cfg["k"],
                     "ms_per_forward": round(ms, 3),
                     "query_tokens_per_s": round(cfg["B"] * cfg["T"] / (ms / 1e3), 1),
                     "timed_calls": n})
        del ins
    out["forward_small"] = {"workload": "torch-vectorised fp32 DSA forward (oracle restatement "
                                        "of dsa_attention_torch) at configs[0] and the config-2 "
                                        "shapes, whole forwards",
                            "method": "bench_avx512.py:25-31 (5 warm-up, mean of up to 30 "
                                      "timed calls, capped to ~1.5 s of work)",
                            "cores": cores, "kind": "port", "rows": rows}
    ref = native.ref()
    trows = []
    for B, T, k, pub_torch, pub_avx in README_TOPK:
        x = torch.randn((B, T, T), generator=torch.Generator().manual_seed(T + k))
        row = {"B": B, "T": T, "k": k, "published_torch_ms": pub_torch,
               "published_avx512_ms": pub_avx}
        row["torch_topk_ms"] = round(time_reference_cpu(lambda: x.topk(k, dim=-1)[0][..., -1:])[0], 4)
        row["host_lib_ms"] = round(time_reference_cpu(lambda: topk_threshold(x, k))[0], 4)
        if ref is not None:
            row["reference_build_ms"] = round(time_reference_cpu(lambda: ref.topk_threshold(x, k))[0], 4)
            row["equal"] = bool(torch.equal(ref.topk_threshold(x, k), topk_threshold(x, k)))
        trows.append(row)
        del x
    out["topk_readme_table"] = {
        "workload": "standalone k-th largest of [B,T,T] N(0,1) fp32 rows at the reference's "
                    "published shapes (README.md:63-67, bench_avx512.py:55-70)",
        "published_on": "Ryzen 9 9950X3D, 16 threads",
        "kind": "reference" if ref is not None else "port",
        "cores": cores, "rows": trows}
    return out


def pmc_workload(args, dev):
    """Kernels whose FETCH_SIZE / WRITE_SIZE give the traffic figures: a plain
    copy of known size (256 MiB read + 256 MiB written) first, so each
    counter's reading per byte can be calibrated in the same run."""
    import torch

    import dsa_attention as D
    from lightning_indexer import indexer_scores_hip
    from topk_threshold import topk_indices, topk_threshold, topk_threshold_mask

    x = torch.ones(64 * 1024 * 1024, device=dev)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    ins = gpu_inputs(C1, torch.float32, dev)
    for _ in range(args.steps):
        D.dsa_fused_hip(*ins, C1["k"])
    torch.cuda.synchronize()
    del ins
    q, kk, w = gpu_inputs(C4, torch.bfloat16, dev, seed=4)[:3]
    scores = indexer_scores_hip(q, kk, w, write_upper=False)
    del q, kk, w
    for _ in range(3):
        thr = topk_threshold(scores, C4["k"], causal=True)
    for _ in range(2):                                      # thresholds + exactly-k indices
        topk_indices(scores, C4["k"], causal=True)
    for _ in range(2):                                      # thresholds + the selection bitmask
        topk_threshold_mask(scores, C4["k"])
    Q, K, V = gpu_inputs(C4, torch.bfloat16, dev, seed=5)[3:]
    out = torch.empty(1, C4["T"], C4["HQ"], C4["DV"], device=dev)
    for _ in range(2):   # selection bitmask + the tile kernel reading it, at this T
        D.sparse_attention_hip(scores, thr, Q, K, V, out=out)
    torch.cuda.synchronize()
    del scores, thr, Q, K, V, out
    # config 3: indexer (fp32), select, and 2 launches of the staged attention
    ins = gpu_inputs(C3, torch.float32, dev, seed=3)
    scores = indexer_scores_hip(*ins[:3], write_upper=False)
    thr = topk_threshold(scores, C3["k"], causal=True)
    out = torch.empty(C3["B"], C3["T"], C3["HQ"], C3["DV"], device=dev)
    for _ in range(2):
        D.sparse_attention_hip(scores, thr, *ins[3:], out=out)  # the staged kernel at this T
    torch.cuda.synchronize()
    log("pmc workload done")


def traffic_from_profile():
    path = os.path.join(ROOT, "profiles", "fused_c1_traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=("graph", "eager"), default="graph")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-select", action="store_true", help="skip the config-4 select leg")
    ap.add_argument("--no-hybrid", action="store_true", help="skip the CPU-offload legs")
    ap.add_argument("--no-long", action="store_true",
                    help="skip the split-forward legs at configs 3 and 4")
    ap.add_argument("--only-headline", action="store_true",
                    help="run only the headline leg (fused config 1: warm-up, the timed "
                         "graph and the event-timed launches) and print its JSON line; "
                         "for a kernel-trace profile of that kernel alone")
    ap.add_argument("--only-select", action="store_true",
                    help="run only the config-4 select leg (thresholds, thresholds + "
                         "indices, thresholds + bitmask; then the config-2 standalone "
                         "top-K) and print its JSON; for a kernel-trace profile of the "
                         "select kernels alone")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run only the workload profiled with counters: one 256 MiB "
                         "device-to-device copy (counter calibration), then --steps eager "
                         "fused launches at config 1, the config-4 indexer, 3 causal "
                         "selects and 2 tile-attention launches at config 4, then the "
                         "config-3 indexer, select and 2 staged-attention launches")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): this build has no "
              "multi-GPU path (the forward would shard by batch element, one process per "
              "GPU, or by zig-zag query tiles after one all-gather of k_idx, K and V).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    if args.pmc_workload:
        pmc_workload(args, dev)
        return
    if args.only_select:
        log("bench: select at config 4 (only)")
        print(json.dumps({"topk_select": bench_select_c4(dev)}), flush=True)
        return
    B, T = C1["B"], C1["T"]
    log("bench: fused config 1")
    elapsed, kern_s = bench_fused(args, dev)
    ms = elapsed / args.steps * 1e3
    value = B * T * args.steps / elapsed
    flops = indexer_flops(B, T, C1["HI"], C1["DI"]) + attention_flops(
        B, T, C1["k"], C1["HQ"], C1["DQ"], C1["DV"])
    achieved = flops / kern_s / 1e12
    split_s = None
    if not args.only_headline:
        log("bench: split config 1")
        split_s = bench_split(dev)
    out = {
        "metric": "DSA fwd ms + query tokens/s at B=16,T=512,k=32; top-K HBM GB/s vs peak",
        "value": round(value, 1),
        "unit": "query tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / (B * T / (BASELINE_MS / 1e3)), 2),
        "baseline": {"ms": BASELINE_MS, "source": "reference README.md:49, fused Triton on "
                     "RTX PRO 6000 Blackwell"},
        "dtype": "f32",
        "data": "synthetic N(0,1) (w ~ N(0,1)/sqrt(HI)), resident in HBM",
        "config": {"workload": "config 1: fused DSA forward (indexer + radix-select + sparse "
                               "attention, one gfx950 kernel)",
                   "B": B, "T": T, "top_k": C1["k"], "HI": C1["HI"], "DI": C1["DI"],
                   "HQ": C1["HQ"], "DQ": C1["DQ"], "DV": C1["DV"], "mode": args.mode},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                     "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 5),
                     "traffic": traffic_from_profile(),
                     "traffic_source": "profiles/fused_c1_traffic.json: FETCH_SIZE and "
                                       "WRITE_SIZE of the fused launch in a rocprofv3 --pmc "
                                       "run of bench.py --pmc-workload, calibrated against a "
                                       "256 MiB copy in the same run (read from that file, "
                                       "not measured by this run)",
                     "kernel": "fused_kernel<F32,32,2,2,2,16,true>",
                     "kernel_ms": round(kern_s * 1e3, 5),
                     "flops_per_launch": flops},
    }
    if args.only_headline:
        print(json.dumps(out), flush=True)
        return
    out["split"] = {"ms_per_step": round(split_s * 1e3, 5),
                    "value": round(B * T / split_s, 1), "unit": "query tokens/s"}
    log("bench: config 2 sweep")
    out["sweep_c2"] = bench_sweep_c2(dev)
    if not args.no_select:
        log("bench: select at config 4")
        out["topk_select"] = bench_select_c4(dev)
    if not args.no_long:
        log("bench: split forward at configs 3 and 4")
        out["split_c3"] = bench_split_long(dev, C3, torch.float32, "config 3", 10)
        out["split_c4"] = bench_split_long(dev, C4, torch.bfloat16, "config 4", 5, fp8_indexer=True)
        log("bench: projection front end")
        out["projection"] = bench_projection(dev)
        log("bench: batch streaming at configs 2, 3 and 4")
        out["stream"] = {
            "c2": bench_stream(dev, C2, torch.float32, "config 2 (B=4,T=512,k=64)", nbatch=16),
            "c3": bench_stream(dev, C3, torch.float32, "config 3"),
            "c4": bench_stream(dev, C4, torch.bfloat16, "config 4"),
        }
    log("bench: eager per-call latency at config 1")
    out["eager_latency_c1"] = bench_eager_latency(dev)
    if not args.no_hybrid:
        log("bench: CPU-offload (hybrid) forward")
        out["hybrid"] = bench_hybrid(dev)
    if not args.no_cpu:
        log("bench: CPU baseline")
        out["cpu_baseline"] = cpu_baseline(dev)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
