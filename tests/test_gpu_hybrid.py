"""GPU: the CPU-offload ("hybrid") forward (dsa_hybrid.py; reference
dsa_hybrid.py:36-66).  GPU indexer -> pinned d2h -> host k-th largest
(libdsa_cpu.so) -> h2d -> GPU sparse attention.  The host select is exact, so
the output must be bit-identical to the all-GPU split forward on the same
inputs; the host thresholds must equal the reference's own compiled
extension (oracle/_ref) on the same GPU-made scores, bit for bit; one case is
also checked against the float64 oracle."""
from __future__ import annotations

import pytest
import torch

import dsa_attention as D
from dsa_hybrid import HybridContext, dsa_hybrid_cpu_topk, dsa_hybrid_stream
from helpers import close, inputs, say, to_dev
from lightning_indexer import indexer_scores_hip
from oracle import dsa_oracle as O
from oracle import native
from topk_threshold import topk_threshold

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["c0", "c1", "c2_b4_k64", "c2_b16_k128"])
@pytest.mark.parametrize("chunks,causal", [(1, False), (4, True), (7, False)])
def test_hybrid_equals_split(dev, name, chunks, causal):
    ins, k = inputs(name)
    say(f"hybrid {name} chunks={chunks} causal={causal}")
    g = to_dev(ins, dev)
    B, T = ins[3].shape[:2]
    ctx = HybridContext(B, T, device=dev)
    split = D.dsa_attention_split_triton(*g, top_k=k)
    for rep in range(2):                      # the context is reused as-is
        hyb = dsa_hybrid_cpu_topk(*g, k, ctx=ctx, chunks=chunks, causal=causal)
        torch.cuda.synchronize()
        assert torch.equal(hyb, split), f"rep {rep}"
    # the thresholds the host wrote are the GPU select's, bit for bit
    gpu_thr = topk_threshold(indexer_scores_hip(*g[:3], write_upper=False), min(k, T),
                             causal=True)
    assert torch.equal(ctx.thr_cpu, gpu_thr.cpu())


def test_hybrid_host_thresholds_match_reference_build(dev):
    """On the GPU's config-1 scores, the host library and the reference's
    own compiled topk_avx512.cpp give identical thresholds."""
    ref = native.ref() if native.ref_available() else None
    if ref is None:
        pytest.skip("oracle/_ref not built for this host")
    ins, k = inputs("c1")
    g = to_dev(ins, dev)
    ctx = HybridContext(16, 512, device=dev)
    dsa_hybrid_cpu_topk(*g, k, ctx=ctx)
    torch.cuda.synchronize()
    assert torch.equal(ctx.thr_cpu, ref.topk_threshold(ctx.scores_cpu, k))


def test_hybrid_vs_oracle(dev):
    ins = O.make_inputs(2, 256, 4, 32, 4, 32, 32, seed0=11, scale=0.3, w_scale=0.3)
    out = dsa_hybrid_cpu_topk(*to_dev(ins, dev), 24).cpu()
    ok, err, _ = close(out, O.dsa_forward(*ins, 24), 1e-4, 1e-4)
    assert ok, f"max abs err {err}"


def test_hybrid_stream_equals_split(dev):
    """Batch streaming: the host select of batch i overlaps the GPU indexer
    and d2h of batch i+1; every output equals the split forward's."""
    say("hybrid stream")
    batches = []
    for i in range(5):
        ins = O.make_inputs(4, 512, 4, 32, 4, 32, 32, seed0=20 + 10 * i)
        batches.append(to_dev(ins, dev))
    for chunks, causal in ((1, True), (3, False)):
        outs = dsa_hybrid_stream(batches, 64, chunks=chunks, causal=causal)
        for bt, o in zip(batches, outs):
            assert torch.equal(o, D.dsa_attention_split_triton(*bt, top_k=64))


def test_hybrid_checks_like_reference(dev):
    ins, k = inputs("c0")
    g = to_dev(ins, dev)
    with pytest.raises(RuntimeError, match="k must be"):
        dsa_hybrid_cpu_topk(*g, 129)
    q3 = g[3][:, :96].contiguous()
    with pytest.raises(AssertionError, match="power of 2"):
        dsa_hybrid_cpu_topk(g[0][:, :96], g[1][:, :96], g[2][:, :96], q3, q3, q3, 8)
