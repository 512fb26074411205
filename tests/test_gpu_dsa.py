"""GPU: end-to-end forward parity (fused and split drop-ins) -- the reference's
test_dsa.py cases plus every BASELINE.json config.

Staged as the tie semantics require: (1) HIP indexer scores vs the oracle's
(1e-4 / 2e-2); (2) the forward vs the float64 oracle run on the GPU's own
score matrix (the select is exact, so this isolates attention error); (3)
the forward vs the oracle from scratch, rows whose selected set flips on a
near-tie of the two score matrices counted separately (they must be rare).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import dsa_attention as D
from helpers import CONFIGS, close, flipped_rows, inputs, sample_rows, say, to_dev
from lightning_indexer import indexer_scores_hip
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def ref_make(B=1, T=32, HI=4, DI=32, HQ=4, DQ=32, DV=32):
    """The reference tests' inputs (test_dsa.py:17-24): everything but V x0.3."""
    return O.make_inputs(B, T, HI, DI, HQ, DQ, DV, scale=0.3, w_scale=0.3)


@pytest.mark.parametrize("T,top_k,BLOCK_S", [(32, 8, 16), (64, 16, 32), (128, 32, 32)])
def test_fused_matches_oracle(dev, T, top_k, BLOCK_S):
    """test_dsa.py:35-41 (max abs diff < 5e-4)."""
    ins = ref_make(T=T)
    out = D.dsa_attention_triton(*to_dev(ins, dev), top_k=top_k, BLOCK_S=BLOCK_S).cpu()
    ref = O.dsa_forward(*ins, top_k)
    assert float((out.double() - ref).abs().max()) < 5e-4


@pytest.mark.parametrize("B,T,top_k", [(2, 256, 32), (2, 512, 100), (16, 512, 32)])
def test_fused_tie_heavy_scores(dev, B, T, top_k):
    """Integer-valued indexer inputs give exactly representable, heavily tied
    scores (the same in fp32 and float64), so the fused kernel's in-LDS
    select must keep exactly the oracle's tied set; batch element 1 has all
    scores 0 (one value in every row).  B=16, T=512 runs the config-1 grid
    (long and short tiles paired per CU)."""
    g = torch.Generator().manual_seed(T)
    HI, DI, HQ, DH = 4, 32, 4, 32
    qi = torch.randint(-1, 2, (B, T, HI, DI), generator=g).float()
    ki = torch.randint(-1, 2, (B, T, DI), generator=g).float()
    wi = torch.randint(1, 3, (B, T, HI), generator=g).float()
    qi[1] = 0.0
    Q, K, V = (torch.randn((B, T, HQ, DH), generator=g) for _ in range(3))
    ins = (qi, ki, wi, Q, K, V)
    say(f"fused tie-heavy B={B} T={T} k={top_k}")
    out = D.dsa_fused_hip(*to_dev(ins, dev), top_k).cpu()
    ref = O.dsa_forward(*ins, top_k)
    assert float((out.double() - ref).abs().max()) < 5e-4


def test_all_three_agree_small(dev):
    """test_dsa.py:44-52: naive / oracle / fused at HI=2, DI=16, HQ=2, D=16."""
    ins = ref_make(B=2, T=32, HI=2, DI=16, HQ=2, DQ=16, DV=16)
    a = O.dsa_forward_naive(*ins, 8)
    b = O.dsa_forward(*ins, 8).numpy()
    c = D.dsa_attention_triton(*to_dev(ins, dev), top_k=8, BLOCK_S=16).cpu().numpy()
    assert np.abs(a - b).max() < 1e-4
    assert np.abs(b - c).max() < 5e-4


@pytest.mark.parametrize("HQ,DH", [(32, 4), (16, 8), (8, 16), (2, 64), (1, 128)])
def test_fused_two_keys_per_load_head_widths(dev, HQ, DH):
    """The fused forward at every head width of the two-keys-per-load
    gathers (fp32 rows of HQ*D = 128 elements): against the float64 oracle,
    and equal to the split forward, whose gather kernel shares the code."""
    B, T, k = 2, 300, 24
    ins = O.make_inputs(B, T, 4, 32, HQ, DH, DH)
    g = to_dev(ins, dev)
    fused = D.dsa_fused_hip(*g, k)
    split = D.dsa_split_hip(*g, k)
    torch.cuda.synchronize()
    s_gpu = indexer_scores_hip(*g[:3]).cpu().double()
    want = O.sparse_attn_threshold(s_gpu, O.topk_threshold(s_gpu, k), *ins[3:])
    ok, err, _ = close(fused.cpu(), want, 1e-4, 1e-4)
    assert ok, f"fused vs oracle on the GPU's scores: max abs err {err}"
    assert float((fused - split).abs().max()) <= 1e-6


@pytest.mark.parametrize("T,top_k", [(32, 8), (64, 16), (128, 32)])
def test_split_matches_oracle(dev, T, top_k):
    """test_dsa.py:55-61."""
    ins = ref_make(T=T)
    out = D.dsa_attention_split_triton(*to_dev(ins, dev), top_k=top_k).cpu()
    ref = O.dsa_forward(*ins, top_k)
    assert float((out.double() - ref).abs().max()) < 5e-4


def test_golden_c0(dev):
    """Config 0 against the committed golden fixture (float64 oracle outputs)."""
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "c0_forward.npz"))
    ins = tuple(torch.from_numpy(z[n]) for n in ("q_idx", "k_idx", "w_idx", "Q", "K", "V"))
    k = int(z["top_k"])
    g = to_dev(ins, dev)
    s = indexer_scores_hip(*g[:3]).cpu()
    causal = torch.ones(128, 128, dtype=torch.bool).tril()
    assert close(s[:, causal], torch.from_numpy(z["scores"])[:, causal], 1e-4, 1e-4)[0]
    flips = flipped_rows(s.double(), torch.from_numpy(z["scores"]), k)
    ok = ~flips
    for fn in (D.dsa_attention_triton, D.dsa_attention_split_triton):
        out = fn(*g, top_k=k).cpu()
        assert close(out[ok], torch.from_numpy(z["out"])[ok], 1e-4, 1e-4)[0], fn.__name__
    assert int(flips.sum()) == 0


def staged_check(dev, name, rows=None, rtol=1e-4, atol=1e-4, max_flip_frac=0.005):
    ins, k = inputs(name)
    B, T = ins[3].shape[:2]
    say(f"dsa {name}: B={B} T={T} k={k} rows={'all' if rows is None else len(rows)}")
    g = to_dev(ins, dev)
    fused = D.dsa_forward_hip(*g, k) if T <= 2048 else None
    split = D.dsa_split_hip(*g, k)
    s_gpu = indexer_scores_hip(*g[:3])
    torch.cuda.synchronize()
    sel = slice(None) if rows is None else rows
    s_cpu = s_gpu[:, sel].cpu().double()
    # (1) scores
    s_ref = O.indexer_scores(*ins[:3], rows=rows)
    ts = torch.arange(T) if rows is None else torch.tensor(rows)
    causal = torch.arange(T)[None, :] <= ts[:, None]
    ok, err, _ = close(s_cpu[:, causal], s_ref[:, causal], rtol, atol)
    assert ok, f"scores max abs err {err}"
    # (2) forward vs oracle on the GPU's own scores
    thr = O.topk_threshold(s_cpu, min(k, T))
    want = O.sparse_attn_threshold(s_cpu, thr, *ins[3:], rows=rows)
    outs = {"split": split}
    if fused is not None:
        outs["fused"] = fused
    for nm, o in outs.items():
        ok, err, _ = close(o[:, sel].cpu(), want, rtol, atol)
        assert ok, f"{nm} vs oracle-on-gpu-scores max abs err {err}"
    if fused is not None:
        assert float((fused - split).abs().max()) <= 1e-6, "fused and split disagree"
    # (3) from scratch, near-tie flips counted apart
    want0 = O.sparse_attn_threshold(s_ref, O.topk_threshold(s_ref, min(k, T)), *ins[3:],
                                    rows=rows)
    flips = flipped_rows(s_cpu, s_ref, min(k, T), rows=rows)
    keep = ~flips
    ok, err, _ = close(split[:, sel].cpu()[keep], want0[keep], rtol, atol)
    assert ok, f"from-scratch max abs err {err}"
    frac = float(flips.float().mean())
    say(f"  flipped rows: {int(flips.sum())} ({frac:.4%})")
    assert frac <= max_flip_frac


@pytest.mark.parametrize("name", ["c0", "c1", "c2_b4_k64", "c2_b16_k64", "c2_b16_k128",
                                  "c2_b32_k64", "c2_b64_k64"])
def test_configs_t512(dev, name):
    staged_check(dev, name)


@pytest.mark.parametrize("name", ["c1_t500", "c1_t496"])
def test_fused_tile_pairing_edges(dev, name):
    """Config-1 widths around the fused kernel's tile pairing per CU: T=500
    has a partial last tile (rows past T in the longest tile), T=496 an odd
    tile count."""
    staged_check(dev, name)


def test_fused_at_max_T(dev):
    """T = 2048, the fused kernel's limit (dsa_fused_max_T), with 16-query
    blocks whose score rows take the most LDS; fused and split must agree."""
    staged_check(dev, "fused_t2048", rows=sample_rows(2048, 16, include=(0, 63, 64, 1023, 2047)))


def test_config3(dev):
    staged_check(dev, "c3", rows=sample_rows(4096, 24, include=(0, 254, 255, 256, 4095)))


def test_config4(dev):
    staged_check(dev, "c4", rows=sample_rows(16384, 8, include=(0, 2046, 2047, 16383)),
                 rtol=2e-2, atol=2e-2)


def test_config4_split_equals_threshold_tile_kernel(dev):
    """The config-4 split forward runs the select writing the bitmask
    (topk_threshold_mask) and the tile kernel on that bitmask; its full
    output, all 16384 rows, equals bit for bit the tile kernel that reads
    the scores and a threshold from the threshold-only select
    (dsa_attention.py:343-345 as three steps)."""
    from topk_threshold import topk_threshold

    ins, k = inputs("c4")
    g = to_dev(ins, dev)
    del ins
    say("config 4 split forward vs threshold tile kernel, all rows")
    split = D.dsa_split_hip(*g, k)
    s = indexer_scores_hip(*g[:3], write_upper=False)
    thr = topk_threshold(s, k, causal=True)
    tiled = D.sparse_attention_hip(s, thr, *g[3:], kernel="tiled")
    torch.cuda.synchronize()
    assert not bool(torch.isnan(split).any())
    assert torch.equal(split, tiled)


def test_hybrid_path_with_reference_cpu_threshold(dev):
    """dsa_hybrid.py:46-66: the hybrid drop-in equals the split forward, and a
    threshold made on the CPU by this repo's port of the reference's AVX-512
    extension, fed to the sparse-attention drop-in, gives the same output."""
    from dsa_hybrid import HybridContext, dsa_hybrid_cpu_topk
    from oracle import native

    ins, k = inputs("c1")
    g = to_dev(ins, dev)
    ctx = HybridContext(16, 512)
    hyb = dsa_hybrid_cpu_topk(*g, k, ctx=ctx)
    split = D.dsa_attention_split_triton(*g, top_k=k)
    assert torch.equal(hyb, split)
    s = indexer_scores_hip(*g[:3])
    thr_cpu = torch.from_numpy(native.port_topk_threshold(s.cpu().numpy(), k))
    ref = native.ref()
    if ref is not None:
        assert torch.equal(ref.topk_threshold(s.cpu().contiguous(), k), thr_cpu)
    out = D.sparse_attention_with_threshold_triton(s, thr_cpu.to(dev), *g[3:])
    assert torch.equal(out, split)


@pytest.mark.parametrize("name", ["wide_f32_t512", "wide_f32_t2048", "wide_bf16_t512",
                                  "wide_bf16_t2048"])
def test_wide_attention_rows(dev, name):
    """dsa_attention_split_triton / dsa_attention_triton on attention rows
    wider than one wave holds (fp32 HQ=16 x D=128, bf16 HQ=128 x D=128): the
    reference accepts them (powers of two only, dsa_attention.py:202-206,
    :338-340).  Staged against the oracle as for the configs."""
    from helpers import sample_rows

    ins, k = inputs(name)
    B, T = ins[3].shape[:2]
    tol = 1e-4 if ins[3].dtype == torch.float32 else 2e-2
    rows = None if T <= 512 else sample_rows(T, 48, seed=2, include=(0, k - 1, k, T - 1))
    staged_check(dev, name, rows=rows, rtol=tol, atol=tol)
    g = to_dev(ins, dev)
    a = D.dsa_attention_split_triton(*g, top_k=k)
    b = D.dsa_attention_triton(*g, top_k=k)        # no fused instance: the split kernels
    torch.cuda.synchronize()
    assert torch.equal(a, b)
