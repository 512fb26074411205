"""GPU: threshold-driven sparse attention vs the float64 oracle on the same
score matrix and threshold (rtol/atol 1e-4 fp32, 2e-2 16-bit)."""
from __future__ import annotations

import math

import pytest
import torch

import _dsa_lib as L
from dsa_attention import sparse_attention_hip, sparse_attention_with_threshold_triton
from helpers import close, say
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def run_case(dev, B, T, HQ, DQ, DV, thr_fn, dtype=torch.float32, rtol=1e-4, atol=1e-4,
             seed0=0, rows=None, tiled=False, kernel=None):
    say(f"attn B={B} T={T} HQ={HQ} DQ={DQ} DV={DV} {dtype} tiled={tiled} kernel={kernel}")
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, DQ, DV, dtype=dtype, seed0=seed0)
    g = torch.Generator().manual_seed(seed0 + 17)
    scores = torch.randn(B, T, T, generator=g)
    scores = torch.where(torch.rand(B, T, T, generator=g) < 0.1, 0.0, scores)   # ties at 0
    thr = thr_fn(scores)
    out = sparse_attention_hip(scores.to(dev), thr.to(dev), Q.to(dev), K.to(dev), V.to(dev),
                               tiled=tiled, kernel=kernel)
    torch.cuda.synchronize()
    if rows is None:
        want = O.sparse_attn_threshold(scores, thr, Q, K, V)
        got = out.cpu()
    else:
        want = O.sparse_attn_threshold(scores[:, rows], thr[:, rows], Q, K, V, rows=rows)
        got = out[:, rows].cpu()
    ok, err, _ = close(got, want, rtol, atol)
    assert ok, f"max abs err {err}"
    return out


def kth(k):
    def f(scores):
        T = scores.shape[-1]
        masked = scores.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), -math.inf)
        return O.topk_threshold(masked, min(k, T))
    return f


@pytest.mark.parametrize("B,T,HQ,D,k", [(1, 128, 4, 32, 8), (16, 512, 4, 32, 32),
                                        (2, 32, 2, 16, 8), (2, 300, 8, 64, 40),
                                        (1, 257, 1, 64, 16), (1, 64, 64, 1, 8),
                                        (2, 200, 16, 64, 20)])
def test_kth_threshold(dev, B, T, HQ, D, k):
    run_case(dev, B, T, HQ, D, D, kth(k))


@pytest.mark.parametrize("HQ,D", [(32, 4), (16, 8), (8, 16), (4, 32), (2, 64), (1, 128)])
def test_two_keys_per_load_head_widths(dev, HQ, D):
    """fp32 rows of HQ*D = 128 elements gather two keys per wave load, each
    half-wave one key's row; a head spans D/4 lanes of a half (1 to 32: the
    logit's butterfly is 0 to 5 steps, the last across 16-lane rows).  Every
    width against the oracle, with ties at the threshold and a ragged T."""
    run_case(dev, 2, 301, HQ, D, D, kth(40))


@pytest.mark.parametrize("HQ,D", [(4, 32), (8, 64)])
def test_gather_empty_selection_rows_are_nan(dev, HQ, D):
    """Per-query gathers (two keys per load at HQ*D = 128, one at 512): rows
    whose threshold nothing reaches (+inf, NaN) give 0/0 = NaN, as the
    reference's softmax over an all -inf row; the other rows match the
    oracle."""
    B, T = 2, 200
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D)
    s = torch.randn(B, T, T, generator=torch.Generator().manual_seed(6))
    thr = kth(24)(s)
    bad = torch.tensor([0, 9, 150, 199])
    thr[1, bad[:2], 0] = math.inf
    thr[1, bad[2:], 0] = math.nan
    out = sparse_attention_hip(s.to(dev), thr.to(dev), Q.to(dev), K.to(dev), V.to(dev)).cpu()
    assert bool(torch.isnan(out[1, bad]).all())
    good = torch.ones(B, T, dtype=torch.bool)
    good[1, bad] = False
    want = O.sparse_attn_threshold(s, thr, Q, K, V)
    assert not bool(torch.isnan(out[good]).any())
    assert close(out[good], want[good], 1e-4, 1e-4)[0]


@pytest.mark.parametrize("HQ,DQ,DV", [(4, 32, 64), (4, 64, 32), (2, 16, 32), (8, 64, 128)])
def test_dq_ne_dv(dev, HQ, DQ, DV):
    run_case(dev, 2, 160, HQ, DQ, DV, kth(12))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("HQ,D", [(16, 128), (4, 32), (8, 64)])
def test_16bit(dev, dtype, HQ, D):
    run_case(dev, 2, 256, HQ, D, D, kth(24), dtype=dtype, rtol=2e-2, atol=2e-2)


def test_external_thresholds(dev):
    """Any threshold tensor works (the hybrid path's CPU-made threshold)."""
    # -inf: every causal key -> dense causal attention
    run_case(dev, 2, 200, 4, 32, 32, lambda s: torch.full(s.shape[:2] + (1,), -math.inf))
    # random thresholds, capped at the s = t score so every row keeps a key
    run_case(dev, 2, 200, 4, 32, 32,
             lambda s: torch.minimum(torch.randn(s.shape[:2] + (1,),
                                                 generator=torch.Generator().manual_seed(3)),
                                     s.diagonal(0, 1, 2)[..., None]))
    # threshold = the score at s = t: keeps exactly the keys scoring >= the diagonal one
    run_case(dev, 2, 200, 4, 32, 32, lambda s: s.diagonal(0, 1, 2)[..., None].contiguous())


def test_single_key_gives_v_row(dev):
    B, T, HQ, D = 1, 96, 4, 32
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D)
    scores = torch.zeros(B, T, T)
    star = torch.randint(0, 10 ** 6, (T,), generator=torch.Generator().manual_seed(1)) % \
        (torch.arange(T) + 1)
    scores[0, torch.arange(T), star] = 1.0
    out = sparse_attention_hip(scores.to(dev), torch.ones(B, T, 1, device=dev), Q.to(dev),
                               K.to(dev), V.to(dev)).cpu()
    assert torch.allclose(out[0], V[0, star], rtol=1e-6, atol=1e-6)


def test_c4_shape_sampled_rows(dev):
    rows = [0, 100, 2047, 2048, 4000, 16383]
    run_case(dev, 1, 16384, 16, 128, 128, kth(2048), dtype=torch.bfloat16, rtol=2e-2,
             atol=2e-2, rows=rows)


def test_reference_wrapper_asserts_and_strided_threshold(dev):
    """threshold may be a non-contiguous view, e.g. topv[..., -1:] (:343-344)."""
    B, T = 2, 64
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, 4, 32, 32)
    s = torch.randn(B, T, T)
    s = s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), -math.inf)
    topv = torch.topk(s, 8, dim=-1).values
    out = sparse_attention_with_threshold_triton(s.to(dev), topv.to(dev)[..., -1:], Q.to(dev),
                                                 K.to(dev), V.to(dev)).cpu()
    want = O.sparse_attn_threshold(s, topv[..., -1:], Q, K, V)
    assert close(out, want, 1e-4, 1e-4)[0]


# --- dense-masked MFMA tile kernel (long rows; forced here at small T) ------
BF, HF = torch.bfloat16, torch.float16


@pytest.mark.parametrize("B,T,HQ,D,k,dtype", [(1, 128, 4, 64, 8, BF), (2, 300, 2, 128, 40, BF),
                                              (1, 257, 1, 64, 16, HF), (2, 200, 16, 128, 20, BF),
                                              (1, 1000, 3, 64, 100, HF), (1, 129, 2, 128, 200, BF)])
def test_tiled_kth_threshold(dev, B, T, HQ, D, k, dtype):
    """Ragged T (not a multiple of the 128-query / 64-key tiles), HQ not a
    power of two, k > T (every causal key), both 16-bit types."""
    run_case(dev, B, T, HQ, D, D, kth(k), dtype=dtype, rtol=2e-2, atol=2e-2, tiled=True)


def test_tiled_external_thresholds(dev):
    """-inf selects every causal key (dense causal attention); a diagonal
    threshold keeps the keys scoring at least the s = t score."""
    run_case(dev, 2, 260, 4, 64, 64, lambda s: torch.full(s.shape[:2] + (1,), -math.inf),
             dtype=BF, rtol=2e-2, atol=2e-2, tiled=True)
    run_case(dev, 2, 260, 4, 64, 64, lambda s: s.diagonal(0, 1, 2)[..., None].contiguous(),
             dtype=BF, rtol=2e-2, atol=2e-2, tiled=True)


def test_tiled_empty_selection_rows_are_nan(dev):
    """Rows whose threshold nothing reaches (+inf, NaN) give 0/0 = NaN, as the
    reference's softmax over an all -inf row; the other rows are unaffected."""
    B, T, HQ, D = 1, 200, 2, 64
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, dtype=BF)
    s = torch.randn(B, T, T, generator=torch.Generator().manual_seed(5))
    thr = kth(16)(s)
    bad = torch.tensor([0, 7, 130, 199])
    thr[0, bad[:2], 0] = math.inf
    thr[0, bad[2:], 0] = math.nan
    out = sparse_attention_hip(s.to(dev), thr.to(dev), Q.to(dev), K.to(dev), V.to(dev),
                               tiled=True).cpu()
    assert bool(torch.isnan(out[0, bad]).all())
    good = torch.ones(T, dtype=torch.bool)
    good[bad] = False
    want = O.sparse_attn_threshold(s, thr, Q, K, V)
    assert close(out[0, good], want[0, good], 2e-2, 2e-2)[0]


def test_tiled_and_gather_agree(dev):
    """Both kernels on the same bf16 inputs (config-4-like head shape)."""
    B, T, HQ, D = 1, 700, 16, 128
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, dtype=BF)
    s = torch.randn(B, T, T, generator=torch.Generator().manual_seed(9))
    thr = kth(64)(s)
    args = (s.to(dev), thr.to(dev), Q.to(dev), K.to(dev), V.to(dev))
    a = sparse_attention_hip(*args, tiled=True).cpu()
    b = sparse_attention_hip(*args).cpu()
    assert close(a, b, 2e-2, 2e-2)[0]


def test_tiled_unsupported_shapes_raise(dev):
    from _dsa_lib import DSAUnsupported

    _, _, _, Q, K, V = O.make_inputs(1, 64, 1, 1, 4, 32, 32)
    s = torch.randn(1, 64, 64)
    with pytest.raises(DSAUnsupported):     # fp32 and D = 32 have no tile kernel
        sparse_attention_hip(s.to(dev), kth(8)(s).to(dev), Q.to(dev), K.to(dev), V.to(dev),
                             tiled=True)


# --- selection bitmask + the tile kernel reading it ------------------------
def _mask_bits_oracle(scores, thr):
    """The bitmask dsa_selection_mask must write, from the selection rule
    itself (per key: s <= t and score >= thr), packed with numpy."""
    import numpy as np
    B, T, _ = scores.shape
    W = (T + 63) // 64
    s = np.arange(W * 64)
    sc = np.full((B, T, W * 64), np.nan, dtype=np.float32)
    sc[:, :, :T] = scores.numpy()
    sel = (s[None, None, :] <= np.arange(T)[None, :, None]) & (sc >= thr.reshape(B, T, 1).numpy())
    bits = sel.reshape(B, T, W, 64).astype(np.uint64) << np.arange(64, dtype=np.uint64)
    return bits.sum(axis=-1, dtype=np.uint64)


@pytest.mark.parametrize("B,T", [(1, 64), (2, 130), (1, 300), (3, 257), (1, 1000)])
def test_selection_mask_bits(dev, B, T):
    """Every word a row's 128-query block reads, bit for bit, against the
    selection rule applied key by key: ties at the threshold, NaN scores,
    +-inf scores, a NaN and an +inf threshold, ragged T."""
    from dsa_attention import selection_mask

    say(f"selection mask B={B} T={T}")
    g = torch.Generator().manual_seed(T)
    s = torch.randn(B, T, T, generator=g)
    s = torch.where(torch.rand(B, T, T, generator=g) < 0.1, 0.0, s)
    s[0, :, 3] = math.nan
    s[0, :, 5] = math.inf
    s[-1, :, 7 % T] = -math.inf
    thr = kth(16)(s)
    thr[0, T // 2, 0] = math.nan
    thr[-1, T - 1, 0] = math.inf
    got = selection_mask(s.to(dev), thr.to(dev)).cpu().numpy().view("uint64")
    want = _mask_bits_oracle(s, thr)
    W = (T + 63) // 64
    for t in range(T):
        nw = min(W, (t | 127) // 64 + 1)
        assert (got[:, t, :nw] == want[:, t, :nw]).all(), f"row {t}"


@pytest.mark.parametrize("B,T,HQ,D,k,dtype", [(1, 128, 4, 64, 8, BF), (2, 300, 2, 128, 40, BF),
                                              (1, 257, 1, 64, 16, HF), (2, 200, 16, 128, 20, BF),
                                              (1, 1000, 3, 64, 100, HF), (1, 129, 2, 128, 200, BF)])
def test_mask_kernel_equals_tiled(dev, B, T, HQ, D, k, dtype):
    """The bitmask path (dsa_selection_mask + dsa_sparse_attn_mask) gives the
    scores-reading tile kernel's output bit for bit, and the oracle's within
    the 16-bit tolerance."""
    out = run_case(dev, B, T, HQ, D, D, kth(k), dtype=dtype, rtol=2e-2, atol=2e-2, kernel="mask")
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, dtype=dtype, seed0=0)
    g = torch.Generator().manual_seed(17)
    scores = torch.randn(B, T, T, generator=g)
    scores = torch.where(torch.rand(B, T, T, generator=g) < 0.1, 0.0, scores)
    ref = sparse_attention_hip(scores.to(dev), kth(k)(scores).to(dev), Q.to(dev), K.to(dev),
                               V.to(dev), kernel="tiled")
    assert torch.equal(out, ref)


@pytest.mark.parametrize("T,D", [(300, 64), (700, 128)])
def test_mask_kernel_nonfinite_logits(dev, T, D):
    """K rows with +inf, -inf or NaN elements and a Q row with +inf give
    non-finite logits.  Unselected keys' logits are masked to -inf whatever
    they are, as the reference masks them before its softmax; selected ones
    make the row NaN where the reference's does.  The bitmask path (whose
    S accumulators start from 0 / -inf biases and re-mask exactly when a NaN
    shows) equals the scores-reading tile kernel bit for bit, NaN positions
    included, and the oracle's NaN positions and values elsewhere."""
    B, HQ, k = 1, 2, 40
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, dtype=BF, seed0=4)
    g = torch.Generator().manual_seed(23)
    rows = torch.randperm(T, generator=g)[:12].tolist()
    for i, r in enumerate(rows):
        K[0, r, i % HQ, (7 * i) % D] = (math.inf, -math.inf, math.nan)[i % 3]
    Q[0, T // 3, 1, 3] = math.inf
    s = torch.randn(B, T, T, generator=g)
    thr = kth(k)(s)
    args = (Q.to(dev), K.to(dev), V.to(dev))
    out = sparse_attention_hip(s.to(dev), thr.to(dev), *args, kernel="mask").cpu()
    ref = sparse_attention_hip(s.to(dev), thr.to(dev), *args, kernel="tiled").cpu()
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(out), nan)
    assert torch.equal(out.nan_to_num(0.0), ref.nan_to_num(0.0))
    want = O.sparse_attn_threshold(s, thr, Q, K, V)
    assert torch.equal(nan, torch.isnan(want))
    assert 0 < int(nan.sum()) < nan.numel()
    assert close(out[~nan], want[~nan], 2e-2, 2e-2)[0]


def test_mask_kernel_empty_rows_and_dense(dev):
    """NaN / +inf thresholds give NaN rows; -inf selects every causal key."""
    B, T, HQ, D = 1, 300, 2, 64
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, dtype=BF)
    s = torch.randn(B, T, T, generator=torch.Generator().manual_seed(5))
    thr = kth(16)(s)
    bad = torch.tensor([0, 7, 130, 299])
    thr[0, bad[:2], 0] = math.inf
    thr[0, bad[2:], 0] = math.nan
    args = (Q.to(dev), K.to(dev), V.to(dev))
    out = sparse_attention_hip(s.to(dev), thr.to(dev), *args, kernel="mask").cpu()
    assert bool(torch.isnan(out[0, bad]).all())
    good = torch.ones(T, dtype=torch.bool)
    good[bad] = False
    want = O.sparse_attn_threshold(s, thr, Q, K, V)
    assert close(out[0, good], want[0, good], 2e-2, 2e-2)[0]
    dense = torch.full((B, T, 1), -math.inf)
    out = sparse_attention_hip(s.to(dev), dense.to(dev), *args, kernel="mask").cpu()
    assert close(out, O.sparse_attn_threshold(s, dense, Q, K, V), 2e-2, 2e-2)[0]


def test_mask_path_is_the_default_for_tile_shapes(dev):
    """At T >= 4096 (16-bit, D = 128) the wrapper takes the bitmask path; its
    output equals the scores-reading tile kernel's bit for bit."""
    B, T, HQ, D = 1, 4096, 2, 128
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, dtype=BF)
    s = torch.randn(B, T, T, generator=torch.Generator().manual_seed(3)).to(dev)
    sd = s.masked_fill(~torch.ones(T, T, dtype=torch.bool, device=dev).tril(), -math.inf)
    thr = torch.topk(sd, 256, dim=-1).values[..., -1:].contiguous()
    args = (s, thr, Q.to(dev), K.to(dev), V.to(dev))
    a = sparse_attention_hip(*args)
    b = sparse_attention_hip(*args, kernel="tiled")
    assert torch.equal(a, b)
    rows = [0, 1, 63, 64, 127, 128, 2047, 4095]
    want = O.sparse_attn_threshold(s.cpu()[:, rows], thr.cpu()[:, rows], Q, K, V, rows=rows)
    assert close(a.cpu()[:, rows], want, 2e-2, 2e-2)[0]


# ---------------------------------------------------------------------------
# Wide attention rows.  The reference only asserts powers of two
# (dsa_attention.py:298-304); rows wider than one wave's registers (fp32
# HQ*D > 1024, 16-bit HQ*D > 2048) run as head-chunked gathers, or -- 16-bit,
# DQ = DV in {64, 128} -- on the tile kernel at any T.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,HQ,DQ,DV,T,k", [
    (torch.float32, 16, 128, 128, 512, 32),     # 2 head chunks
    (torch.float32, 16, 128, 128, 2048, 64),
    (torch.float32, 4, 512, 512, 256, 16),      # 2 chunks of 2 heads x 512
    (torch.float32, 32, 64, 128, 256, 20),      # DQ != DV, 4 chunks
    (torch.bfloat16, 128, 128, 128, 512, 32),   # tile kernel at T < 4096
    (torch.bfloat16, 128, 128, 128, 2048, 64),
    (torch.bfloat16, 16, 256, 256, 512, 32),    # no tile kernel for D=256: 2 chunks
    (torch.float16, 64, 64, 64, 256, 24),       # tile kernel, f16
])
def test_wide_rows_threshold_wrapper(dev, dtype, HQ, DQ, DV, T, k):
    """sparse_attention_with_threshold_triton on wide rows vs the float64
    oracle (1e-4 fp32, 2e-2 16-bit), sampled rows at T = 2048."""
    from helpers import sample_rows

    B = 1
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    say(f"wide attn B={B} T={T} HQ={HQ} DQ={DQ} DV={DV} {dtype}")
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, DQ, DV, dtype=dtype, seed0=3)
    g = torch.Generator().manual_seed(29)
    scores = torch.randn(B, T, T, generator=g)
    thr = kth(k)(scores)
    out = sparse_attention_with_threshold_triton(scores.to(dev), thr.to(dev), Q.to(dev),
                                                 K.to(dev), V.to(dev))
    torch.cuda.synchronize()
    rows = None if T <= 512 else sample_rows(T, 48, seed=1, include=(0, 1, k - 1, k, T - 1))
    if rows is None:
        want = O.sparse_attn_threshold(scores, thr, Q, K, V)
        got = out.cpu()
    else:
        want = O.sparse_attn_threshold(scores[:, rows], thr[:, rows], Q, K, V, rows=rows)
        got = out[:, rows].cpu()
    ok, err, _ = close(got, want, tol, tol)
    assert ok, f"max abs err {err}"


# ---------------------------------------------------------------------------
# Staged kernel (K/V streamed through LDS per block of 64 consecutive
# queries), forced at small T; the threshold entry point takes it for fp32
# rows of 512 at T >= 3072.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,T,HQ,D,k,dtype", [
    (1, 64, 8, 64, 8, torch.float32),       # two tiles, one pair
    (2, 96, 8, 64, 12, torch.float32),      # three tiles: the middle one alone
    (3, 200, 4, 64, 20, torch.float32),     # ragged T (not a multiple of 16 or 32)
    (1, 333, 8, 32, 40, torch.float32),     # E = 4 (row of 256), 8 lanes per head
    (2, 130, 2, 128, 16, torch.float32),    # E = 4, 32 lanes per head
    (1, 257, 1, 256, 30, torch.float32),    # one head of 256 (64 lanes per head)
    (2, 300, 8, 64, 40, torch.bfloat16),
    (1, 190, 4, 128, 25, torch.float16),
])
def test_staged_kth_threshold(dev, B, T, HQ, D, k, dtype):
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    run_case(dev, B, T, HQ, D, D, kth(k), dtype=dtype, rtol=tol, atol=tol, kernel="staged")


def test_staged_external_thresholds(dev):
    # -inf: every causal key (dense causal attention)
    run_case(dev, 2, 150, 8, 64, 64, lambda s: torch.full(s.shape[:2] + (1,), -math.inf),
             kernel="staged")
    # the diagonal score: keeps the keys scoring >= the s = t one
    run_case(dev, 2, 150, 8, 64, 64, lambda s: s.diagonal(0, 1, 2)[..., None].contiguous(),
             kernel="staged")


def test_staged_empty_rows_nan_and_large_logits(dev):
    """A NaN threshold selects nothing: NaN output, as the reference.  Large
    logits (Q, K scaled by 8) exercise the running-max rescale."""
    B, T, HQ, D = 1, 120, 8, 64
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, seed0=4)
    g = torch.Generator().manual_seed(6)
    scores = torch.randn(B, T, T, generator=g)
    thr = kth(10)(scores)
    thr[0, 5] = math.nan
    thr[0, 77] = math.nan
    out = sparse_attention_hip(scores.to(dev), thr.to(dev), (Q * 8).to(dev), (K * 8).to(dev),
                               V.to(dev), kernel="staged").cpu()
    assert bool(torch.isnan(out[0, 5]).all()) and bool(torch.isnan(out[0, 77]).all())
    keep = torch.ones(T, dtype=torch.bool)
    keep[[5, 77]] = False
    want = O.sparse_attn_threshold(scores, thr, Q * 8, K * 8, V)
    ok, err, _ = close(out[:, keep], want[:, keep], 1e-4, 1e-4)
    assert ok, f"max abs err {err}"


def test_staged_and_gather_agree(dev):
    """Same selection, two kernels: within fp32 rounding of each other."""
    B, T, HQ, D = 2, 700, 8, 64
    _, _, _, Q, K, V = (x.to(dev) for x in O.make_inputs(B, T, 1, 1, HQ, D, D, seed0=9))
    scores = torch.randn(B, T, T, generator=torch.Generator().manual_seed(1)).to(dev)
    thr = kth(70)(scores.cpu()).to(dev)
    a = sparse_attention_hip(scores, thr, Q, K, V, kernel="staged")
    b = sparse_attention_hip(scores, thr, Q, K, V)
    torch.cuda.synchronize()
    assert float((a - b).abs().max()) <= 1e-5


def test_staged_auto_at_config3_shape(dev):
    """B = 4, T = 4096 fp32, HQ = 8, D = 64 (config 3's attention): the
    threshold entry point runs the staged kernel (256 tiles of 64 queries, at
    least one per compute unit; long key ranges split over two blocks);
    sampled rows against the oracle."""
    from helpers import sample_rows

    B, T, HQ, D, k = 4, 4096, 8, 64, 256
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, seed0=12)
    scores = torch.randn(B, T, T, generator=torch.Generator().manual_seed(2))
    thr = kth(k)(scores)
    out = sparse_attention_with_threshold_triton(scores.to(dev), thr.to(dev), Q.to(dev),
                                                 K.to(dev), V.to(dev))
    forced = sparse_attention_hip(scores.to(dev), thr.to(dev), Q.to(dev), K.to(dev), V.to(dev),
                                  kernel="staged")
    torch.cuda.synchronize()
    assert torch.equal(out, forced), "T = 4096 fp32 must take the staged kernel"
    rows = sample_rows(T, 40, seed=3, include=(0, 1, 255, 256, 4095))
    want = O.sparse_attn_threshold(scores[:, rows], thr[:, rows], Q, K, V, rows=rows)
    ok, err, _ = close(out[:, rows].cpu(), want, 1e-4, 1e-4)
    assert ok, f"max abs err {err}"


def _staged_plain(scores, thr, Q, K, V):
    """The staged entry point without a workspace (no tile is split)."""
    B, T, HQ, D = Q.shape
    dt = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[Q.dtype]
    out = torch.empty(B, T, HQ, D, device=Q.device, dtype=torch.float32)
    rc = L.lib().dsa_sparse_attn_threshold_staged(
        scores.data_ptr(), T, thr.data_ptr(), Q.data_ptr(), K.data_ptr(), V.data_ptr(), dt, B, T,
        HQ, D, D, 1.0 / math.sqrt(D), out.data_ptr(), L.stream_ptr(Q.device))
    L.check(rc, "staged")
    return out


@pytest.mark.parametrize("B,T,HQ,D,k,dtype", [
    (1, 1300, 8, 64, 100, torch.float32),   # ragged T; tiles split into up to 3 chunks
    (2, 1100, 4, 64, 60, torch.float32),    # E = 4 (rows of 256)
    (1, 1000, 8, 64, 50, torch.bfloat16),
])
def test_staged_split_tiles(dev, B, T, HQ, D, k, dtype):
    """Shapes where the staged kernel splits long key ranges into chunks (a
    workspace from dsa_sparse_attn_workspace_bytes) and merges them: against
    the oracle, and against the same kernel run without the split."""
    nws = L.lib().dsa_sparse_attn_workspace_bytes(1, {torch.float32: 0, torch.bfloat16: 1}[dtype],
                                                  B, T, HQ, D, D, T)
    assert nws > 0, "this shape must split"
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    out = run_case(dev, B, T, HQ, D, D, kth(k), dtype=dtype, rtol=tol, atol=tol, kernel="staged")
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, dtype=dtype, seed0=0)
    g = torch.Generator().manual_seed(17)
    scores = torch.randn(B, T, T, generator=g)
    scores = torch.where(torch.rand(B, T, T, generator=g) < 0.1, 0.0, scores)
    thr = kth(k)(scores)
    plain = _staged_plain(scores.to(dev), thr.to(dev), Q.to(dev), K.to(dev), V.to(dev))
    torch.cuda.synchronize()
    assert float((out - plain).abs().max()) <= 1e-5


def test_staged_workspace_too_small_runs_unsplit(dev):
    """A workspace below dsa_sparse_attn_workspace_bytes (or misaligned)
    runs the staged kernel without the split: the plain entry point's result,
    bit for bit; the right size splits (equal within rounding)."""
    B, T, HQ, D, k = 1, 1300, 8, 64, 100
    _, _, _, Q, K, V = (x.to(dev) for x in O.make_inputs(B, T, 1, 1, HQ, D, D, seed0=41))
    scores = torch.randn(B, T, T, generator=torch.Generator().manual_seed(42))
    thr = kth(k)(scores).to(dev)
    scores = scores.to(dev)
    nws = L.lib().dsa_sparse_attn_workspace_bytes(1, 0, B, T, HQ, D, D, T)
    assert nws > 0
    ws = torch.empty(nws + 16, device=dev, dtype=torch.uint8)
    plain = _staged_plain(scores, thr, Q, K, V)

    def run(ptr, n):
        out = torch.empty(B, T, HQ, D, device=dev)
        rc = L.lib().dsa_sparse_attn_threshold_staged_ws(
            scores.data_ptr(), T, thr.data_ptr(), Q.data_ptr(), K.data_ptr(), V.data_ptr(), 0, B,
            T, HQ, D, D, 1.0 / math.sqrt(D), out.data_ptr(), ptr, n, L.stream_ptr(dev))
        L.check(rc, "staged_ws")
        return out

    small = run(ws.data_ptr(), nws - 1)
    misaligned = run(ws.data_ptr() + 4, nws)
    split = run(ws.data_ptr(), nws)
    torch.cuda.synchronize()
    assert torch.equal(small, plain) and torch.equal(misaligned, plain)
    assert float((split - plain).abs().max()) <= 1e-5


def test_staged_groups_mode(dev):
    """B*ceil(T/64) >= 2x the compute units: the staged kernel takes one
    64-query group per block (no tile pairs, no split).  All rows against
    the gathers (the threshold entry point's choice below T = 3072), sampled
    rows against the oracle."""
    from helpers import sample_rows

    B, T, HQ, D, k = 16, 2048, 8, 64, 100
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, seed0=31)
    scores = torch.randn(B, T, T, generator=torch.Generator().manual_seed(32))
    thr = kth(k)(scores)
    sd, td, Qd, Kd, Vd = (x.to(dev) for x in (scores, thr, Q, K, V))
    st = sparse_attention_hip(sd, td, Qd, Kd, Vd, kernel="staged")
    ga = sparse_attention_hip(sd, td, Qd, Kd, Vd)
    torch.cuda.synchronize()
    assert float((st - ga).abs().max()) <= 1e-5
    rows = sample_rows(T, 24, seed=5, include=(0, 63, 64, 2047))
    want = O.sparse_attn_threshold(scores[:3, rows], thr[:3, rows], Q[:3], K[:3], V[:3], rows=rows)
    ok, err, _ = close(st[:3, rows].cpu(), want, 1e-4, 1e-4)
    assert ok, f"max abs err {err}"


def test_staged_split_chunks_that_select_nothing(dev):
    """Rows of split tiles whose selection falls in one chunk only (the other
    chunks' partial sums are empty and weigh nothing), rows that select
    nothing at all (NaN threshold: NaN through the merge), every causal key
    (-inf threshold) and large logits."""
    B, T, HQ, D, k = 1, 1200, 8, 64, 50
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, seed0=21)
    g = torch.Generator().manual_seed(22)
    scores = torch.randn(B, T, T, generator=g)
    scores[0, 1100, :600] = -10.0    # top-k of row 1100 all in keys >= 600
    scores[0, 1101, 512:] = -10.0    # top-k of row 1101 all in keys < 512
    scores[0, 1150, :1100] = -10.0   # top-k of row 1150 all in the last keys
    thr = kth(k)(scores)
    thr[0, 1000] = math.nan
    thr[0, 1199] = math.nan
    thr[0, 900] = -math.inf
    out = sparse_attention_hip(scores.to(dev), thr.to(dev), (Q * 8).to(dev), (K * 8).to(dev),
                               V.to(dev), kernel="staged").cpu()
    assert bool(torch.isnan(out[0, 1000]).all()) and bool(torch.isnan(out[0, 1199]).all())
    keep = torch.ones(T, dtype=torch.bool)
    keep[[1000, 1199]] = False
    want = O.sparse_attn_threshold(scores, thr, Q * 8, K * 8, V)
    ok, err, _ = close(out[:, keep], want[:, keep], 1e-4, 1e-4)
    assert ok, f"max abs err {err}"


def test_staged_unsupported_shapes_raise(dev):
    s = torch.zeros(1, 64, 64, device=dev)
    t = torch.zeros(1, 64, 1, device=dev)
    for HQ, D, dt in ((4, 32, torch.float32), (8, 128, torch.float32), (8, 32, torch.bfloat16)):
        x = torch.zeros(1, 64, HQ, D, device=dev, dtype=dt)
        with pytest.raises(AssertionError):
            sparse_attention_hip(s, t, x, x, x, kernel="staged")
