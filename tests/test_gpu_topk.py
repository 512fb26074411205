"""GPU: radix-select parity.  Thresholds and exactly-k index sets must be
bit-identical to the oracle on the same score matrix (north star: "top-K
index set bit-exact when selection is run on the same score matrix, with ties
broken by lowest index")."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import say
from oracle import dsa_oracle as O
from topk_threshold import (topk_indices, topk_threshold, topk_threshold_batch_merge,
                            topk_threshold_mask)

pytestmark = pytest.mark.gpu


def cpu_randn(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float32)


def check_rows(x_cpu, k, dev, causal=False, what=""):
    say(f"topk {what} shape={tuple(x_cpu.shape)} k={k} causal={causal}")
    thr, idx = topk_indices(x_cpu.to(dev), k, causal=causal)
    torch.cuda.synchronize()
    want_thr = O.topk_threshold(x_cpu, k)
    assert torch.equal(thr.cpu(), want_thr), "threshold differs from torch.topk k-th value"
    want_idx = O.select_indices(x_cpu.numpy(), k)
    got_idx = idx.cpu().numpy()
    bad = np.flatnonzero((got_idx != want_idx).any(-1).reshape(-1))
    assert bad.size == 0, f"{bad.size} rows with a different index set, first row {bad[:3]}"
    # threshold-only entry point agrees too
    assert torch.equal(topk_threshold(x_cpu.to(dev), k, causal=causal).cpu(), want_thr)


@pytest.mark.parametrize("rows,n,k", [
    (8, 1, 1), (16, 5, 3), (33, 100, 7), (7, 256, 1), (5, 256, 256), (9, 513, 32),
    (4, 1000, 999), (64, 2048, 128), (8, 4096, 256), (4, 8191, 100), (3, 16384, 2048),
    (2, 32768, 5000), (2, 40000, 1234), (1, 100003, 77),
    (3, 6000, 700), (2, 20000, 64), (2, 24576, 1000),
])
def test_random_rows(dev, rows, n, k):
    check_rows(cpu_randn((rows, n), rows * 1000 + n), k, dev, what="randn")


@pytest.mark.parametrize("n,k", [(64, 10), (512, 32), (2048, 128), (5000, 400), (40000, 3000)])
def test_tie_heavy_rows(dev, n, k):
    g = torch.Generator().manual_seed(n)
    x = torch.randint(0, 6, (6, n), generator=g).float()
    x[1] = 2.0                                           # one all-equal row
    x[2] = torch.where(torch.rand(n, generator=g) < 0.5, 0.0, -0.0)   # +-0 only
    x[3, : n // 2] = float("-inf")                       # half -inf
    x[4] = float("-inf")                                 # all -inf
    x[5, ::3] = float("inf")
    check_rows(x, k, dev, what="ties")


def test_special_values(dev):
    x = cpu_randn((4, 300), 9)
    x[0, 5] = float("inf")
    x[1] = torch.finfo(torch.float32).max * torch.sign(x[1])
    x[2] = torch.finfo(torch.float32).tiny * x[2]       # denormal-range magnitudes
    x[3, :] = -0.0
    for k in (1, 2, 150, 300):
        check_rows(x, k, dev, what="special")


@pytest.mark.parametrize("n", [300, 1000, 2048, 4096])
def test_nan_inf_rows_threshold_only(dev, n):
    """Threshold-only rows with non-finite values (rows up to 2048 entries
    take one wave per row, 4096 the block kernel): NaN is the largest value
    (torch.topk's order), +-inf and -0 as keys order them, and heavy ties
    take the radix fallback; every k checked against torch.topk."""
    g = torch.Generator().manual_seed(n)
    x = torch.randn((8, n), generator=g)
    x[0, ::7] = float("nan")
    x[1, ::5] = float("inf")
    x[1, 1::5] = float("-inf")
    x[2] = torch.where(torch.rand(n, generator=g) < 0.5, 1.0, float("nan"))
    x[3] = torch.randint(0, 3, (n,), generator=g).float()        # three values, heavy ties
    x[3, 17] = float("nan")
    x[4] = float("-inf")
    x[4, 3] = 0.0
    x[5] = torch.where(torch.rand(n, generator=g) < 0.5, 0.0, -0.0)
    x[6] = x[6] * 1e-42                                            # denormal magnitudes
    x[7, :] = 3.0e38
    x[7, ::3] = -3.0e38
    xg = x.to(dev)
    for k in sorted({1, 2, 7, n // 3, n // 2, n - 1, n}):
        say(f"topk nan/inf n={n} k={k}")
        torch.testing.assert_close(topk_threshold(xg, k).cpu(), O.topk_threshold(x, k),
                                   rtol=0, atol=0, equal_nan=True, msg=f"n={n} k={k}")


def nonfinite_rows(n, seed):
    """Rows of n entries with NaN, +-inf, heavy ties, +-0, denormals and a
    span that overflows (the cases the value bins of the register kernel
    must order exactly as keys do)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((8, n), generator=g)
    x[0, ::7] = float("nan")
    x[1, ::5] = float("inf")
    x[1, 1::5] = float("-inf")
    x[2] = torch.where(torch.rand(n, generator=g) < 0.5, 1.0, float("nan"))
    x[3] = torch.randint(0, 3, (n,), generator=g).float()
    x[3, 17] = float("nan")
    x[4] = float("-inf")
    x[4, 3] = 0.0
    x[5] = torch.where(torch.rand(n, generator=g) < 0.5, 0.0, -0.0)
    x[6] = x[6] * 1e-42
    x[7, :] = 3.0e38
    x[7, ::3] = -3.0e38
    return x


@pytest.mark.parametrize("n", [1000, 4096])
def test_nan_inf_rows_with_indices(dev, n):
    """Thresholds with exactly-k indices on rows with non-finite values
    (block kernel: value bins, NaN counted in the top bin and ranked first
    by key); index sets bit-exact against the stable descending sort."""
    x = nonfinite_rows(n, n + 1)
    xg = x.to(dev)
    for k in sorted({1, 7, n // 3, n - 1, n}):
        say(f"topk indices nan/inf n={n} k={k}")
        thr, idx = topk_indices(xg, k)
        torch.testing.assert_close(thr.cpu(), O.topk_threshold(x, k), rtol=0, atol=0,
                                   equal_nan=True, msg=f"n={n} k={k}")
        want = O.select_indices(x.numpy(), k)
        bad = np.flatnonzero((idx.cpu().numpy() != want).any(-1).reshape(-1))
        assert bad.size == 0, f"n={n} k={k}: rows {bad[:4]} differ"


def test_causal_nonfinite_rows_2d_grid(dev):
    """Causal rows of 1..4096 entries (the register kernel's 2-D grid: batch
    element x row, longest rows first) with non-finite scores in the causal
    part: thresholds and index sets equal the dense select on rows whose
    s > t entries are -inf."""
    B, T, k = 2, 4096, 256
    s = torch.randn((B, T, T), generator=torch.Generator().manual_seed(3))
    s[0, :, ::11] = float("nan")
    s[1, ::2, ::13] = float("inf")
    s[1, 1::2, 5::7] = float("-inf")
    dense = s.clone()
    dense[:, torch.ones(T, T, dtype=torch.bool).triu(1)] = float("-inf")
    rows = [0, 1, 2, 255, 256, 257, 1000, 2047, 2048, 4094, 4095]
    sg = s.to(dev)
    thr_c, idx_c = topk_indices(sg, k, causal=True)
    thr_t = topk_threshold(sg, k, causal=True)
    say(f"topk causal nonfinite B={B} T={T} k={k}")
    want_thr = O.topk_threshold(dense[:, rows], k)
    torch.testing.assert_close(thr_c[:, rows].cpu(), want_thr, rtol=0, atol=0, equal_nan=True)
    torch.testing.assert_close(thr_t[:, rows].cpu(), want_thr, rtol=0, atol=0, equal_nan=True)
    want_idx = O.select_indices(dense[:, rows].numpy(), k)
    assert np.array_equal(idx_c[:, rows].cpu().numpy(), want_idx)


def test_bracket_path_misses_fall_back(dev):
    """Threshold-only rows above 4096 entries are selected in one pass from a
    bracket that an evenly spread 4096-entry sample (chunks 0, 4, 8, 12 of
    1024 entries here) predicts.  Rows that the sample misrepresents, or whose
    bracket holds more keys than fit on chip, take the exact fallback: every
    row must still be bit-exact."""
    n = 16384
    x = cpu_randn((12, n), 77)
    x[1, 1024:2048] += 100.0                      # large values in a chunk the sample skips
    x[2, 1024:4096] -= 100.0                      # small values the sample skips
    x[3] = 1.0                                    # one value: every key kept
    x[4] = torch.randint(0, 3, (n,), generator=torch.Generator().manual_seed(4)).float()
    x[5] = torch.sort(x[5]).values                # ascending row
    x[6, 4096:5120] = float("inf")                # a sample chunk of +inf
    x[7, ::97] = float("nan")                     # NaN, the largest in torch.topk's order
    x[8, : n // 2] = float("-inf")                # half -inf
    x[9, 100:] = float("-inf")                    # almost all -inf
    x[10] = x[10] * 1e30                          # wide range
    x[11, 777] = 3e38                             # one huge outlier
    xg = x.to(dev)
    for k in (1, 100, 1024, 2048, 3000, 8000, 16383, 16384):
        say(f"topk bracket misses k={k}")
        torch.testing.assert_close(topk_threshold(xg, k).cpu(), O.topk_threshold(x, k),
                                   rtol=0, atol=0, equal_nan=True, msg=f"k={k}")


def mask_words_cpu(srow, t, thr, T):
    """Bitmask words of causal row t by the selection rule itself: bit i of
    word w set iff key 64w + i <= t and srow[key] >= thr; words 0 ..
    min(ceil(T/64) - 1, (t | 127) // 64)."""
    W = (T + 63) // 64
    nw = min(W, ((t | 127) >> 6) + 1)
    keys = np.arange(64 * nw)
    vals = np.full(64 * nw, np.nan, dtype=np.float32)
    vals[: min(64 * nw, T)] = srow[: min(64 * nw, T)]
    with np.errstate(invalid="ignore"):
        sel = (keys <= t) & (vals >= thr)
    bits = sel.reshape(nw, 64).astype(np.uint64) << np.arange(64, dtype=np.uint64)
    return np.bitwise_or.reduce(bits, axis=1).view(np.int64)


@pytest.mark.parametrize("B,T,k", [(1, 8192, 1), (1, 8192, 1000), (2, 4608, 300), (2, 2048, 64),
                                   (1, 8192, 8192), (1, 16448, 1000)])
def test_threshold_mask_matches_two_launches(dev, B, T, k):
    """topk_threshold_mask -- rows of 4097-16384 entries: the single-pass
    select writes each row's bitmask words from its own flag bitmap once it
    has the row's threshold (NaN, which indices rank first, selects nothing
    here); longer rows (T = 16448): it re-reads the row for them; shorter
    rows: the select and the mask kernel -- equals topk_threshold(causal)
    followed by selection_mask, bit for bit, on causal rows with NaN, +-inf,
    heavy ties, a large chunk the select's sample skips and short rows
    (t < k); entries above the diagonal hold 1e30, so a read past t shows.
    Sampled rows are also checked against the selection rule on the CPU."""
    from dsa_attention import selection_mask

    g = torch.Generator().manual_seed(T + k)
    s = torch.randn((B, T, T), generator=g)
    s[0, :, ::97] = float("nan")
    s[0, 3::5, 11::13] = float("inf")
    s[-1, 1::3, 7::17] = float("-inf")
    s[-1, ::4] = torch.randint(0, 3, (T,), generator=g).float()   # heavy ties
    s[0, T - 1, 1024:2048] += 100.0                                # outside the sample
    s[:, torch.ones(T, T, dtype=torch.bool).triu(1)] = 1e30
    sg = s.to(dev)
    say(f"topk+mask B={B} T={T} k={k}")
    thr2, mask2 = topk_threshold_mask(sg, k)
    thr1 = topk_threshold(sg, k, causal=True)
    mask1 = selection_mask(sg, thr1)
    torch.cuda.synchronize()
    torch.testing.assert_close(thr2.cpu(), thr1.cpu(), rtol=0, atol=0, equal_nan=True)
    W = (T + 63) // 64
    t = torch.arange(T)
    written = torch.arange(W)[None, :] <= torch.clamp((t | 127) // 64, max=W - 1)[:, None]
    m1, m2 = mask1.cpu(), mask2.cpu()
    assert torch.equal(m2[:, written], m1[:, written])
    thr_np, s_np, m2_np = thr2.cpu().numpy(), s.numpy(), m2.numpy()
    for b in range(B):
        for r in sorted({0, min(k, T) - 1, min(k, T - 1), T // 2, T - 1}):
            want = mask_words_cpu(s_np[b, r], r, thr_np[b, r, 0], T)
            assert np.array_equal(m2_np[b, r, : want.size], want), (b, r)


@pytest.mark.parametrize("k", [1, 2048, 16384])
def test_threshold_mask_config4_full(dev, k):
    """The select form the config-4 split forward runs -- topk_threshold_mask
    at B=1, T=16384 (the bracket kernel's MASK form, bitmap path) -- at full
    size: thresholds and every written bitmask word equal
    topk_threshold(causal) + selection_mask bit for bit on all 16384 rows,
    with NaN columns, +-inf entries, heavy-tie rows, a chunk the sample
    skips and 1e30 above the diagonal (a read past t shows); sampled rows
    against the selection rule on the CPU.  k = 1 (NaN rows give a NaN
    threshold), 2048 (config 4), 16384 (every row but the last is short)."""
    from dsa_attention import selection_mask

    T = 16384
    g = torch.Generator(device=dev).manual_seed(1000 + k)
    s = torch.randn((1, T, T), generator=g, device=dev)
    s[0, :, ::97] = float("nan")
    s[0, 3::5, 11::13] = float("inf")
    s[0, 1::3, 7::17] = float("-inf")
    s[0, ::4] = torch.randint(0, 3, (T,), generator=g, device=dev).float()   # heavy ties
    s[0, T - 1, 1024:2048] += 100.0                                         # outside the sample
    s[0].masked_fill_(torch.ones(T, T, dtype=torch.bool, device=dev).triu_(1), 1e30)
    say(f"topk+mask config-4 full size k={k}")
    thr2, mask2 = topk_threshold_mask(s, k)
    thr1 = topk_threshold(s, k, causal=True)
    mask1 = selection_mask(s, thr1)
    torch.cuda.synchronize()
    torch.testing.assert_close(thr2, thr1, rtol=0, atol=0, equal_nan=True)
    W = T // 64
    t = torch.arange(T, device=dev)
    written = torch.arange(W, device=dev)[None, :] <= torch.clamp((t | 127) // 64, max=W - 1)[:, None]
    assert torch.equal(mask2[:, written], mask1[:, written])
    del mask1
    thr_np = thr2.cpu().numpy()
    for r in sorted({0, 1, min(k, T) - 1, min(k, T - 1), 4096, T // 2, T - 2, T - 1}):
        want = mask_words_cpu(s[0, r].cpu().numpy(), r, thr_np[0, r, 0], T)
        assert np.array_equal(mask2[0, r, : want.size].cpu().numpy(), want), r
    # thresholds of sampled rows against the oracle on the same entries
    rows = [0, 2047, 2048, 9999, T - 1]
    srows = s[0, rows].cpu()
    causal = torch.arange(T)[None, :] <= torch.tensor(rows)[:, None]
    want_thr = O.topk_threshold(srows.masked_fill(~causal, float("-inf")), k)
    torch.testing.assert_close(thr2[0, rows].cpu(), want_thr, rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize("T,k,plant", [(12288, 3000, False), (16380, 2048, True),
                                       (9216, 700, True)])
def test_threshold_mask_bitmap_path_other_lengths(dev, T, k, plant):
    """The bitmap form of topk_threshold_mask (rows of 4097-16384 entries) at
    row counts that are not powers of two -- partial last chunks, between
    9 and 16 chunks of 1024 entries per row, and causal rows of every length
    below -- bit for bit against topk_threshold(causal) + selection_mask on
    every written word; with NaN columns, +-inf and heavy ties planted, or on
    plain N(0,1) scores, whose rows keep hundreds of values in the sample
    bracket (the kept-value walks and the wave that finishes the row)."""
    from dsa_attention import selection_mask

    g = torch.Generator(device=dev).manual_seed(T + k)
    s = torch.randn((1, T, T), generator=g, device=dev)
    if plant:
        s[0, :, ::89] = float("nan")
        s[0, 5::7, 3::11] = float("inf")
        s[0, 2::5, 9::13] = float("-inf")
        s[0, ::6] = torch.randint(0, 4, (T,), generator=g, device=dev).float()
    s[0].masked_fill_(torch.ones(T, T, dtype=torch.bool, device=dev).triu_(1), 1e30)
    say(f"topk+mask bitmap path T={T} k={k} plant={plant}")
    thr2, mask2 = topk_threshold_mask(s, k)
    thr1 = topk_threshold(s, k, causal=True)
    mask1 = selection_mask(s, thr1)
    torch.cuda.synchronize()
    torch.testing.assert_close(thr2, thr1, rtol=0, atol=0, equal_nan=True)
    W = (T + 63) // 64
    t = torch.arange(T, device=dev)
    written = torch.arange(W, device=dev)[None, :] <= torch.clamp((t | 127) // 64, max=W - 1)[:, None]
    assert torch.equal(mask2[:, written], mask1[:, written])
    thr_np = thr2.cpu().numpy()
    for r in sorted({min(k, T - 1), 4095, 4096, T // 2 + 1, T - 1}):
        want = mask_words_cpu(s[0, r].cpu().numpy(), r, thr_np[0, r, 0], T)
        assert np.array_equal(mask2[0, r, : want.size].cpu().numpy(), want), r


@pytest.mark.parametrize("k", [1, 100, 2048, 3000, 16383])
def test_bracket_indices_single_pass(dev, k):
    """Thresholds with exactly-k indices of rows up to 16384 entries come from
    the bracket kernel's single read: the same rows as above (sample misses,
    one value, three values, ascending, +inf chunk, NaN, -inf halves, wide
    range, outlier) plus ragged lengths, every index set against the oracle
    (lowest positions win ties, ascending order)."""
    n = 16384
    x = cpu_randn((12, n), 77)
    x[1, 1024:2048] += 100.0
    x[2, 1024:4096] -= 100.0
    x[3] = 1.0
    x[4] = torch.randint(0, 3, (n,), generator=torch.Generator().manual_seed(4)).float()
    x[5] = torch.sort(x[5]).values
    x[6, 4096:5120] = float("inf")
    x[7, ::97] = float("nan")
    x[8, : n // 2] = float("-inf")
    x[9, 100:] = float("-inf")
    x[10] = x[10] * 1e30
    x[11, 777] = 3e38
    say(f"topk bracket+indices k={k}")
    thr, idx = topk_indices(x.to(dev), k)
    torch.testing.assert_close(thr.cpu(), O.topk_threshold(x, k), rtol=0, atol=0, equal_nan=True)
    got = idx.cpu().numpy()
    want = O.select_indices(x.numpy(), k)
    bad = np.flatnonzero((got != want).any(-1))
    assert bad.size == 0, f"rows {bad} with a different index set"
    for m in (4097, 5000, 9999):
        check_rows(cpu_randn((3, m), m), min(k, m), dev, what="bracket+indices ragged")


def test_reference_extension_test_cases(dev):
    """test_topk_avx512.py:20-35 on the GPU drop-in: torch.equal vs torch.topk."""
    torch.manual_seed(0)
    x = torch.randn(3, 128, 128, dtype=torch.float32)
    for k in (1, 8, 16, 32, 64, 96, 128):
        ref = x.topk(k, dim=-1).values[..., -1:]
        assert torch.equal(topk_threshold(x.to(dev), k).cpu(), ref), f"k={k}"
    torch.manual_seed(1)
    x = torch.randn(3, 128, 128, dtype=torch.float32)
    for k in (64, 128):
        ref = x.topk(k, dim=-1).values[..., -1:]
        assert torch.equal(topk_threshold_batch_merge(x.to(dev), k).cpu(), ref), f"k={k}"


def test_golden_reference_vectors(dev):
    """The reference's own compiled extension's outputs (tests/golden/ref_topk.npz)."""
    import os

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_topk.npz"))
    for x, ks, thr in ((z["x0"], z["ks0"], z["thr0"]), (z["x1"], z["ks1"], z["thr1"])):
        xg = torch.from_numpy(x).to(dev)
        for i, k in enumerate(ks):
            assert np.array_equal(topk_threshold(xg, int(k)).cpu().numpy(), thr[i]), f"k={k}"


def test_standalone_c2_topk_vs_torch_topk_sets(dev):
    """Config 2 standalone top-K: [64,2048,2048] N(0,1), k=128; thresholds
    bit-exact and index sets equal to torch.topk's (tie-free data)."""
    say("topk c2 standalone [64,2048,2048] k=128")
    x = torch.randn((64, 2048, 2048), generator=torch.Generator().manual_seed(2),
                    dtype=torch.float32)
    xg = x.to(dev)
    thr, idx = topk_indices(xg, 128)
    tv, ti = torch.topk(xg, 128, dim=-1)
    torch.cuda.synchronize()
    assert torch.equal(thr, tv[..., -1:])
    assert torch.equal(torch.sort(idx.long(), dim=-1).values, torch.sort(ti, dim=-1).values)
    rows = [0, 77, 4095, 131071]
    xr = x.reshape(-1, 2048)[rows]
    assert np.array_equal(idx.reshape(-1, 128)[rows].cpu().numpy(), O.select_indices(xr.numpy(), 128))


def test_causal_mode_on_indexer_scores(dev):
    """Causal select on indexer score matrices: reads only s <= t; rows with
    t+1 < k give -inf and indices 0..k-1."""
    from lightning_indexer import indexer_scores_hip

    for (B, T, HI, DI, k) in ((2, 512, 4, 32, 32), (2, 300, 4, 32, 64), (1, 2048, 8, 64, 256)):
        q, kk, w, *_ = O.make_inputs(B, T, HI, DI, 1, 1, 1, seed0=T)
        s = indexer_scores_hip(q.to(dev), kk.to(dev), w.to(dev), write_upper=True)
        check_rows(s.cpu(), k, dev, causal=True, what=f"causal T={T}")
        # garbage above the diagonal must not matter in causal mode
        g = s.clone()
        upper = torch.ones(T, T, dtype=torch.bool, device=dev).triu(1)
        g[:, upper] = float("nan")
        thr_c, idx_c = topk_indices(g, k, causal=True)
        thr_f, idx_f = topk_indices(s, k, causal=False)
        assert torch.equal(thr_c, thr_f) and torch.equal(idx_c, idx_f)


def test_causal_c4_shape_properties(dev):
    """Config-4 shape (T=16384, k=2048) at full size: size-independent
    properties on every row, bit-exact on sampled rows."""
    T, k = 16384, 2048
    say("topk causal c4-shape T=16384 k=2048")
    g = torch.Generator(device=dev).manual_seed(4)
    s = torch.randn((1, T, T), generator=g, device=dev, dtype=torch.float32)
    s = torch.where(torch.rand((1, T, T), generator=g, device=dev) < 0.05, 0.0, s)  # zero ties
    thr, idx = topk_indices(s, k, causal=True)
    # the threshold-only entry point (one-pass bracket kernel) agrees
    assert torch.equal(topk_threshold(s, k, causal=True), thr)
    torch.cuda.synchronize()
    tril = torch.ones(T, T, dtype=torch.bool, device=dev).tril()
    masked = s.masked_fill(~tril, float("-inf"))
    n_gt = (masked > thr).sum(-1)[0]
    n_ge = (masked >= thr).sum(-1)[0]
    long_rows = torch.arange(T, device=dev) + 1 >= k
    assert bool((n_gt[long_rows] < k).all()) and bool((n_ge[long_rows] >= k).all())
    assert bool(torch.isneginf(thr[0, ~long_rows, 0]).all())
    # every emitted index is a valid position whose score passes the threshold
    vals = torch.gather(masked[0], 1, idx[0].long())
    assert bool((vals >= thr[0]).all())
    srt = torch.sort(idx[0].long(), dim=-1).values
    assert bool((srt[:, 1:] > srt[:, :-1]).all()), "indices must be distinct and ascending"
    del masked
    rows = [0, 1, k - 2, k - 1, k, 5000, T - 2, T - 1]
    sub = s[0, rows].cpu()
    sub = sub.masked_fill(torch.arange(T)[None, :] > torch.tensor(rows)[:, None], float("-inf"))
    assert torch.equal(thr[0, rows].cpu(), O.topk_threshold(sub, k))
    assert np.array_equal(idx[0, rows].cpu().numpy(), O.select_indices(sub.numpy(), k))
