"""CPU: pin the oracle (oracle/dsa_oracle.py) before trusting it.

Each oracle function is checked against something that does not share its
formula: plain loops, closed forms, numpy sorting, this repo's C++ port of
the reference's AVX-512 extension, the reference's own compiled extension
(oracle/_ref, when built) and the golden fixtures.  The last test plants
plausible mistakes in copies of the oracle (on the CPU) and checks that the
pins catch every one of them.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O
from oracle import native

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")


# ---------------------------------------------------------------------------
# Pin checks (each returns True when the given implementation passes)
# ---------------------------------------------------------------------------
def pin_indexer_loops(indexer) -> bool:
    """Against the per-(t,s) loop on odd shapes (catches transposes, wrong axes)."""
    q, k, w, *_ = O.make_inputs(2, 11, 3, 5, 1, 1, 1, seed0=7)
    got = indexer(q, k, w).numpy()
    ref = O.indexer_scores_naive(q, k, w)
    return bool(np.array_equal(np.isinf(got), np.isinf(ref))) and \
        bool(np.allclose(np.where(np.isinf(ref), 0, got), np.where(np.isinf(ref), 0, ref),
                         rtol=1e-12, atol=1e-12))


def pin_indexer_closed_forms(indexer) -> bool:
    T, DI = 6, 4
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, T, 1, DI, generator=g, dtype=torch.float64)
    # (a) k_s = q_s, w = 1: diagonal = |q_t|^2 (ReLU of a positive dot)
    s = indexer(q, q[:, :, 0].clone(), torch.ones(1, T, 1, dtype=torch.float64))
    ok = torch.allclose(torch.diagonal(s[0]), (q[0, :, 0] ** 2).sum(-1), rtol=1e-12)
    # (b) k_s = -q_s: diagonal dot < 0 -> ReLU 0 -> exactly 0
    s = indexer(q, -q[:, :, 0].clone(), torch.full((1, T, 1), 2.0, dtype=torch.float64))
    ok &= bool((torch.diagonal(s[0]) == 0).all())
    # (c) w = 0 -> every causal entry exactly 0, every s > t exactly -inf
    s = indexer(q, q[:, :, 0].clone(), torch.zeros(1, T, 1, dtype=torch.float64))
    tril = torch.ones(T, T, dtype=torch.bool).tril()
    ok &= bool((s[0][tril] == 0).all()) and bool(torch.isneginf(s[0][~tril]).all())
    # (d) w = -1 on a positive dot -> negative score (the sign of w is kept)
    s = indexer(q, q[:, :, 0].clone(), -torch.ones(1, T, 1, dtype=torch.float64))
    ok &= bool((torch.diagonal(s[0]) < 0).all())
    return bool(ok)


def pin_threshold(threshold) -> bool:
    """Against numpy sorting, the C++ port and (if built) the reference build."""
    rng = np.random.default_rng(11)
    rows = [rng.standard_normal((4, 37)).astype(np.float32),
            rng.integers(0, 4, (4, 37)).astype(np.float32),          # heavy ties
            np.concatenate([rng.standard_normal((4, 20)),
                            np.full((4, 17), -np.inf)], 1).astype(np.float32)]
    ref = native.ref()
    for x in rows:
        for k in (1, 2, 5, 17, 20, 36, 37):
            got = np.asarray(threshold(torch.from_numpy(x), k)).reshape(-1)
            want = np.sort(x, axis=-1)[:, -k]
            if not np.array_equal(got, want):
                return False
            if not np.array_equal(native.port_topk_threshold(x, k).reshape(-1), want):
                return False
            if ref is not None and not np.array_equal(
                    ref.topk_threshold(torch.from_numpy(x).contiguous(), k).numpy().reshape(-1),
                    want):
                return False
    return True


def _brute_select(row, k):
    order = sorted(range(len(row)), key=lambda i: (-float(row[i]), i))
    return sorted(order[:k])


def pin_select(select) -> bool:
    """Against an explicit (value desc, index asc) sort, on rows with ties,
    +-0.0 and -inf."""
    rng = np.random.default_rng(5)
    cases = [rng.standard_normal((3, 23)).astype(np.float32),
             rng.integers(-2, 3, (3, 23)).astype(np.float32),
             np.where(rng.random((3, 23)) < 0.5, 0.0, -0.0).astype(np.float32),
             np.concatenate([rng.integers(0, 2, (3, 9)), np.full((3, 14), -np.inf)],
                            1).astype(np.float32)]
    for x in cases:
        for k in (1, 3, 9, 12, 23):
            got = np.asarray(select(x, k))
            for r in range(x.shape[0]):
                if list(got[r]) != _brute_select(x[r], k):
                    return False
    return True


def pin_attention(attn) -> bool:
    B, T, HQ, D = 1, 7, 2, 3
    Q, K, V = (torch.randn(B, T, HQ, D, generator=torch.Generator().manual_seed(s),
                           dtype=torch.float64) for s in (1, 2, 3))
    # (a) row t keeps one key s*: output = V[s*]
    scores = torch.full((B, T, T), -1.0, dtype=torch.float64)
    star = [0, 1, 1, 2, 0, 4, 3]
    for t, s in enumerate(star):
        scores[0, t, s] = 5.0
    out = attn(scores, torch.full((B, T, 1), 5.0, dtype=torch.float64), Q, K, V)
    ok = all(torch.allclose(out[0, t], V[0, s], rtol=1e-12) for t, s in enumerate(star))
    # (b) Q = 0: equal logits -> mean of the kept V rows (keep s <= t with s even)
    scores = torch.zeros(B, T, T, dtype=torch.float64)
    scores[..., 1::2] = -1.0
    out = attn(scores, torch.zeros(B, T, 1, dtype=torch.float64), torch.zeros_like(Q), K, V)
    for t in range(T):
        keep = [s for s in range(t + 1) if s % 2 == 0]
        ok &= bool(torch.allclose(out[0, t], V[0, keep].mean(0), rtol=1e-12))
    # (c) threshold -inf keeps every causal key: dense causal softmax attention
    out = attn(torch.randn(B, T, T, dtype=torch.float64), torch.full((B, T, 1), -math.inf,
                                                                      dtype=torch.float64), Q, K, V)
    lg = torch.einsum("bthd,bshd->bhts", Q, K) / math.sqrt(D)
    lg = lg.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), -math.inf)
    dense = torch.einsum("bhts,bshd->bthd", torch.softmax(lg, -1), V)
    ok &= bool(torch.allclose(out, dense, rtol=1e-12, atol=1e-12))
    return bool(ok)


def pin_forward(forward) -> bool:
    """Against the plain-loop forward, at the reference test's small shapes."""
    for B, T, HI, DI, HQ, D, k in ((1, 16, 2, 16, 2, 16, 4), (2, 32, 2, 16, 2, 16, 8),
                                   (1, 24, 4, 8, 2, 4, 30)):
        ins = O.make_inputs(B, T, HI, DI, HQ, D, D, scale=0.3, w_scale=0.3, seed0=B * T)
        got = forward(*ins, k).numpy()
        if not np.allclose(got, O.dsa_forward_naive(*ins, k), rtol=1e-10, atol=1e-12):
            return False
    return True


# ---------------------------------------------------------------------------
# The oracle passes every pin
# ---------------------------------------------------------------------------
def test_indexer_matches_loops():
    assert pin_indexer_loops(lambda q, k, w: O.indexer_scores(q, k, w))


def test_indexer_closed_forms():
    assert pin_indexer_closed_forms(lambda q, k, w: O.indexer_scores(q, k, w))


def test_indexer_rows_subset_matches_full():
    ins = O.make_inputs(2, 40, 4, 8, 1, 1, 1)
    full = O.indexer_scores(*ins[:3])
    rows = [0, 7, 39, 22]
    assert torch.equal(O.indexer_scores(*ins[:3], rows=rows), full[:, rows])


def test_threshold_pins():
    assert pin_threshold(O.topk_threshold)


def test_threshold_short_causal_rows_are_neg_inf():
    s = O.indexer_scores(*O.make_inputs(1, 20, 4, 8, 1, 1, 1)[:3])
    thr = O.topk_threshold(s, 8)[0, :, 0]
    assert torch.isneginf(thr[:7]).all() and torch.isfinite(thr[7:]).all()


def test_select_pins():
    assert pin_select(O.select_indices)


def test_select_properties_at_size():
    x = np.random.default_rng(2).integers(0, 50, (16, 2048)).astype(np.float32)
    k = 128
    idx = O.select_indices(x, k)
    thr = O.topk_threshold(torch.from_numpy(x), k).numpy()
    for r in range(x.shape[0]):
        sel = x[r, idx[r]]
        assert len(set(idx[r].tolist())) == k
        assert (sel >= thr[r, 0]).all()
        assert (x[r] > thr[r, 0]).sum() <= k <= (x[r] >= thr[r, 0]).sum()
        ties = np.flatnonzero(x[r] == thr[r, 0])
        need = k - int((x[r] > thr[r, 0]).sum())
        assert set(idx[r][x[r, idx[r]] == thr[r, 0]].tolist()) == set(ties[:need].tolist())


def test_attention_pins():
    assert pin_attention(lambda s, th, Q, K, V: O.sparse_attn_threshold(s, th, Q, K, V))


def test_forward_pins():
    assert pin_forward(lambda *a: O.dsa_forward(*a))


def test_forward_rows_subset_matches_full():
    ins = O.make_inputs(1, 48, 4, 8, 2, 8, 8)
    full = O.dsa_forward(*ins, 6)
    rows = [47, 3, 20]
    assert torch.allclose(O.dsa_forward(*ins, 6, rows=rows), full[:, rows], rtol=1e-12)


def test_float32_mode_matches_float64_mode():
    ins = O.make_inputs(2, 64, 4, 32, 4, 32, 32)
    a = O.dsa_forward(*ins, 8, acc=torch.float32)
    b = O.dsa_forward(*ins, 8, acc=torch.float64)
    assert a.dtype == torch.float32
    assert torch.allclose(a.double(), b, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------------------
# Golden fixtures
# ---------------------------------------------------------------------------
def test_golden_c0_forward():
    z = np.load(os.path.join(GOLD, "c0_forward.npz"))
    ins = [torch.from_numpy(z[n]) for n in ("q_idx", "k_idx", "w_idx", "Q", "K", "V")]
    k = int(z["top_k"])
    out, scores, thr = O.dsa_forward(*ins, k, return_parts=True)
    assert np.allclose(scores.numpy(), z["scores"], rtol=1e-13, atol=0)
    assert np.array_equal(thr.numpy(), z["thr"])
    assert np.allclose(out.numpy(), z["out"], rtol=1e-12, atol=1e-13)
    assert np.array_equal(O.select_indices(scores.numpy(), k), z["idx"])
    # the reference's own compiled select on the fp32 scores
    assert np.array_equal(O.topk_threshold(torch.from_numpy(z["scores_f32"]), k).numpy(),
                          z["thr_ref"])


def test_golden_reference_topk_vectors():
    z = np.load(os.path.join(GOLD, "ref_topk.npz"))
    for x, ks, thr in ((z["x0"], z["ks0"], z["thr0"]), (z["x1"], z["ks1"], z["thr1"])):
        for i, k in enumerate(ks):
            want = thr[i]
            assert np.array_equal(O.topk_threshold(torch.from_numpy(x), int(k)).numpy(), want)
            assert np.array_equal(native.port_topk_threshold(x, int(k)), want)


@pytest.mark.skipif(not native.ref_available(), reason="oracle/_ref not built")
def test_reference_build_own_tests():
    """The reference's test_topk_avx512.py cases, run against its own build."""
    ref = native.ref()
    if ref is None:
        pytest.skip("host CPU lacks the AVX-512 subsets oracle/_ref was built for")
    torch.manual_seed(0)
    x = torch.randn(3, 128, 128, dtype=torch.float32)
    for k in (1, 8, 16, 32, 64, 96, 128):
        assert torch.equal(ref.topk_threshold(x.contiguous(), k), x.topk(k, dim=-1).values[..., -1:])
    torch.manual_seed(1)
    x = torch.randn(3, 128, 128, dtype=torch.float32)
    for k in (64, 128):
        assert torch.equal(ref.topk_threshold_batch_merge(x.contiguous(), k),
                           x.topk(k, dim=-1).values[..., -1:])


def test_port_scalar_and_avx512_agree():
    x = np.random.default_rng(9).standard_normal((64, 300)).astype(np.float32)
    for k in (1, 7, 32, 33, 200, 300):
        a = native.port_topk_threshold(x, k, use_avx512=False)
        b = native.port_topk_threshold(x, k, use_avx512=True)
        assert np.array_equal(a, b)
        assert np.array_equal(a[:, 0], np.sort(x, -1)[:, -k])


# ---------------------------------------------------------------------------
# Planted mistakes: every pin must catch its mutant
# ---------------------------------------------------------------------------
def _mut_indexer_no_relu(q, k, w):
    B, T, HI, DI = q.shape
    dots = torch.einsum("bthd,bsd->bths", q.double(), k.double())
    sc = (w.double().unsqueeze(-1) * dots).sum(2)
    return sc.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), -math.inf)


def _mut_indexer_mask_transposed(q, k, w):
    s = O.indexer_scores(q, k, w)
    T = s.shape[-1]
    s = s.masked_fill(torch.isinf(s), 0.0)
    return s.masked_fill(~torch.ones(T, T, dtype=torch.bool).triu(), -math.inf)


def _mut_indexer_qk_swapped(q, k, w):
    # scores[t,s] computed from q[s] and k[t]
    s = O.indexer_scores(q, k, w)
    B, T, HI, DI = q.shape
    dots = torch.einsum("bshd,btd->bths", q.double(), k.double())
    sc = (w.double().unsqueeze(-1) * torch.relu(dots)).sum(2)
    return sc.masked_fill(torch.isinf(s), -math.inf)


def _mut_threshold_off_by_one(x, k):
    return O.topk_threshold(x, min(k + 1, x.shape[-1]))


def _mut_threshold_unique_values(x, k):
    a = np.asarray(x, dtype=np.float32)
    out = []
    for r in a.reshape(-1, a.shape[-1]):
        u = np.unique(r)[::-1]
        out.append(u[min(k, len(u)) - 1])
    return np.array(out, dtype=np.float32)


def _mut_select_highest_index_ties(x, k):
    key = O.radix_key(x)[..., ::-1]
    order = np.argsort(-key, axis=-1, kind="stable")[..., :k]
    n = np.asarray(x).shape[-1]
    return np.sort(n - 1 - order, axis=-1)


def _mut_select_signed_zero(x, k):
    a = np.asarray(x, dtype=np.float32)
    key = a.view(np.uint32).astype(np.int64)
    key = np.where(key & 0x80000000, (~key) & 0xFFFFFFFF, key | 0x80000000)
    order = np.argsort(-key, axis=-1, kind="stable")[..., :k]
    return np.sort(order, axis=-1)


def _mut_attention_no_causal(s, th, Q, K, V):
    T = Q.shape[1]
    sel = s >= th
    lg = torch.einsum("bthd,bshd->bths", Q, K) / math.sqrt(Q.shape[-1])
    lg = lg.masked_fill(~sel.unsqueeze(2), -math.inf)
    return torch.einsum("bths,bshd->bthd", torch.softmax(lg, -1), V)


def _mut_attention_no_scale(s, th, Q, K, V):
    return O.sparse_attn_threshold(s, th, Q * math.sqrt(Q.shape[-1]), K, V)


def _mut_forward_strict_gt(*a):
    q, k, w, Q, K, V, top_k = a
    scores = O.indexer_scores(q, k, w)
    thr = O.topk_threshold(scores, min(top_k, Q.shape[1]))
    # '>' instead of '>=': drops the k-th key and its ties
    return O.sparse_attn_threshold(scores, torch.nextafter(thr, torch.tensor(math.inf,
                                   dtype=thr.dtype)), Q, K, V)


@pytest.mark.parametrize("pin,mutant", [
    (pin_indexer_loops, _mut_indexer_no_relu),
    (pin_indexer_loops, _mut_indexer_mask_transposed),
    (pin_indexer_loops, _mut_indexer_qk_swapped),
    (pin_indexer_closed_forms, _mut_indexer_no_relu),
    (pin_threshold, _mut_threshold_off_by_one),
    (pin_threshold, _mut_threshold_unique_values),
    (pin_select, _mut_select_highest_index_ties),
    (pin_select, _mut_select_signed_zero),
    (pin_attention, _mut_attention_no_causal),
    (pin_attention, _mut_attention_no_scale),
    (pin_forward, _mut_forward_strict_gt),
])
def test_pins_catch_planted_mistakes(pin, mutant):
    assert not pin(mutant)
