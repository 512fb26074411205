"""CPU: the host k-th largest of the CPU-offload path (libdsa_cpu.so,
include/dsa_cpu.h) -- the replacement of the reference's AVX-512 extension
(topk_avx512.cpp:226-264).  Pinned against torch.topk (the reference's own
pin, test_topk_avx512.py:20-35), the reference's compiled source in
oracle/_ref (bit for bit), the committed vectors that build wrote, and
special values; both the AVX-512 and the scalar loop."""
from __future__ import annotations

import math
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import _dsa_lib as L
from oracle import native
from topk_threshold import topk_threshold, topk_threshold_batch_merge, topk_threshold_into

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")


def want(x, k):
    return x.topk(k, dim=-1).values[..., -1:]


def same(a, b):
    """Bitwise-equal float tensors, NaN equal to NaN."""
    return bool(((a == b) | (torch.isnan(a) & torch.isnan(b))).all()) and a.shape == b.shape


def test_reference_test_cases():
    """test_topk_avx512.py:20-35, run against this library."""
    torch.manual_seed(0)
    x = torch.randn(3, 128, 128, dtype=torch.float32)
    for k in (1, 8, 16, 32, 64, 96, 128):
        assert torch.equal(topk_threshold(x.contiguous(), k), want(x, k)), f"k={k}"
    torch.manual_seed(1)
    x = torch.randn(3, 128, 128, dtype=torch.float32)
    for k in (64, 128):
        assert torch.equal(topk_threshold_batch_merge(x.contiguous(), k), want(x, k)), f"k={k}"


def test_golden_reference_vectors():
    """Thresholds written by the reference's own compiled extension."""
    z = np.load(os.path.join(GOLD, "ref_topk.npz"))
    for x, ks, thr in ((z["x0"], z["ks0"], z["thr0"]), (z["x1"], z["ks1"], z["thr1"])):
        for i, k in enumerate(ks):
            got = topk_threshold(torch.from_numpy(x), int(k)).numpy()
            assert np.array_equal(got, thr[i]), f"k={k}"


@pytest.mark.skipif(not native.ref_available(), reason="oracle/_ref not built")
def test_matches_reference_build_bit_for_bit():
    ref = native.ref()
    if ref is None:
        pytest.skip("host CPU lacks the AVX-512 subsets oracle/_ref was built for")
    g = torch.Generator().manual_seed(4)
    for shape, k in (((16, 512, 512), 32), ((2, 512, 512), 128), ((4, 1000), 1),
                     ((8, 2048), 2048), ((3, 333), 17), ((64, 4096), 256)):
        x = torch.randn(shape, generator=g)
        x[x.abs() < 0.05] = 0.0            # ties
        assert torch.equal(topk_threshold(x, k), ref.topk_threshold(x, k)), (shape, k)
    # causal indexer-shaped rows (-inf above the diagonal), read causally here
    T = 300
    s = torch.randn(2, T, T, generator=g).masked_fill(
        ~torch.ones(T, T, dtype=torch.bool).tril(), -math.inf)
    for k in (1, 16, 299, 300):
        assert torch.equal(topk_threshold(s, k, causal=True), ref.topk_threshold(s, k)), k


@pytest.mark.parametrize("n", [1, 15, 16, 17, 100, 511, 512, 513, 2048, 5000])
@pytest.mark.parametrize("kfrac", [0.0, 0.1, 0.5, 1.0])
def test_random_rows(n, kfrac):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(7, n, generator=g)
    k = max(1, min(n, int(round(kfrac * n))))
    assert torch.equal(topk_threshold(x, k), want(x, k))


def test_ties_and_signed_zero():
    g = torch.Generator().manual_seed(2)
    x = torch.randint(-3, 4, (32, 700), generator=g).float()
    x[x == 0] = -0.0                       # -0 and +0 mixed: equal under >=
    x[:, ::3] = 0.0
    for k in (1, 2, 50, 233, 699, 700):
        got = topk_threshold(x, k)
        assert torch.equal(got, want(x, k)), k


def test_special_values():
    nan, inf = math.nan, math.inf
    x = torch.tensor([[nan, 1.0, 2.0, 3.0] * 5,
                      [-inf] * 20,
                      [inf, nan, -inf, 5.0] * 5,
                      [-0.0, 0.0] * 10,
                      [nan] * 20,
                      [1e-45, -1e-45, 3.4e38, -3.4e38] * 5])
    for k in range(1, 21):
        assert same(topk_threshold(x, k), want(x, k)), k


def test_mostly_neg_inf_rows():
    """Rows with fewer than k finite values: the k-th largest is -inf."""
    x = torch.full((5, 600), -math.inf)
    for i in range(5):
        x[i, torch.arange(i * 7, 600, 97)] = torch.arange(len(range(i * 7, 600, 97))).float()
    for k in (1, 3, 7, 8, 50, 600):
        assert torch.equal(topk_threshold(x, k), want(x, k)), k


def test_causal_rows_and_row_offset():
    T = 130
    g = torch.Generator().manual_seed(5)
    s = torch.randn(3, T, T, generator=g).masked_fill(
        ~torch.ones(T, T, dtype=torch.bool).tril(), -math.inf)
    for k in (1, 5, 64, 129, 130):
        assert torch.equal(topk_threshold(s, k, causal=True), want(s, k)), k
    # a block of rows starting inside a batch element (the hybrid path's
    # chunked copies): row0 places it
    lib = L.cpu_lib()
    flat = s.reshape(-1, T)
    r0, r1 = 170, 333
    out = torch.empty(r1 - r0)
    rc = lib.dsa_cpu_topk_threshold(flat.data_ptr() + r0 * T * 4, r1 - r0, T, T, 40, T, r0,
                                    out.data_ptr(), 0)
    assert rc == 0
    assert torch.equal(out, want(flat[r0:r1], 40).reshape(-1))


def test_into_and_thread_counts():
    x = torch.randn(33, 777, generator=torch.Generator().manual_seed(6))
    ref = want(x, 99)
    for nt in (1, 2, 3, 8):
        out = torch.empty(33, 1)
        assert topk_threshold_into(x, 99, out, nthreads=nt) is out
        assert torch.equal(out, ref), nt


def test_contract_errors():
    x = torch.randn(4, 16)
    with pytest.raises(RuntimeError, match="contiguous"):
        topk_threshold(x.t(), 2)
    with pytest.raises(RuntimeError, match="fp32"):
        topk_threshold(x.double(), 2)
    with pytest.raises(RuntimeError, match="k must be > 0"):
        topk_threshold(x, 0)
    with pytest.raises(RuntimeError, match="k must be <= N"):
        topk_threshold(x, 17)
    lib = L.cpu_lib()
    assert lib.dsa_cpu_topk_threshold(None, 4, 16, 16, 2, 0, 0, None, 0) == L.DSA_EINVAL
    assert lib.dsa_cpu_topk_threshold(None, 4, 16, 8, 2, 0, 0, None, 0) == L.DSA_EINVAL
    assert b"ld" in lib.dsa_cpu_last_error()
    assert lib.dsa_cpu_topk_threshold(None, 0, 16, 16, 2, 0, 0, None, 0) == L.DSA_OK


def test_scalar_loop_matches():
    """The scalar loop (hosts without AVX-512F), forced through the
    environment in a child process, gives the same thresholds."""
    code = (
        "import sys, math, torch; sys.path[:0] = [%r, %r];"
        "import _dsa_lib as L; from topk_threshold import topk_threshold;"
        "assert L.cpu_lib().dsa_cpu_isa() == 0;"
        "g = torch.Generator().manual_seed(8);"
        "x = torch.randn(40, 1500, generator=g); x[x.abs() < 0.1] = 0.0;"
        "x[3, 7] = math.nan; x[5] = -math.inf; x[6, :10] = math.inf;"
        "bad = [k for k in (1, 9, 64, 700, 1500)"
        "       if not bool(((topk_threshold(x, k) == x.topk(k, -1).values[..., -1:])"
        "                    | torch.isnan(x.topk(k, -1).values[..., -1:])).all())];"
        "assert not bad, bad; print('scalar ok')"
    ) % (os.path.join(ROOT, "dsa-cpu-topk_amd"), ROOT)
    env = dict(os.environ, DSA_CPU_ISA="scalar")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and "scalar ok" in r.stdout, r.stderr[-2000:]
