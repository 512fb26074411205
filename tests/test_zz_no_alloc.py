"""GPU: dsa_sparse_attn_mask_noalloc, the allocation-free bitmask attention
(its bitmask in the library's static per-GPU scratch), against the entry
points that take caller memory, through the C ABI, on the same inputs:
bit for bit, on two calls in a row (the second smaller, so the scratch
holds the first call's words past the second's rows)."""
from __future__ import annotations

import math

import pytest
import torch

import _dsa_lib as L
from helpers import say
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(dev, B, T, HQ, D, dtype, k, seed):
    _, _, _, Q, K, V = O.make_inputs(B, T, 1, 1, HQ, D, D, dtype=dtype, seed0=seed)
    g = torch.Generator().manual_seed(seed + 1)
    s = torch.randn(B, T, T, generator=g)
    s = torch.where(torch.rand(B, T, T, generator=g) < 0.1, 0.0, s)   # ties at 0
    causal = s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), -math.inf)
    thr = O.topk_threshold(causal, min(k, T))
    return dtype, [x.to(dev).contiguous() for x in (s, thr, Q, K, V)]


def _args(dt, s, thr, Q, K, V):
    B, T, HQ, D = Q.shape
    return B, T, HQ, D, L.dtype_code(dt), 1.0 / math.sqrt(D), L.stream_ptr(Q.device)


def _noalloc(dt, s, thr, Q, K, V):
    B, T, HQ, D, code, scale, st = _args(dt, s, thr, Q, K, V)
    out = torch.empty(B, T, HQ, D, device=Q.device)
    rc = L.lib().dsa_sparse_attn_mask_noalloc(
        s.data_ptr(), T, thr.data_ptr(), Q.data_ptr(), K.data_ptr(), V.data_ptr(), code, B, T, HQ,
        D, D, scale, out.data_ptr(), st)
    L.check(rc, "dsa_sparse_attn_mask_noalloc")
    return out


def _caller_mask(dt, s, thr, Q, K, V):
    B, T, HQ, D, code, scale, st = _args(dt, s, thr, Q, K, V)
    W = (T + 63) // 64
    mask = torch.empty(B, T, W, device=Q.device, dtype=torch.int64)
    L.check(L.lib().dsa_selection_mask(s.data_ptr(), T, thr.data_ptr(), B, T, mask.data_ptr(), W,
                                       st), "dsa_selection_mask")
    out = torch.empty(B, T, HQ, D, device=Q.device)
    L.check(L.lib().dsa_sparse_attn_mask(mask.data_ptr(), W, Q.data_ptr(), K.data_ptr(),
                                         V.data_ptr(), code, B, T, HQ, D, D, scale,
                                         out.data_ptr(), st), "dsa_sparse_attn_mask")
    return out


def _threshold_tiled(dt, s, thr, Q, K, V):
    B, T, HQ, D, code, scale, st = _args(dt, s, thr, Q, K, V)
    out = torch.empty(B, T, HQ, D, device=Q.device)
    L.check(L.lib().dsa_sparse_attn_threshold_tiled(
        s.data_ptr(), T, thr.data_ptr(), Q.data_ptr(), K.data_ptr(), V.data_ptr(), code, B, T, HQ,
        D, D, scale, out.data_ptr(), st), "dsa_sparse_attn_threshold_tiled")
    return out


def test_noalloc_two_calls_match_allocating_entry_points(dev):
    cases = [(2, 1000, 4, 128, torch.bfloat16, 100, 11),   # first call
             (1, 300, 2, 64, torch.float16, 40, 12)]       # second, smaller
    ins = [_inputs(dev, *c) for c in cases]
    got = []
    for c, (dt, x) in zip(cases, ins):
        say(f"noalloc B={c[0]} T={c[1]} HQ={c[2]} D={c[3]} {dt}")
        got.append(_noalloc(dt, *x))
    torch.cuda.synchronize()
    for c, (dt, x), a in zip(cases, ins, got):
        b = _caller_mask(dt, *x)
        t = _threshold_tiled(dt, *x)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"noalloc vs caller-allocated mask, case {c}"
        assert torch.equal(a, t), f"noalloc vs threshold tile kernel, case {c}"
        # and the oracle, at the 16-bit tolerance, on a few rows
        s, thr, Q, K, V = (y.cpu() for y in x)
        rows = [0, 1, c[1] // 2, c[1] - 1]
        want = O.sparse_attn_threshold(s[:, rows], thr[:, rows], Q, K, V, rows=rows)
        assert torch.allclose(a.cpu()[:, rows], want.float(), rtol=2e-2, atol=2e-2)


def test_noalloc_under_graph_capture(dev):
    """The entry point captured into a HIP graph: one eager call first (the
    library looks up the scratch array's address on a device's first call,
    outside the capture), then a capture on torch's capture stream, replayed
    three times with new inputs copied into the captured buffers and eager
    work between the replays; every replay is bit-equal to the caller-
    allocated two-launch form on the same inputs.  (The size check that
    refuses inputs past the scratch runs on the CPU in test_capi.py.)"""
    say("noalloc under graph capture")
    case = (1, 777, 4, 64, torch.bfloat16, 64, 21)
    dt, x = _inputs(dev, *case)
    eager = _noalloc(dt, *x)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured_out = _noalloc(dt, *x)
    for rep in range(3):
        _, fresh = _inputs(dev, *case[:-1], 100 + rep)
        for dst, src in zip(x, fresh):
            dst.copy_(src)
        g.replay()
        torch.cuda.synchronize()
        want = _caller_mask(dt, *x)
        torch.cuda.synchronize()
        assert torch.equal(captured_out, want), f"replay {rep} differs from the eager form"
        assert not torch.equal(captured_out, eager), "replay did not see the new inputs"
