"""GPU: MFMA lightning-indexer parity vs the float64 oracle (rtol/atol 1e-4
for fp32 inputs, 2e-2 for 16-bit inputs; off-causal entries exactly -inf)."""
from __future__ import annotations

import pytest
import torch

from helpers import close, say
from lightning_indexer import indexer_scores_hip, indexer_scores_triton, indexer_triton
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def run_case(dev, B, T, HI, DI, dtype=torch.float32, rtol=1e-4, atol=1e-4, seed0=0,
             rows=None, w_scale=None, scale=1.0):
    say(f"indexer B={B} T={T} HI={HI} DI={DI} {dtype}")
    q, k, w, *_ = O.make_inputs(B, T, HI, DI, 1, 1, 1, dtype=dtype, seed0=seed0,
                                w_scale=w_scale, scale=scale)
    s = indexer_scores_triton(q.to(dev), k.to(dev), w.to(dev)) if rows is None else \
        indexer_scores_hip(q.to(dev), k.to(dev), w.to(dev))
    torch.cuda.synchronize()
    got = s.cpu() if rows is None else s[:, rows].cpu()
    want = O.indexer_scores(q, k, w, rows=rows)
    ts = torch.arange(T) if rows is None else torch.tensor(rows)
    causal = torch.arange(T)[None, :] <= ts[:, None]
    ok, err, _ = close(got[:, causal], want[:, causal], rtol, atol)
    assert ok, f"max abs err {err}"
    assert bool(torch.isneginf(got[:, ~causal]).all()), "off-causal entries must be -inf"
    return s


@pytest.mark.parametrize("B,T,H,d", [(1, 64, 4, 64), (2, 128, 8, 64), (1, 200, 4, 32)])
def test_reference_shapes(dev, B, T, H, d):
    """test_indexer.py:18-33 (N(0,1) inputs, atol = rtol = 1e-4)."""
    run_case(dev, B, T, H, d, w_scale=1.0)


@pytest.mark.parametrize("B,T,HI,DI", [(1, 128, 4, 32), (16, 512, 4, 32), (2, 37, 3, 16),
                                       (3, 100, 2, 16), (1, 300, 5, 128), (1, 96, 9, 256),
                                       (2, 1024, 8, 64)])
def test_shapes_fp32(dev, B, T, HI, DI):
    run_case(dev, B, T, HI, DI)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,HI,DI", [(1, 256, 64, 128), (2, 130, 4, 32), (1, 200, 12, 64),
                                       (1, 64, 8, 256)])
def test_shapes_16bit(dev, dtype, B, T, HI, DI):
    # products of 16-bit inputs are exact in fp32 and the sum is fp32, so the
    # error is fp32 rounding only; 2e-2 is the north-star bound.
    run_case(dev, B, T, HI, DI, dtype=dtype, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("dtype,B,T,HI,DI", [(torch.float32, 1, 80, 64, 256),
                                              (torch.bfloat16, 2, 70, 160, 256)])
def test_wide_q_rows_stream_kernel(dev, dtype, B, T, HI, DI):
    """q rows too wide for a 4-query LDS tile (HI*DI*bytes > 40 KiB) take the
    register-streaming kernel."""
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    run_case(dev, B, T, HI, DI, dtype=dtype, rtol=tol, atol=tol)


def test_c3_shape_sampled_rows(dev):
    T = 4096
    rows = [0, 1, 15, 16, 255, 256, 1000, 2047, 4094, 4095]
    run_case(dev, 4, T, 8, 64, rows=rows)


def test_c4_shape_sampled_rows(dev):
    T = 16384
    rows = [0, 5, 2047, 2048, 9000, 16383]
    run_case(dev, 1, T, 64, 128, dtype=torch.bfloat16, rtol=2e-2, atol=2e-2, rows=rows)


def test_write_upper_false_leaves_upper_untouched(dev):
    q, k, w, *_ = O.make_inputs(2, 200, 4, 32, 1, 1, 1)
    out = torch.full((2, 200, 200), 123.0, device=dev)
    indexer_scores_hip(q.to(dev), k.to(dev), w.to(dev), write_upper=False, out=out)
    upper = torch.ones(200, 200, dtype=torch.bool, device=dev).triu(1)
    assert bool((out[:, upper] == 123.0).all())
    full = indexer_scores_hip(q.to(dev), k.to(dev), w.to(dev))
    assert torch.equal(out[:, ~upper], full[:, ~upper])


def test_projection_pipeline(dev):
    """test_indexer.py:36-48: projection (torch GEMMs) + MFMA indexer, 1e-3."""
    B, T, D, H, d = 2, 96, 128, 4, 64
    g = torch.Generator().manual_seed(0)
    h = torch.randn(B, T, D, generator=g)
    W_Q = torch.randn(D, H * d, generator=g) * 0.1
    W_K = torch.randn(D, d, generator=g) * 0.1
    W_W = torch.randn(D, H, generator=g) * 0.1
    out = indexer_triton(h.to(dev), W_Q.to(dev), W_K.to(dev), W_W.to(dev), H, d,
                         BLOCK_T=32, BLOCK_S=32).cpu()
    hq, hk, hw = (h.double() @ W.double() for W in (W_Q, W_K, W_W))
    ref = O.indexer_scores(hq.view(B, T, H, d), hk, hw)
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    assert float((out[:, causal].double() - ref[:, causal]).abs().max()) < 1e-3


def test_topk_mask_consistency(dev):
    """test_indexer.py:51-62: top-k masks from HIP scores and oracle scores
    agree (>99%; near-tie flips allowed), and the HIP mask has exactly k
    entries per row, the lowest indices winning ties."""
    from lightning_indexer import topk_mask

    B, T, H, d = 1, 64, 4, 64
    q, k, w, *_ = O.make_inputs(B, T, H, d, 1, 1, 1, w_scale=1.0)
    s = indexer_scores_triton(q.to(dev), k.to(dev), w.to(dev), BLOCK_T=32, BLOCK_S=32)
    m = topk_mask(s, 8).cpu()
    ref = O.indexer_scores(q, k, w)
    mref = torch.zeros(B, T, T, dtype=torch.bool)
    mref.scatter_(-1, torch.from_numpy(O.select_indices(ref.numpy(), 8)).long(), True)
    assert float((m == mref).float().mean()) > 0.99
    assert bool((m.sum(-1) == 8).all())
    mine = torch.zeros(B, T, T, dtype=torch.bool)
    mine.scatter_(-1, torch.from_numpy(O.select_indices(s.cpu().numpy(), 8)).long(), True)
    assert torch.equal(m, mine)


# ---------------------------------------------------------------------------
# fp8 (OCP E4M3) q_idx/k_idx with fp32 w: no reference counterpart (its
# kernel upcasts every load to fp32, lightning_indexer.py:81-91), so the
# oracle takes the e4m3 values upcast to float64.  E4M3 x E4M3 products are
# exact, but the fp8 MFMA's internal sum of its 128 products is not an IEEE
# fp32 sum (about 13-14 significant bits): measured max errors are 6e-4 to
# 2e-3 on scores of magnitude ~10, against ~1e-5 for the fp32 path, and
# reached 0.93 of a 1e-3 bound.  Bound: rtol = atol = 2e-3 (atol scaled with
# the operands), inside the 2e-2 low-precision bound.
# ---------------------------------------------------------------------------
def run_fp8_case(dev, B, T, HI, DI, *, seed0=0, rows=None, qk_scale=1.0):
    say(f"indexer fp8 B={B} T={T} HI={HI} DI={DI} scale={qk_scale}")
    q, k, w, *_ = O.make_inputs(B, T, HI, DI, 1, 1, 1, seed0=seed0)
    q8 = (q * qk_scale).to(torch.float8_e4m3fn)
    k8 = (k * qk_scale).to(torch.float8_e4m3fn)
    s = indexer_scores_hip(q8.to(dev), k8.to(dev), w.to(dev))
    torch.cuda.synchronize()
    got = s.cpu() if rows is None else s[:, rows].cpu()
    want = O.indexer_scores(q8, k8, w, rows=rows)
    ts = torch.arange(T) if rows is None else torch.tensor(rows)
    causal = torch.arange(T)[None, :] <= ts[:, None]
    tol = 2e-3 * qk_scale * qk_scale
    ok, err, excess = close(got[:, causal], want[:, causal], 2e-3, tol)
    say(f"  max abs err {err:.3g}, worst err/bound {excess:.3g}")
    assert ok, f"max abs err {err}"
    assert bool(torch.isneginf(got[:, ~causal]).all()), "off-causal entries must be -inf"


@pytest.mark.parametrize("B,T,HI,DI", [(1, 256, 64, 128), (2, 130, 4, 64), (1, 200, 12, 256),
                                       (3, 77, 5, 64), (16, 512, 4, 64)])
def test_fp8_shapes(dev, B, T, HI, DI):
    run_fp8_case(dev, B, T, HI, DI)


def test_fp8_subnormal_and_large_operands(dev):
    """Operands scaled by 2^-8 put much of q/k in E4M3's subnormal range
    (|x| < 2^-6); scaled by 2^5 they reach the top binades (max 448).  Both
    must come out as the exact upcast values' products."""
    run_fp8_case(dev, 1, 96, 8, 128, seed0=3, qk_scale=2.0 ** -8)
    run_fp8_case(dev, 1, 96, 8, 128, seed0=4, qk_scale=32.0)


def test_fp8_c4_shape_sampled_rows(dev):
    rows = [0, 5, 2047, 2048, 9000, 16383]
    run_fp8_case(dev, 1, 16384, 64, 128, rows=rows)


def test_fp8_wide_rows_unsupported(dev):
    """fp8 has no register-streaming kernel: q tiles beyond LDS are refused."""
    from _dsa_lib import DSAUnsupported

    q = torch.zeros(1, 8, 160, 256, device=dev).to(torch.float8_e4m3fn)
    k = torch.zeros(1, 8, 256, device=dev).to(torch.float8_e4m3fn)
    with pytest.raises(DSAUnsupported):
        indexer_scores_hip(q, k, torch.zeros(1, 8, 160, device=dev))


# ---------------------------------------------------------------------------
# Row-strided inputs and the fused projection front end
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype,B,T,HI,DI,pad", [(torch.float32, 2, 200, 4, 32, 4),
                                                  (torch.bfloat16, 1, 300, 8, 64, 8),
                                                  (torch.float32, 1, 96, 64, 256, 12)])
def test_strided_rows_equal_packed(dev, dtype, B, T, HI, DI, pad):
    """q, k, w as column ranges of one [B*T, HI*DI+DI+HI+pad] buffer give the
    packed entry point's scores bit for bit (same kernel, same values).  The
    last case takes the register-streaming kernel (q rows too wide for LDS)."""
    import _dsa_lib as L

    say(f"strided indexer {dtype} B={B} T={T} HI={HI} DI={DI}")
    q, k, w, *_ = O.make_inputs(B, T, HI, DI, 1, 1, 1, dtype=dtype, seed0=9)
    RS = HI * DI + DI + HI + pad
    buf = torch.zeros(B * T, RS, dtype=dtype)
    buf[:, :HI * DI] = q.reshape(B * T, HI * DI)
    buf[:, HI * DI:HI * DI + DI] = k.reshape(B * T, DI)
    buf[:, HI * DI + DI:HI * DI + DI + HI] = w.reshape(B * T, HI)
    buf = buf.to(dev)
    want = indexer_scores_hip(q.to(dev), k.to(dev), w.to(dev))
    got = torch.empty(B, T, T, device=dev)
    es, base = buf.element_size(), buf.data_ptr()
    rc = L.lib().dsa_indexer_scores_strided(
        base, base + HI * DI * es, base + (HI * DI + DI) * es, L.dtype_code(dtype), B, T, HI,
        DI, RS, RS, RS, got.data_ptr(), T, 1, L.stream_ptr(dev))
    L.check(rc, "strided")
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
def test_projection_front_end_fused(dev, dtype, tol):
    """indexer_from_hidden (one GEMM read in place) against the float64 oracle
    of project() + indexer (test_indexer.py:36-48 tolerance for fp32)."""
    from lightning_indexer import indexer_from_hidden

    B, T, D, H, d = 2, 160, 256, 8, 64
    g = torch.Generator().manual_seed(5)
    h = torch.randn(B, T, D, generator=g)
    W_Q = torch.randn(D, H * d, generator=g) * 0.06
    W_K = torch.randn(D, d, generator=g) * 0.06
    W_W = torch.randn(D, H, generator=g) * 0.06
    hd, Wq, Wk, Ww = (x.to(dtype) for x in (h, W_Q, W_K, W_W))
    out = indexer_from_hidden(hd.to(dev), Wq.to(dev), Wk.to(dev), Ww.to(dev), H, d).cpu()
    hq, hk, hw = (hd.double() @ W.double() for W in (Wq, Wk, Ww))
    ref = O.indexer_scores(hq.view(B, T, H, d), hk, hw)
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    err = float((out[:, causal].double() - ref[:, causal]).abs().max())
    scale = float(ref[:, causal].abs().max())
    assert err <= tol * max(1.0, scale), f"max abs err {err} (scale {scale})"
    assert bool(torch.isneginf(out[:, ~causal]).all())


def test_projection_weights_replaced_between_calls(dev):
    """indexer_triton with weight set A, then A freed and set B of the same
    shape and dtype (the caching allocator tends to hand B A's blocks): each
    call must match the float64 oracle of its own weights (1e-3, the
    reference's projection tolerance, test_indexer.py:36-48)."""
    import gc

    B, T, D, H, d = 2, 96, 128, 4, 64
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    h = torch.randn(B, T, D, generator=torch.Generator().manual_seed(21))
    hd = h.to(dev)
    reused = 0
    last_ptrs = None
    for trial in range(4):
        g = torch.Generator().manual_seed(100 + trial)
        Ws = [torch.randn(D, n, generator=g) * 0.06 for n in (H * d, d, H)]
        Wd = [W.to(dev) for W in Ws]
        ptrs = tuple(W.data_ptr() for W in Wd)
        same = ptrs == last_ptrs
        reused += same
        last_ptrs = ptrs
        say(f"projection weights trial {trial} (same addresses as before: {same})")
        out = indexer_triton(hd, *Wd, H, d).cpu()
        hq, hk, hw = (h.double() @ W.double() for W in Ws)
        ref = O.indexer_scores(hq.view(B, T, H, d), hk, hw)
        err = float((out[:, causal].double() - ref[:, causal]).abs().max())
        scale = float(ref[:, causal].abs().max())
        assert err <= 1e-3 * max(1.0, scale), f"trial {trial}: max abs err {err} (scale {scale})"
        del Wd, out
        gc.collect()
    say(f"weights landed at the previous set's addresses in {reused} of 3 replacements")


# ---------------------------------------------------------------------------
# fp8 with quantisation scales (dsa_indexer_scores_fp8_scaled): q quantised
# per (token, head) row and k per token to E4M3 with scale = amax / 448, the
# layout of a block-128 activation quantisation (the reference's fp8
# follow-up, DEVLOG.md:203-205).  Oracle: the float64 indexer of the
# dequantised values scale * e4m3, which is what the kernel computes
# (positive scales factor out of the ReLU); bound as for unscaled fp8.
# ---------------------------------------------------------------------------
def quantise_rows(x, dim_last):
    """e4m3 values and positive per-row scales (amax over the last dim / 448)."""
    amax = x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12)
    scale = amax / 448.0
    return (x / scale).to(torch.float8_e4m3fn), scale.squeeze(-1)


@pytest.mark.parametrize("B,T,HI,DI", [(1, 256, 64, 128), (2, 130, 4, 64), (1, 200, 12, 256)])
def test_fp8_scaled_against_dequantised_oracle(dev, B, T, HI, DI):
    say(f"indexer fp8 scaled B={B} T={T} HI={HI} DI={DI}")
    q, k, w, *_ = O.make_inputs(B, T, HI, DI, 1, 1, 1, seed0=7)
    # spread the rows' magnitudes over several binades so the scales differ
    g = torch.Generator().manual_seed(8)
    q = q * torch.exp2(torch.randint(-4, 5, (B, T, HI, 1), generator=g).float())
    k = k * torch.exp2(torch.randint(-4, 5, (B, T, 1), generator=g).float())
    q8, qs = quantise_rows(q, DI)
    k8, ks = quantise_rows(k, DI)
    s = indexer_scores_hip(q8.to(dev), k8.to(dev), w.to(dev), q_scale=qs.to(dev),
                           k_scale=ks.to(dev))
    torch.cuda.synchronize()
    got = s.cpu()
    want = O.indexer_scores(q8.double() * qs.double()[..., None],
                            k8.double() * ks.double()[..., None], w)
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    mag = float(want[:, causal].abs().max())
    ok, err, excess = close(got[:, causal], want[:, causal], 2e-3, 2e-3 * max(1.0, mag / 10))
    say(f"  max abs err {err:.3g} (scores up to {mag:.3g}), worst err/bound {excess:.3g}")
    assert ok, f"max abs err {err}"
    assert bool(torch.isneginf(got[:, ~causal]).all()), "off-causal entries must be -inf"


def test_fp8_unit_scales_equal_unscaled(dev):
    """Scales of 1 (either or both) give the unscaled fp8 kernel's scores
    bit for bit."""
    B, T, HI, DI = 2, 150, 8, 128
    q, k, w, *_ = O.make_inputs(B, T, HI, DI, 1, 1, 1, seed0=9)
    q8, k8 = (x.to(torch.float8_e4m3fn).to(dev) for x in (q, k))
    w = w.to(dev)
    base = indexer_scores_hip(q8, k8, w)
    ones_q = torch.ones(B, T, HI, device=dev)
    ones_k = torch.ones(B, T, device=dev)
    for qs, ks in ((ones_q, None), (None, ones_k), (ones_q, ones_k)):
        got = indexer_scores_hip(q8, k8, w, q_scale=qs, k_scale=ks)
        torch.cuda.synchronize()
        assert torch.equal(got, base)


def test_fp8_scales_need_fp8_inputs(dev):
    q = torch.zeros(1, 8, 4, 64, device=dev)
    k = torch.zeros(1, 8, 64, device=dev)
    with pytest.raises(AssertionError):
        indexer_scores_hip(q, k, torch.zeros(1, 8, 4, device=dev), k_scale=torch.ones(1, 8, device=dev))
