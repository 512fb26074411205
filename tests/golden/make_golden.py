"""Writes the golden fixtures in tests/golden/ (run in the build container).

    python tests/golden/make_golden.py

c0_forward.npz -- config 0 (B=1, T=128, k=8, HI=4, DI=32, HQ=4, DQ=DV=32):
    inputs from oracle.make_inputs (CPU generator, seeds 0..5) and the float64
    oracle's scores, thr (k=8), exactly-k idx and output.  Before writing, the
    vectorised oracle is checked against dsa_forward_naive (plain loops).
    Also `thr_ref`: the reference's own compiled topk_threshold
    (oracle/_ref) run on the fp32 copy of those scores.
ref_topk.npz -- the reference's own compiled extension (oracle/_ref, built
    from /root/reference/topk_avx512.cpp) on the inputs of its own tests
    (test_topk_avx512.py:20-35): torch.manual_seed(0); randn(3,128,128) with
    k in (1,8,16,32,64,96,128) via topk_threshold, and seed 1 with k in
    (64,128) via topk_threshold_batch_merge.  Inputs are stored too.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import dsa_oracle as O  # noqa: E402
from oracle import native  # noqa: E402

C0 = dict(B=1, T=128, HI=4, DI=32, HQ=4, DQ=32, DV=32)
C0_K = 8
REF_KS = (1, 8, 16, 32, 64, 96, 128)
REF_BM_KS = (64, 128)


def make_c0():
    ins = O.make_inputs(**C0)
    out, scores, thr = O.dsa_forward(*ins, C0_K, acc=torch.float64, return_parts=True)
    naive = O.dsa_forward_naive(*ins, C0_K)
    err = float(np.max(np.abs(out.numpy() - naive)))
    assert err < 1e-10, f"oracle vs naive loops: {err}"
    idx = O.select_indices(scores.numpy(), C0_K)
    s32 = scores.to(torch.float32).contiguous()
    ref = native.ref()
    if ref is None:
        raise SystemExit("oracle/_ref not built: run python oracle/build.py first")
    thr_ref = ref.topk_threshold(s32, C0_K).numpy()
    names = ("q_idx", "k_idx", "w_idx", "Q", "K", "V")
    np.savez_compressed(
        os.path.join(HERE, "c0_forward.npz"),
        **{n: x.numpy() for n, x in zip(names, ins)},
        top_k=np.int64(C0_K), scores=scores.numpy(), thr=thr.numpy(), idx=idx,
        out=out.numpy(), scores_f32=s32.numpy(), thr_ref=thr_ref)


def make_ref_topk():
    ref = native.ref()
    if ref is None:
        raise SystemExit("oracle/_ref not built: run python oracle/build.py first")
    torch.manual_seed(0)
    x0 = torch.randn(3, 128, 128, dtype=torch.float32)
    torch.manual_seed(1)
    x1 = torch.randn(3, 128, 128, dtype=torch.float32)
    thr0 = np.stack([ref.topk_threshold(x0.contiguous(), k).numpy() for k in REF_KS])
    thr1 = np.stack([ref.topk_threshold_batch_merge(x1.contiguous(), k).numpy()
                     for k in REF_BM_KS])
    np.savez_compressed(os.path.join(HERE, "ref_topk.npz"), x0=x0.numpy(), x1=x1.numpy(),
                        ks0=np.array(REF_KS), ks1=np.array(REF_BM_KS), thr0=thr0, thr1=thr1)


if __name__ == "__main__":
    make_c0()
    make_ref_topk()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
