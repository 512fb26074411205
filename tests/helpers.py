"""Helpers shared by the GPU parity tests."""
from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import dsa_oracle as O

# (B, T, k, HI, DI, HQ, DQ, DV, dtype, w_scale) of BASELINE.json configs[0..4]
CONFIGS = {
    "c0": (1, 128, 8, 4, 32, 4, 32, 32, torch.float32),
    "c1": (16, 512, 32, 4, 32, 4, 32, 32, torch.float32),
    "c2_b4_k64": (4, 512, 64, 4, 32, 4, 32, 32, torch.float32),
    "c2_b16_k64": (16, 512, 64, 4, 32, 4, 32, 32, torch.float32),
    "c2_b16_k128": (16, 512, 128, 4, 32, 4, 32, 32, torch.float32),
    "c2_b32_k64": (32, 512, 64, 4, 32, 4, 32, 32, torch.float32),
    "c2_b64_k64": (64, 512, 64, 4, 32, 4, 32, 32, torch.float32),
    # config-1 widths around the fused kernel's tile pairing (tests only)
    "c1_t500": (16, 500, 32, 4, 32, 4, 32, 32, torch.float32),
    "c1_t496": (16, 496, 32, 4, 32, 4, 32, 32, torch.float32),
    # the fused kernel's largest T (16-query blocks: the most LDS it takes)
    "fused_t2048": (2, 2048, 64, 4, 32, 4, 32, 32, torch.float32),
    # wide attention rows (more than one wave's registers hold): head-chunked
    # gathers (fp32) and the tile kernel (16-bit) at T < 4096 (tests only)
    "wide_f32_t512": (2, 512, 32, 4, 32, 16, 128, 128, torch.float32),
    "wide_f32_t2048": (1, 2048, 64, 4, 32, 16, 128, 128, torch.float32),
    "wide_bf16_t512": (1, 512, 32, 4, 32, 128, 128, 128, torch.bfloat16),
    "wide_bf16_t2048": (1, 2048, 64, 4, 32, 128, 128, 128, torch.bfloat16),
    "c3": (4, 4096, 256, 8, 64, 8, 64, 64, torch.float32),
    "c4": (1, 16384, 2048, 64, 128, 16, 128, 128, torch.bfloat16),
}


def say(*a):
    """Progress line, flushed (names the case before each GPU step)."""
    print(*a, flush=True)
    sys.stdout.flush()


def inputs(name, seed0=0, **kw):
    B, T, k, HI, DI, HQ, DQ, DV, dt = CONFIGS[name]
    return O.make_inputs(B, T, HI, DI, HQ, DQ, DV, dtype=dt, seed0=seed0, **kw), k


def to_dev(xs, dev):
    return tuple(x.to(dev) for x in xs)


def close(a, b, rtol, atol):
    """(ok, max_abs_err, worst relative excess) for float tensors/arrays."""
    a = torch.as_tensor(a).double()
    b = torch.as_tensor(b).double()
    err = (a - b).abs()
    lim = atol + rtol * b.abs()
    return bool((err <= lim).all()), float(err.max()), float((err / lim).max())


def flipped_rows(scores_a, scores_b, k, rows=None):
    """Rows whose selected set (>= k-th largest, ties kept) differs between
    two score matrices [B,R,T] (CPU tensors; R = T or len(rows))."""
    ta = O.topk_threshold(scores_a, k)
    tb = O.topk_threshold(scores_b, k)
    T = scores_a.shape[-1]
    ts = torch.arange(T) if rows is None else torch.as_tensor(rows)
    causal = torch.arange(T)[None, :] <= ts[:, None]
    sa = (scores_a >= ta) & causal
    sb = (scores_b >= tb) & causal
    return (sa != sb).any(-1)          # [B,T] bool


def sample_rows(T, n, seed=0, include=()):
    rng = np.random.default_rng(seed)
    picks = set(int(x) for x in include)
    picks |= set(int(x) for x in rng.choice(T, size=min(n, T), replace=False))
    return sorted(picks)
