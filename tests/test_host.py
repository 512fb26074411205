"""CPU: host-side logic of the Python mirror that needs no GPU -- the
projection weight cache of lightning_indexer (reference
lightning_indexer.py:36-47,128-130 computes h @ W_Q, h @ W_K, h @ W_W on every
call; the MI355X front end concatenates the three weights once and must
never hand out a stale concatenation)."""
from __future__ import annotations

import gc

import torch

import lightning_indexer as LI


def _weights(seed, D=64, H=4, d=16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(D, H * d, generator=g), torch.randn(D, d, generator=g),
            torch.randn(D, H, generator=g))


def _cat(W_Q, W_K, W_W):
    return torch.cat([W_Q, W_K, W_W], dim=1)


def _check(wc, ws):
    n = sum(W.shape[1] for W in ws)
    assert torch.equal(wc[:, :n], _cat(*ws)), "cached concatenation is not cat(W_Q, W_K, W_W)"
    assert not bool(wc[:, n:].any()), "padding columns must be zero"
    assert (wc.shape[1] * wc.element_size()) % 16 == 0


def test_new_weights_at_a_freed_address_are_not_served_stale():
    """Free set A, build set B of the same shape and dtype: whenever B lands
    at A's address (the CPU allocator reuses freed blocks), the result must
    still be cat(B).  Every trial is checked; address reuse is what makes a
    data_ptr-keyed cache fail."""
    LI._WCAT_CACHE.clear()
    reused = 0
    for trial in range(60):
        A = _weights(2 * trial)
        ptrs = tuple(W.data_ptr() for W in A)
        _check(LI._fused_weights(*A, torch.float32), A)
        del A
        gc.collect()
        B = _weights(2 * trial + 1)
        reused += tuple(W.data_ptr() for W in B) == ptrs
        _check(LI._fused_weights(*B, torch.float32), B)
        del B
        gc.collect()
    # not asserted (allocator dependent), only reported on failure above
    print(f"address reused in {reused} of 60 trials")


def test_same_address_same_version_new_values():
    """The failure case made deterministic: tensors built with from_numpy over
    one host buffer start at _version 0 and share its address, so set B sits
    exactly where set A was, with A's shapes and version, but other values."""
    import numpy as np

    LI._WCAT_CACHE.clear()
    D, H, d = 48, 2, 16
    bufs = [np.empty((D, n), dtype=np.float32) for n in (H * d, d, H)]
    rng = np.random.default_rng(0)
    for trial in range(4):
        for b in bufs:
            b[...] = rng.standard_normal(b.shape)       # no torch version bump
        ws = tuple(torch.from_numpy(b) for b in bufs)
        assert all(W._version == 0 for W in ws)
        _check(LI._fused_weights(*ws, torch.float32), ws)
        del ws
        gc.collect()


def test_in_place_update_and_data_swap_invalidate():
    LI._WCAT_CACHE.clear()
    ws = list(_weights(7))
    _check(LI._fused_weights(*ws, torch.float32), ws)
    ws[1].mul_(2.0)                                  # in place: _version moves
    _check(LI._fused_weights(*ws, torch.float32), ws)
    ws[2].data = torch.randn_like(ws[2])             # same object, new storage
    _check(LI._fused_weights(*ws, torch.float32), ws)


def test_hits_per_layer_and_drops_dead_entries():
    LI._WCAT_CACHE.clear()
    layers = [_weights(100 + i) for i in range(5)]
    first = [LI._fused_weights(*ws, torch.float32) for ws in layers]
    again = [LI._fused_weights(*ws, torch.float32) for ws in layers]
    assert all(a is b for a, b in zip(first, again)), "one entry per layer must hit"
    assert len(LI._WCAT_CACHE) == 5
    del layers[2], first, again
    gc.collect()
    assert len(LI._WCAT_CACHE) == 4, "an entry whose weights died must be dropped"


def test_capacity_bound():
    cache = LI._ProjectionWeightCache(capacity=3)
    keep = [_weights(200 + i) for i in range(5)]
    for ws in keep:
        _check(cache.get(*ws, torch.float32), ws)
    assert len(cache) == 3
    # the most recent entries stay
    for ws in keep[2:]:
        _check(cache.get(*ws, torch.float32), ws)
    assert len(cache) == 3


def test_dtype_is_part_of_the_key():
    LI._WCAT_CACHE.clear()
    ws = _weights(9)
    a = LI._fused_weights(*ws, torch.float32)
    b = LI._fused_weights(*ws, torch.bfloat16)
    assert a.dtype == torch.float32 and b.dtype == torch.bfloat16
    n = sum(W.shape[1] for W in ws)
    assert torch.equal(b[:, :n], _cat(*ws).to(torch.bfloat16))
    assert (b.shape[1] * 2) % 16 == 0


def test_fuse_projection_weights_matches_cache():
    ws = _weights(11, D=32, H=3, d=8)    # n = 24 + 8 + 3 = 35 -> padded to 36 (fp32)
    wc = LI.fuse_projection_weights(*ws)
    assert wc.shape == (32, 36)
    _check(wc, ws)


def test_stream_pipeline_refuses_capture(monkeypatch):
    """DSAStreamPipeline is eager only: submit() and join() raise while the
    current stream is capturing, before anything is enqueued.  The capture
    state is faked from the host; no graph is captured."""
    import pytest

    import dsa_stream

    pipe = dsa_stream.DSAStreamPipeline.__new__(dsa_stream.DSAStreamPipeline)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="cannot be captured"):
        pipe.submit(None, None, None, None, None, None)
    with pytest.raises(RuntimeError, match="cannot be captured"):
        pipe.join()
    with pytest.raises(RuntimeError, match="cannot be captured"):
        pipe.synchronize()
