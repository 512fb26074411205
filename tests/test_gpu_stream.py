"""GPU: batch streaming (dsa_stream.py) -- every batch's output equals the
split forward's bit for bit (same kernels and inputs; only the launch order
across the two streams differs), for several pipeline depths, and one batch
against the float64 oracle."""
from __future__ import annotations

import pytest
import torch

from dsa_attention import dsa_split_hip
from dsa_stream import DSAStreamGraph, DSAStreamPipeline, dsa_attention_stream
from helpers import close, say
from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def make_batches(n, B, T, HI, DI, HQ, D, dtype, dev, seed0=0):
    out = []
    for i in range(n):
        ins = O.make_inputs(B, T, HI, DI, HQ, D, D, dtype=dtype, seed0=seed0 + 10 * i)
        out.append(tuple(x.to(dev) for x in ins))
    return out


@pytest.mark.parametrize("depth", [1, 2, 3])
def test_stream_matches_split_fp32(dev, depth):
    say(f"stream fp32 depth={depth}")
    batches = make_batches(5, 2, 512, 4, 32, 4, 32, torch.float32, dev)
    outs = dsa_attention_stream(batches, top_k=32, depth=depth)
    for bt, o in zip(batches, outs):
        assert torch.equal(o, dsa_split_hip(*bt, 32))


def test_stream_tile_path_bf16(dev):
    """T = 4096 with 16-bit Q/K/V and D = 64 takes the tile attention kernel."""
    say("stream bf16 T=4096")
    batches = make_batches(3, 1, 4096, 8, 64, 8, 64, torch.bfloat16, dev, seed0=7)
    pipe = DSAStreamPipeline(1, 4096, 256, device=dev)
    outs = [pipe.submit(*bt) for bt in batches]
    pipe.synchronize()
    for bt, o in zip(batches, outs):
        assert torch.equal(o, dsa_split_hip(*bt, 256))


def test_stream_one_batch_vs_oracle(dev):
    say("stream vs oracle")
    ins = O.make_inputs(2, 256, 4, 32, 4, 32, 32, seed0=3)
    out = dsa_attention_stream([tuple(x.to(dev) for x in ins)], top_k=16)[0].cpu()
    want = O.dsa_forward(*ins, 16)
    ok, err, _ = close(out, want, 1e-4, 1e-4)
    assert ok, f"max abs err {err}"


def test_stream_rejects_other_shapes(dev):
    pipe = DSAStreamPipeline(2, 256, 16, device=dev)
    ins = tuple(x.to(dev) for x in O.make_inputs(1, 256, 4, 32, 4, 32, 32))
    with pytest.raises(AssertionError):
        pipe.submit(*ins)


@pytest.mark.skip(reason="capturing the two-stream pipeline into one graph crashed the host "
                         "process inside the runtime's end of capture (segfault, cause not "
                         "established); that form is switched off -- DSAStreamGraph captures "
                         "on one stream")
def test_stream_two_stream_graph_capture(dev):
    """Two-stream pipeline captured into one graph (switched off)."""
    pytest.skip("switched off")


def test_stream_graph_replays_match_eager(dev):
    """The captured batches, replayed several times with new inputs and
    eager work in between, match the eager split forward every time."""
    say("stream graph replays (one-stream capture)")
    B, T, HI, DI, HQ, D, k, n = 4, 512, 4, 32, 4, 32, 64, 3
    sg = DSAStreamGraph(B, T, HI, DI, HQ, D, D, k, n, device=dev)
    for rep in range(3):
        batches = make_batches(n, B, T, HI, DI, HQ, D, torch.float32, dev, seed0=100 * rep)
        for dst, src in zip(sg.inputs, batches):
            for d_, s_ in zip(dst, src):
                d_.copy_(s_)
        sg.replay()
        torch.cuda.synchronize()
        for bt, o in zip(batches, sg.outputs):
            assert torch.equal(o, dsa_split_hip(*bt, k)), f"replay {rep}"
        torch.cuda.synchronize()


def test_stream_default_form_matches_split(dev):
    """dsa_attention_stream's default: batches one after another on the
    caller's stream with reused buffers."""
    say("stream default form")
    batches = make_batches(4, 2, 512, 4, 32, 4, 32, torch.float32, dev, seed0=50)
    outs = dsa_attention_stream(batches, top_k=32)
    assert len({o.data_ptr() for o in outs}) == len(outs), "each batch gets its own output"
    for bt, o in zip(batches, outs):
        assert torch.equal(o, dsa_split_hip(*bt, 32))
