"""Launches go to the caller's current stream (attention.py:54,80 run under
the current stream of the device).

On a side stream the call gives the default stream's results.  Under HIP
graph capture every launch must be on the capturing stream or on a stream
that joined the capture through an event (the pairing kernels' own stream
forks from the caller's stream and joins it again; a launch on any other
stream makes the capture fail), and the captured graph replays to the eager
result, checked on every replay with eager work and synchronisation in
between.
"""

import pytest
import torch

from sol_attn_amd import IndexedPlan, _native, dense_attention, sol_attention, sol_attention_indexed
from sol_testlib import HAS_GPU, block_smooth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


def inputs(tokens=2048, heads=4, dim=128):
    return [block_smooth(1, tokens, heads, dim, seed, device="cuda") for seed in (51, 52, 53)]


def test_side_stream_matches_default_stream():
    q, k, v = inputs()
    ref, ref_stats = sol_attention(q, k, v, kv_sink_tokens=64, return_stats=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out, stats = sol_attention(q, k, v, kv_sink_tokens=64, return_stats=True)
        dense = dense_attention(q, k, v)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(stats.exact_blocks, ref_stats.exact_blocks)
    assert torch.equal(dense, dense_attention(q, k, v))


def _capture_cases():
    """(name, setup(monkeypatch) -> call) for the launch shapes: the
    small-launch kernel (key-split groups) after the pooling kernel, and as one
    launch that pools its keys itself; the one-block form; the two-block form
    with the pairing kernels (dynamic-LDS lag kernel included); query sinks
    split by key range with the merge kernel; indexed windows with the fused
    scatter into out=."""

    def small(mp):
        q, k, v = inputs()
        return lambda: sol_attention(q, k, v, kv_sink_tokens=64)

    def one_launch(mp):
        q, k, v = inputs(1024, 8, 64)
        assert _native.library().sol_attention_pools_keys(1, 1024, 1024, 8, 64) == 1
        return lambda: sol_attention(q, k, v, kv_sink_tokens=128, query_sink_tokens=128)

    def plain(mp):
        mp.setattr(_native, "WORKGROUP_FORM", 1)
        q, k, v = inputs()
        return lambda: sol_attention(q, k, v, kv_sink_tokens=64)

    def paired(mp):
        mp.setattr(_native, "WORKGROUP_FORM", 2)
        mp.setattr(_native, "PAIR_MIN_QUERY_BLOCKS", 4)
        q, k, v = inputs()
        return lambda: sol_attention(q, k, v, kv_sink_tokens=64)

    def split(mp):
        q, k, v = inputs(4096)
        assert _native.library().sol_split_workspace_size(1, 4096, 4096, 4, 128, 1.0, 128) > 0
        return lambda: sol_attention(q, k, v, kv_sink_tokens=64, query_sink_tokens=128)

    def indexed(mp):
        q, k, v = (x[0] for x in inputs())             # NHD [2048, 4, 128]
        rows = torch.stack((torch.arange(0, 700), torch.arange(1000, 1700)))
        keys = [torch.arange(0, 1200), torch.arange(600, 2048)]
        plan = IndexedPlan.create(rows, keys, 2048, protected_ranges=((0, 64),)).to("cuda")
        out = torch.zeros_like(q)
        return lambda: sol_attention_indexed(q, k, v, plan, beta=1.0, out=out)

    return {"small-launch": small, "one-launch": one_launch, "one-block": plain, "paired": paired,
            "split-sinks": split, "indexed-scatter": indexed}


@pytest.mark.parametrize("case", sorted(_capture_cases()))
def test_graph_capture_replays_the_eager_result(case, monkeypatch):
    call = _capture_cases()[case](monkeypatch)
    eager = call().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the default stream, as torch's capture expects
        for _ in range(2):
            call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    for r in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"{case} replay {r}"
        again = call()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
