"""Launches go to the caller's current stream (attention.py:54,80 run under
the current stream of the device).

On a side stream the call gives the default stream's results.  Under HIP
graph capture every launch must be on the capturing stream (a launch on
another stream makes the capture fail), and the captured graph replays to
the eager result, checked on every replay with eager work and
synchronisation in between.
"""

import pytest
import torch

from sol_attn_amd import dense_attention, sol_attention
from sol_testlib import HAS_GPU, block_smooth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


def inputs():
    return [block_smooth(1, 2048, 4, 128, seed, device="cuda") for seed in (51, 52, 53)]


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


def test_graph_capture_replays_the_eager_result():
    q, k, v = inputs()
    eager = sol_attention(q, k, v, kv_sink_tokens=64)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the default stream, as torch's capture expects
        for _ in range(2):
            sol_attention(q, k, v, kv_sink_tokens=64)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = sol_attention(q, k, v, kv_sink_tokens=64)
    for r in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        again = sol_attention(q, k, v, kv_sink_tokens=64)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
