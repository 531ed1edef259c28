"""Cost-ordered dispatch of routed two-block launches (order_kernel): a
schedule choice that never changes results.

No counterpart in the reference (one Triton program per query block).  When
the routing masks come from the routing kernel, order_kernel ranks each
head's regular query tiles (after the query-sink tiles) by the size of their
key-block union and deals them to the XCD slices of the workgroup map in
snake order, costly tiles first.  The checks, on the order array the launch
leaves in its route workspace: it is a permutation of each head's tiles;
inside every XCD's slice the costs do not rise; the j-th tile of a slice lies
between the costs of ranks 8j and 8j + 7 (each round of eight ranks goes to
eight different XCDs); the leftover slots hold the cheapest tiles.  Outputs
and counts are bit-identical to the one-block workgroup form (no order) under
the same routing masks, with and without query-block pairing and for keys
past one routing segment (8,192 key blocks), and match the oracle under the
kernel's routing.
"""

import numpy as np
import pytest
import torch

from sol_attn_amd import _native, sol_attention
from sol_testlib import HAS_GPU, assert_close, block_smooth, to_np

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]

XCDS = 8


def _aligned(n):
    return -(-n // 256) * 256


def _run(q, k, v, form, monkeypatch, beta=1.0, kv_sink=64, q_sink=128, keep=None):
    monkeypatch.setattr(_native, "WORKGROUP_FORM", form)
    monkeypatch.setattr(_native, "ROUTE_PREPASS", "always")
    monkeypatch.setattr(_native, "SPLIT_SINKS", False)   # the order applies to unsplit launches
    if keep is not None:
        make = _native.route_workspace

        def kept(*a):
            ws = make(*a)
            keep.append(ws)
            return ws
        monkeypatch.setattr(_native, "route_workspace", kept)
    try:
        out, stats = sol_attention(q, k, v, beta=beta, kv_sink_tokens=kv_sink, query_sink_tokens=q_sink,
                                   return_stats=True)
        torch.cuda.synchronize()
    finally:
        if keep is not None:
            monkeypatch.setattr(_native, "route_workspace", make)
    return out, stats.exact_blocks


def _check_order(ws, b, tq, tk, h, q_sink):
    """Order properties per (entry, head) from the route workspace's masks."""
    nqb, nkb = -(-tq // 64), -(-tk // 64)
    nw = -(-nkb // 32)
    words = ws.cpu().numpy().view(np.uint32)
    mask = words[:b * h * nqb * nw].reshape(b * h, nqb, nw)
    order = words[_aligned(b * h * nqb * nw * 4) // 4:].view(np.int32).reshape(b * h, nqb)
    ntiles = (nqb + 1) // 2
    front = min(-(-q_sink // 64) if q_sink else 0, ntiles)
    r_tiles = ntiles - front
    base, rem = divmod(r_tiles, XCDS)
    for bh in range(b * h):
        t = front + np.arange(r_tiles)
        a, c2 = 2 * t, np.minimum(2 * t + 1, nqb - 1)
        union = mask[bh, a] | np.where((2 * t + 1 < nqb)[:, None], mask[bh, c2], 0)
        cost = np.bitwise_count(union).sum(-1).astype(np.int64)
        o = order[bh, :r_tiles]
        assert sorted(o.tolist()) == list(range(r_tiles)), f"head {bh}: not a permutation"
        ranked = np.sort(cost)[::-1]
        c = (front * b * h + bh * rem) % XCDS          # first XCD holding a leftover slot
        extra = [((x - c) % XCDS) < rem for x in range(XCDS)]
        start = 0
        for x in range(XCDS):
            n = base + int(extra[x])
            sl = cost[o[start:start + n]]
            assert (np.diff(sl) <= 0).all(), f"head {bh} XCD {x}: costs rise inside the slice"
            for j in range(min(n, base)):
                assert ranked[XCDS * j + XCDS - 1] <= sl[j] <= ranked[XCDS * j], (bh, x, j)
            if n > base and base:
                assert sl[base] <= ranked[XCDS * base - 1], (bh, x)   # a leftover: among the cheapest
            start += n
        assert start == r_tiles
    return cost


@pytest.mark.parametrize("shape", [(2, 6000, 5000, 3, 128, 128), (1, 20000, 9000, 2, 64, 0)])
def test_order_is_a_balanced_permutation_and_outputs_are_unchanged(shape, monkeypatch):
    b, tq, tk, h, d, q_sink = shape
    print(f"tile order: B{b} Tq{tq} Tk{tk} H{h} D{d} q_sink {q_sink}", flush=True)
    q, k, v = (block_smooth(b, t, h, d, seed=s, device="cuda") for t, s in ((tq, 21), (tk, 22), (tk, 23)))
    monkeypatch.setattr(_native, "PAIRING", False)   # adjacent pairs: tile t holds blocks 2t, 2t + 1
    keep = []
    two, counts2 = _run(q, k, v, 2, monkeypatch, q_sink=q_sink, keep=keep)
    assert len(keep) == 1
    cost = _check_order(keep[0], b, tq, tk, h, q_sink)
    assert cost.max() > cost.min()                      # the costs differ, so the order matters
    one, counts1 = _run(q, k, v, 1, monkeypatch, q_sink=q_sink)
    assert torch.equal(one, two)
    assert torch.equal(counts1, counts2)


def test_ordered_paired_launch_matches_one_block_form_and_oracle(monkeypatch):
    from test_kernels import check_routing
    q, k, v = (block_smooth(1, 9000, 2, 128, seed=s, device="cuda") for s in (31, 32, 33))
    monkeypatch.setattr(_native, "PAIR_MIN_QUERY_BLOCKS", 1)   # pairing strides and query means
    two, counts2 = _run(q, k, v, 2, monkeypatch)
    one, counts1 = _run(q, k, v, 1, monkeypatch)
    assert torch.equal(one, two)
    assert torch.equal(counts1, counts2)
    monkeypatch.setattr(_native, "WORKGROUP_FORM", 2)
    actual, ref, _ = check_routing(q, k, v, 1.0, kv_sink=64, q_sink=128, local=1, label="ordered tiles")
    assert_close(actual, ref)
    assert (actual == to_np(two)).all()     # the debug launch (same masks, same order) gives the same output


def test_ordered_tiles_across_routing_segments(monkeypatch):
    """Keys past one routing segment (8,192 key blocks): the order kernel
    counts every segment's mask words; outputs equal the one-block form's."""
    tq, tk, h, d = 2200, 8192 * 64 + 300 * 64 + 17, 1, 128   # 35 query blocks: 17 regular tiles
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, t, h, d, generator=gen).to(torch.bfloat16).cuda() for t in (tq, tk, tk))
    print(f"tile order across segments: Tq {tq} Tk {tk}", flush=True)
    monkeypatch.setattr(_native, "PAIRING", False)
    keep = []
    two, counts2 = _run(q, k, v, 2, monkeypatch, beta=0.0, q_sink=64, keep=keep)
    assert len(keep) == 1
    cost = _check_order(keep[0], 1, tq, tk, h, 64)
    assert cost.max() > cost.min()
    one, counts1 = _run(q, k, v, 1, monkeypatch, beta=0.0, q_sink=64)
    assert torch.equal(one, two)
    assert torch.equal(counts1, counts2)


def test_order_at_the_largest_ordered_launch(monkeypatch):
    """4,096 regular tiles per head (8,192 query blocks), the most the order
    kernel takes: still a balanced permutation, outputs equal to the
    one-block form's."""
    t, h, d = 8192 * 64, 1, 64
    q, k, v = (block_smooth(1, t, h, d, seed=s, device="cuda") for s in (41, 42, 43))
    print(f"tile order: {t} tokens, 4,096 tiles per head", flush=True)
    monkeypatch.setattr(_native, "PAIRING", False)
    keep = []
    two, counts2 = _run(q, k, v, 2, monkeypatch, q_sink=0, keep=keep)
    assert len(keep) == 1
    cost = _check_order(keep[0], 1, t, t, h, 0)
    assert cost.max() > cost.min()
    one, counts1 = _run(q, k, v, 1, monkeypatch, q_sink=0)
    assert torch.equal(one, two)
    assert torch.equal(counts1, counts2)
