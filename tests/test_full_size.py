"""Parity at the headline size: 84,672 tokens (a 21 x 48 x 84 smooth field),
24 heads, D = 128, beta 1, kv and query sinks of 128 tokens, local band 1.

The oracle runs on a sample of query blocks (the first, a query sink that
selects every key block; one from the middle; the last) x all 24 heads:
routing decisions within the stated band, proxies, cutoffs, counts, and the
outputs under identical routing.  Whole-size properties: the exact-block
counts equal the decision masks' popcounts (checked on the sample above), a
repeated call is bit-identical, and beta = -inf equals the dense kernel
within the BF16 tolerance.  The same field as 21 frame windows (window f:
queries frame f, keys frames {0, f-1, f, f+1}, frame 0 protected): one
ragged call with the fused scatter against the oracle on window 10, and
bit-identical to a separate call over the windows of 16,128 keys.
"""

import math

import numpy as np
import pytest
import torch

import bench
from oracle.sol_oracle import sol_oracle
from sol_attn_amd import IndexedPlan, dense_attention, sol_attention, sol_attention_indexed
from sol_testlib import HAS_GPU, assert_close
from oracle import sol_oracle as orc
from test_kernels import check_routing, run_debug

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]

CFG = bench.WORKLOADS["videodit-84672"]


@pytest.fixture(scope="module")
def field():
    with torch.no_grad():
        return bench.make_inputs(CFG, torch.device("cuda"))


def test_full_size_sampled_parity(field):
    q, k, v = field
    nqb = -(-q.shape[1] // 64)
    sample = [0, nqb // 2, nqb - 1]
    got, ref, _ = check_routing(q, k, v, CFG["beta"], local=CFG["local_blocks"],
                                kv_sink=CFG["kv_sink_tokens"], q_sink=CFG["query_sink_tokens"],
                                query_blocks=sample)
    assert_close(got, ref)


def test_full_size_routing_every_decision(field):
    # All 1,323 x 1,323 x 24 = 42.0M (query block, key block, head) decisions
    # against the oracle's (float64 Qc . Kc_j): none outside the routing band.
    q, k, v = field
    _, _, dbg = run_debug(q, k, v, CFG["beta"], local=CFG["local_blocks"], kv_sink=CFG["kv_sink_tokens"],
                          q_sink=CFG["query_sink_tokens"])
    sel = dbg["selected"].cpu()
    del dbg
    res = orc.routing_check(q.cpu(), k.cpu(), sel, beta=CFG["beta"], local_blocks=CFG["local_blocks"],
                            kv_sink_tokens=CFG["kv_sink_tokens"], query_sink_tokens=CFG["query_sink_tokens"])
    print(f"routing every decision (84,672 tokens): {res}", flush=True)
    assert res["decisions"] == 1323 * 1323 * 24
    assert res["outside_band"] == 0


def test_full_size_properties(field):
    q, k, v = field
    kw = dict(beta=CFG["beta"], kv_sink_tokens=CFG["kv_sink_tokens"],
              query_sink_tokens=CFG["query_sink_tokens"], local_blocks=CFG["local_blocks"])
    a, sa = sol_attention(q, k, v, return_stats=True, **kw)
    b, sb = sol_attention(q, k, v, return_stats=True, **kw)
    assert torch.equal(a, b) and torch.equal(sa.exact_blocks, sb.exact_blocks)
    assert 0.05 < sa.density() < 0.5
    del a, b
    every = sol_attention(q, k, v, beta=-math.inf)
    assert_close(every.cpu(), dense_attention(q, k, v).cpu())


def test_full_size_frame_windows(field):
    q, k, v = (x[0] for x in field)                       # NHD [84672, 24, 128]
    tpf = CFG["height"] * CFG["width"]
    rows, keys = bench.window_plans(CFG["frames"], tpf)
    prot = dict(protected_ranges=((0, tpf),), local_tokens=64)
    plan = IndexedPlan.create(rows, keys, q.shape[0], **prot).to("cuda")
    full = torch.empty_like(q)
    _, stats = sol_attention_indexed(q, k, v, plan, beta=1.0, return_stats=True, out=full)
    # Windows 2 .. 18 have 16,128 keys each: their own equal-length plan.
    mid = list(range(2, CFG["frames"] - 2))
    sub = IndexedPlan.create(rows[mid], torch.stack([keys[w] for w in mid]), q.shape[0], **prot).to("cuda")
    part, sub_stats = sol_attention_indexed(q, k, v, sub, beta=1.0, return_stats=True)
    assert torch.equal(part, full[rows[mid].cuda()])
    assert torch.equal(sub_stats.exact_blocks, stats.exact_blocks[mid])
    w, sample = 10, [0, 31, 62]
    nkb = -(-len(keys[w]) // 64)
    cpu = [x.cpu() for x in (q, k, v)]
    ref, counts, _ = sol_oracle(cpu[0][rows[w]][None], cpu[1][keys[w]][None], cpu[2][keys[w]][None], beta=1.0,
                                local_blocks=-1, protected_blocks=plan.protected_blocks[w:w + 1, :, :nkb].cpu(),
                                query_blocks=sample)
    qrows = np.concatenate([np.arange(64 * b, 64 * b + 64) for b in sample])
    assert_close(full[rows[w][qrows].cuda()].cpu()[None], ref[:, qrows])
    np.testing.assert_array_equal(stats.exact_blocks[w:w + 1, sample].cpu().numpy(), counts[:, sample])


def test_full_size_anchor_rows_over_every_key(field):
    # Frame 0's queries attend all 84,672 keys (a window adapter's anchor rows,
    # integrations/vdn.py:57-61): one dense launch gathering the rows and
    # scattering the results; the oracle on three of its 63 query blocks.
    q, k, v = (x[0] for x in field)
    n = q.shape[0]
    tpf = CFG["height"] * CFG["width"]
    rows = torch.arange(tpf)[None]
    plan = IndexedPlan.create(rows, torch.arange(n)[None], n).to("cuda")
    assert plan.key_range == (0, n)
    out = torch.zeros_like(q)
    sol_attention_indexed(q, k, v, plan, beta=-math.inf, out=out)
    assert bool((out[tpf:] == 0).all())
    sample = [0, 31, 62]
    qrows = np.concatenate([np.arange(64 * b, 64 * b + 64) for b in sample])
    print(f"anchor rows: {tpf} queries x {n} keys, oracle on blocks {sample}", flush=True)
    ref = orc.dense_oracle(q.cpu()[qrows][None], k.cpu()[None], v.cpu()[None])
    assert_close(out[torch.as_tensor(qrows).cuda()].cpu()[None], ref)
