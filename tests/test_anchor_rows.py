"""Anchor-row and global queries over one contiguous key range: the
``out[rows] = dense(q[rows], k, v)`` of a window adapter
(``integrations/vdn.py:57-61``) as one dense launch that gathers the query
rows and scatters the results inside the kernel (``sol_dense_fwd`` with
``query_index`` / ``out_index``).  ``sol_attention_indexed`` takes it at
beta = -inf when every window's keys are one and the same contiguous range.

Checked against the dense oracle on the gathered rows; against the one-block
SOL kernel's beta = -inf path on the same plan, which reads zero-padded block
tiles: bit-identical when the keys fill whole 64-key blocks, equal to
rounding otherwise (rows mode reads a partial last block as the range's last
64 rows, so its valid keys meet the matrix cores' sums in other groups); and
for the scatter: rows outside the plan untouched.
"""

import dataclasses
import math

import numpy as np
import pytest
import torch

from oracle import sol_oracle as orc
from sol_attn_amd import IndexedPlan, _native, sol_attention_indexed
from sol_testlib import HAS_GPU, assert_close

gpu = pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")


def field(n, h, d, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn((n, h, d), generator=g).to(torch.bfloat16).cuda() for _ in range(3))


def sorted_rows(n, count, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(n, generator=g)[:count].sort().values


# (sequence length, heads, head_dim, windows x query rows, key range [a, b))
CASES = [(3072, 3, 64, (1, 200), (0, 3072)),       # anchor rows over every key
         (2600, 2, 128, (3, 130), (0, 2600)),      # three windows, ragged query blocks, partial key block
         (4100, 2, 128, (2, 96), (700, 2750)),     # a key range inside the sequence
         (1000, 4, 64, (1, 64), (960, 1000))]      # fewer than 64 keys: block tiles


@pytest.mark.gpu
@gpu
@pytest.mark.parametrize("case", range(len(CASES)))
def test_anchor_rows_match_the_dense_oracle_and_the_sol_path(case, monkeypatch):
    n, h, d, (w, nq), (a, b) = CASES[case]
    print(f"anchor rows case {case}: N{n} H{h} D{d} W{w} nq{nq} keys [{a}, {b})", flush=True)
    q, k, v = field(n, h, d, seed=80 + case)
    rows = torch.stack([sorted_rows(n, nq, 90 + case + 7 * i) for i in range(w)])
    keys = torch.arange(a, b)[None].expand(w, -1).contiguous()
    plan = IndexedPlan.create(rows, keys, n, protected_ranges=((0, 64),)).to("cuda")
    assert plan.key_range == (a, b - a)
    got, stats = sol_attention_indexed(q, k, v, plan, beta=-math.inf, return_stats=True)
    assert got.shape == (w, nq, h, d)
    assert bool((stats.exact_blocks == -(-(b - a) // 64)).all())
    # The one-block SOL kernel's beta = -inf path over the same plan (pooled
    # block tiles; the small-launch kernel's key split sums in other orders).
    sol_plan = dataclasses.replace(plan, key_range=None)
    monkeypatch.setattr(_native, "WORKGROUP_FORM", 1)
    ref_sol = sol_attention_indexed(q, k, v, sol_plan, beta=-math.inf)
    monkeypatch.setattr(_native, "WORKGROUP_FORM", 0)
    if (b - a) % 64 == 0:
        assert torch.equal(got, ref_sol)
    else:
        assert_close(got.cpu(), ref_sol.cpu())
    cpu = [x.cpu() for x in (q, k, v)]
    for i in range(w):
        ref = orc.dense_oracle(cpu[0][rows[i]][None], cpu[1][a:b][None], cpu[2][a:b][None])
        assert_close(got[i].cpu()[None], ref)
    # Scatter: the plan's rows receive the same values, the others keep theirs.
    if w == 1 or torch.unique(rows).numel() == rows.numel():
        out = torch.full_like(q, 3.0)
        res = sol_attention_indexed(q, k, v, plan, beta=-math.inf, out=out)
        assert res is out
        flat = rows.reshape(-1).cuda()
        assert torch.equal(out[flat], got.reshape(-1, h, d))
        keep = torch.ones(n, dtype=torch.bool)
        keep[rows.reshape(-1)] = False
        assert bool((out[keep.cuda()] == 3.0).all())


def test_key_range_only_for_one_shared_contiguous_range():
    n = 2000
    rows = torch.stack([torch.arange(0, 128), torch.arange(128, 256)])
    same = torch.arange(300, 1300)[None].expand(2, -1).contiguous()
    assert IndexedPlan.create(rows, same, n).key_range == (300, 1000)
    assert IndexedPlan.create(rows, [torch.arange(0, 900)] * 2, n).key_range == (0, 900)
    # Different ranges per window, a gap inside a window, ragged lengths: none.
    assert IndexedPlan.create(rows, torch.stack([torch.arange(0, 1000), torch.arange(500, 1500)]), n).key_range is None
    gap = torch.cat([torch.arange(0, 500), torch.arange(600, 1100)])
    assert IndexedPlan.create(rows, torch.stack([gap, gap]), n).key_range is None
    assert IndexedPlan.create(rows, [torch.arange(0, 900), torch.arange(0, 1000)], n).key_range is None
    assert IndexedPlan.create(rows, same, n).to("cpu").key_range == (300, 1000)


@pytest.mark.gpu
@gpu
def test_device_built_plan_takes_the_dense_route():
    n, h, d = 2000, 2, 64
    rows = torch.stack([torch.arange(0, 128), torch.arange(128, 256)])
    dev = IndexedPlan.create(rows.cuda(), torch.arange(0, 1000)[None].expand(2, -1).contiguous().cuda(), n)
    assert dev.key_range == (0, 1000)
    q, k, v = field(n, h, d, seed=7)
    got = sol_attention_indexed(q, k, v, dev, beta=-math.inf)
    ref = orc.dense_oracle(q.cpu()[rows[1]][None], k.cpu()[:1000][None], v.cpu()[:1000][None])
    assert_close(got[1].cpu()[None], ref)
    np.testing.assert_array_equal(rows.numpy(), dev.rows.cpu().numpy())
