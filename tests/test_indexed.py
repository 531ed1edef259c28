"""GPU parity of the indexed-window path, mirroring the reference's tests/test_indexed.py."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.sol_oracle import sol_oracle
from sol_attn_amd import _native, IndexedPlan, sol_attention_indexed
from sol_testlib import HAS_GPU

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


@pytest.mark.parametrize("beta", [-math.inf, math.inf, 1.0])
def test_indexed_mask_pooling_oracle_and_unchanged_inputs(beta):
    # test_indexed.py:59-88
    g = torch.Generator().manual_seed(719)
    cpu = [torch.randn((1200, 4, 128), generator=g, dtype=torch.bfloat16)[:, ::2] for _ in range(3)]
    rows = torch.stack((torch.arange(231, 361), torch.arange(901, 1031)))
    keys = torch.stack((torch.cat((torch.arange(7), torch.arange(191, 703), torch.arange(1180, 1193))),
                        torch.cat((torch.arange(7), torch.arange(661, 1173), torch.arange(1180, 1193)))))
    p = IndexedPlan.create(rows, keys, 1200, protected_ranges=((0, 7), (1180, 1193)), local_tokens=64)
    gpu = [torch.empty((1200, 4, 128), device="cuda", dtype=torch.bfloat16)[:, ::2].copy_(x) for x in cpu]
    before = [x.clone() for x in gpu]
    actual, stats = sol_attention_indexed(*gpu, p.to("cuda"), beta=beta, return_stats=True)
    assert actual.shape == (2, 130, 2, 128) and actual.is_contiguous()
    ref, counts, _ = sol_oracle(cpu[0][rows], cpu[1][keys], cpu[2][keys], beta=beta,
                                local_blocks=-1, protected_blocks=p.protected_blocks)
    torch.testing.assert_close(actual.cpu().float(), torch.from_numpy(ref), atol=0.012, rtol=0.025)
    assert (actual.cpu().float() - torch.from_numpy(ref)).norm() / np.linalg.norm(ref) < 0.008
    np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)
    if beta == -math.inf:
        dense = F.scaled_dot_product_attention(cpu[0][rows].float().transpose(1, 2),
            cpu[1][keys].float().transpose(1, 2), cpu[2][keys].float().transpose(1, 2)).transpose(1, 2)
        torch.testing.assert_close(actual.cpu().float(), dense, atol=0.012, rtol=0.025)
    # Keys outside the declared set must not affect exact OR approximate output.
    seen = torch.unique(keys)
    excluded = torch.ones(1200, dtype=torch.bool, device="cuda")
    excluded[seen.to("cuda")] = False
    gpu[1][excluded] = 80
    gpu[2][excluded] = 80
    assert torch.equal(actual, sol_attention_indexed(*gpu, p.to("cuda"), beta=beta))
    assert torch.equal(gpu[0], before[0])
    assert torch.equal(gpu[1][seen], before[1][seen])
    assert torch.equal(gpu[2][seen], before[2][seen])


def test_indexed_equals_bthd_on_gathered_rows():
    # With no protection and the local band off, indexed windows are the BTHD
    # operator on gathered copies.
    g = torch.Generator().manual_seed(5)
    x = [torch.randn((700, 3, 64), generator=g, dtype=torch.bfloat16).cuda() for _ in range(3)]
    rows = torch.stack((torch.arange(0, 150), torch.arange(300, 450)))
    keys = torch.stack((torch.arange(100, 400), torch.arange(350, 650)))
    p = IndexedPlan.create(rows, keys, 700, local_tokens=0).to("cuda")
    out, stats = sol_attention_indexed(*x, p, beta=0.5, return_stats=True)
    ref, counts, _ = sol_oracle(x[0].cpu()[rows], x[1].cpu()[keys], x[2].cpu()[keys], beta=0.5,
                                local_blocks=-1, protected_blocks=p.protected_blocks.cpu())
    np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)
    torch.testing.assert_close(out.cpu().float(), torch.from_numpy(ref), atol=0.012, rtol=0.025)


def _ragged_case(seed, n=1500, heads=2, d=128):
    g = torch.Generator().manual_seed(seed)
    x = [torch.randn((n, heads, d), generator=g, dtype=torch.bfloat16) for _ in range(3)]
    rows = torch.stack((torch.arange(64, 194), torch.arange(500, 630), torch.arange(1300, 1430)))
    keys = [torch.cat((torch.arange(0, 7), torch.arange(40, 300))),     # 267 keys, 5 blocks
            torch.cat((torch.arange(0, 7), torch.arange(380, 1000))),   # 627 keys, 10 blocks
            torch.arange(1250, 1330)]                                  # 80 keys, 2 blocks
    return x, rows, keys


@pytest.mark.parametrize("group", ["1", "2"])  # one- and two-block workgroups
@pytest.mark.parametrize("beta", [-math.inf, math.inf, 1.0, 0.0])
def test_ragged_windows_one_call_equal_separate_calls_and_oracle(beta, group, monkeypatch):
    monkeypatch.setattr(_native, "WORKGROUP_FORM", int(group))
    x, rows, keys = _ragged_case(11)
    kw = dict(protected_ranges=((0, 7),), local_tokens=64)
    p = IndexedPlan.create(rows, keys, 1500, **kw)
    gpu = [t.cuda() for t in x]
    out, stats = sol_attention_indexed(*gpu, p.to("cuda"), beta=beta, return_stats=True)
    assert out.shape == (3, 130, 2, 128)
    densities = []
    for w in range(3):
        pw = IndexedPlan.create(rows[w:w + 1], keys[w][None], 1500, **kw)
        ow, sw = sol_attention_indexed(*gpu, pw.to("cuda"), beta=beta, return_stats=True)
        assert torch.equal(out[w:w + 1], ow), f"window {w} differs from its own call"
        assert torch.equal(stats.exact_blocks[w:w + 1], sw.exact_blocks)
        ref, counts, _ = sol_oracle(x[0][rows[w:w + 1]], x[1][keys[w][None]], x[2][keys[w][None]],
                                    beta=beta, local_blocks=-1, protected_blocks=pw.protected_blocks)
        got = out[w:w + 1].cpu().float()
        torch.testing.assert_close(got, torch.from_numpy(ref), atol=0.012, rtol=0.025)
        assert (got - torch.from_numpy(ref)).norm() / np.linalg.norm(ref) < 0.008
        np.testing.assert_array_equal(stats.exact_blocks[w:w + 1].cpu().numpy(), counts)
        densities.append(counts.mean() / -(-len(keys[w]) // 64))
    assert stats.density() == pytest.approx(float(np.mean(densities)), rel=1e-6)


@pytest.mark.parametrize("group", ["1", "2"])
def test_scatter_epilogue_equals_indexed_assignment(group, monkeypatch):
    monkeypatch.setattr(_native, "WORKGROUP_FORM", int(group))
    x, rows, keys = _ragged_case(12)
    gpu = [t.cuda() for t in x]
    for plan in (IndexedPlan.create(rows, keys, 1500),
                 IndexedPlan.create(rows, torch.stack([k[:80] for k in keys]), 1500)):
        p = plan.to("cuda")
        ref = sol_attention_indexed(*gpu, p, beta=1.0)
        out = torch.full_like(gpu[0], 3.0)
        got = sol_attention_indexed(*gpu, p, beta=1.0, out=out)
        assert got is out
        expected = torch.full_like(gpu[0], 3.0)
        expected[p.rows] = ref
        assert torch.equal(out, expected)
    with pytest.raises(ValueError, match="out must be"):
        sol_attention_indexed(*gpu, p, out=torch.empty_like(gpu[0]).float())


def test_scatter_rejects_shared_rows_and_tampered_plans_stay_in_bounds():
    x, rows, keys = _ragged_case(13)
    gpu = [t.cuda() for t in x]
    # Two windows with one query row in common: out= would race on it.
    shared = torch.stack((torch.arange(64, 194), torch.arange(193, 323)))
    p = IndexedPlan.create(shared, torch.stack([k[:80] for k in keys[:2]]), 1500).to("cuda")
    assert p.rows_distinct is False
    with pytest.raises(ValueError, match="share no query row"):
        sol_attention_indexed(*gpu, p, beta=1.0, out=torch.empty_like(gpu[0]))
    sol_attention_indexed(*gpu, p, beta=1.0)  # without out= the plan is fine
    # A plan changed after create(): index entries outside the sequence are
    # clamped for reads and such rows are not stored, so nothing outside
    # Q/K/V and out is touched; the valid rows keep their results.
    plan = IndexedPlan.create(rows, keys, 1500).to("cuda")
    ref = sol_attention_indexed(*gpu, plan, beta=1.0)
    rows_t = plan.rows.clone()
    rows_t[0, 5] = -7
    rows_t[2, 9] = 1500 + 10
    tampered = IndexedPlan(rows_t, plan.keys, plan.protected_blocks, 1500, plan.key_lengths, True)
    out = torch.full_like(gpu[0], 3.0)
    sol_attention_indexed(*gpu, tampered, beta=1.0, out=out)
    torch.cuda.synchronize()
    # Window 1 is untouched: its rows hold exactly its result.
    assert torch.equal(out[plan.rows[1]], ref[1])
    # Every row the tampered plan does not name validly keeps its old value;
    # in particular rows 0 and 1499, where the bad entries were clamped for
    # reading, are not written.
    valid = torch.ones_like(rows_t, dtype=torch.bool)
    valid[0, 5] = valid[2, 9] = False
    untouched = torch.ones(1500, dtype=torch.bool, device="cuda")
    untouched[rows_t[valid]] = False
    assert bool(untouched[0]) and bool(untouched[1499])
    assert (out[untouched] == 3.0).all()
    assert torch.isfinite(out.float()).all()
