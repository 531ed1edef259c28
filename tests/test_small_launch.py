"""Small launches: one query block per workgroup with its exact tiles split
over key-split groups of two waves (sol_small_kernel), and, for at most 16
key blocks of plain K / V rows at head_dim 64, the keys pooled inside that
one launch.

Checks:
- routing within the band and outputs under identical routing against the
  oracle, counts equal to the decisions (check_routing, whole call);
- against the one-block kernel (forced workgroup form 1, no key split):
  equal decisions and counts, outputs equal to rounding;
- the self-pooled launch against the pooling kernel's buffers: bit-identical
  outputs and counts (the same centroids and moments);
- which launches take which path (sol_attention_pools_keys), repeats
  bitwise equal.
"""

import math

import pytest
import torch

from sol_attn_amd import IndexedPlan, _native, sol_attention, sol_attention_indexed
from sol_testlib import HAS_GPU, assert_close, block_smooth, tensors
from test_kernels import check_routing

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]

# (batch, query tokens, key tokens, heads, head_dim, inputs, query sink tokens)
CASES = [(1, 1024, 1024, 8, 64, "smooth", 128),    # one launch, keys pooled inside (the 1,024-token case)
         (1, 1024, 1024, 4, 128, "smooth", 128),   # D = 128, two key-split groups, pooling kernel first
         (2, 700, 1000, 3, 64, "random", 64),      # tails, 16 blocks pooled inside, two entries
         (1, 1500, 2000, 2, 128, "random", 128),   # 32 key blocks: centroid tiles from the pooling kernel
         (1, 600, 4000, 2, 64, "smooth", 0),       # 63 key blocks, 4 groups
         (1, 300, 40, 2, 64, "random", 0)]         # fewer keys than a block: block tiles


def inputs(case):
    b, tq, tk, h, d, kind, _ = case
    if kind == "smooth":
        return tuple(block_smooth(b, t, h, d, seed, device="cuda") for t, seed in ((tq, 71), (tk, 72), (tk, 73)))
    return tensors(nq=tq, nk=tk, d=d, b=b, h=h, device="cuda", seed=74)


def pools_keys(case):
    b, tq, tk, h, d, _, _ = case
    return bool(_native.library().sol_attention_pools_keys(b, tq, tk, h, d))


def test_paths_by_size():
    assert [pools_keys(c) for c in CASES] == [True, False, True, False, False, False]
    lib = _native.library()
    assert lib.sol_attention_pools_keys(1, 1024, 1025, 8, 64) == 0      # 17 key blocks
    assert lib.sol_attention_pools_keys(1, 4096, 1024, 16, 64) == 0     # 1,024 query blocks
    assert lib.sol_attention_pools_keys(1, 1024, 63, 8, 64) == 0        # below one block: block tiles


@pytest.mark.parametrize("beta", [1.0, 0.0, math.inf])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_small_launch_against_oracle(case, beta):
    c = CASES[case]
    q, k, v = inputs(c)
    print(f"small launch case {case} beta {beta}", flush=True)
    actual, ref, _ = check_routing(q, k, v, beta, local=1, kv_sink=64, q_sink=c[6], label=f"small {case}")
    assert_close(actual, ref)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_small_launch_against_the_one_block_kernel(case, monkeypatch):
    c = CASES[case]
    q, k, v = inputs(c)
    kw = dict(beta=1.0, kv_sink_tokens=min(64, c[2]), query_sink_tokens=c[6], return_stats=True)
    print(f"small launch case {case}: key split vs one-block kernel", flush=True)
    split, split_stats = sol_attention(q, k, v, **kw)
    again, _ = sol_attention(q, k, v, **kw)
    assert torch.equal(split, again)
    monkeypatch.setattr(_native, "WORKGROUP_FORM", 1)
    one, one_stats = sol_attention(q, k, v, **kw)
    assert torch.equal(split_stats.exact_blocks, one_stats.exact_blocks)
    assert_close(split.cpu(), one.cpu())


@pytest.mark.parametrize("beta", [1.0, math.inf])
@pytest.mark.parametrize("case", [0, 2])
def test_self_pooled_launch_is_bit_identical(case, beta, monkeypatch):
    c = CASES[case]
    q, k, v = inputs(c)
    kw = dict(beta=beta, kv_sink_tokens=64, query_sink_tokens=c[6], return_stats=True)
    print(f"self-pooled case {case} beta {beta}", flush=True)
    one, one_stats = sol_attention(q, k, v, **kw)
    monkeypatch.setattr(_native, "SELF_POOLING", False)
    two, two_stats = sol_attention(q, k, v, **kw)
    assert torch.equal(one, two)
    assert torch.equal(one_stats.exact_blocks, two_stats.exact_blocks)


def test_small_launch_full_covariance_and_indexed_windows():
    # Full covariance keeps the pooling kernel (its covariance pass reads the
    # centroid tiles) and runs the small kernel over them.
    c = CASES[0]
    q, k, v = inputs(c)
    print("small launch: full covariance", flush=True)
    actual, ref, _ = check_routing(q, k, v, 1.0, local=1, kv_sink=64, q_sink=128, estimator="full_covariance",
                                   label="small cov")
    assert_close(actual, ref)
    # Indexed windows over a short sequence: gathered block tiles, scatter.
    n, h, d = 2000, 2, 64
    g = torch.Generator().manual_seed(5)
    qn, kn, vn = (torch.randn((n, h, d), generator=g).to(torch.bfloat16).cuda() for _ in range(3))
    rows = torch.stack([torch.arange(0, 200), torch.arange(1000, 1200)])
    keys = torch.stack([torch.arange(0, 700), torch.arange(900, 1600)])
    plan = IndexedPlan.create(rows, keys, n, protected_ranges=((0, 64),)).to("cuda")
    print("small launch: indexed windows", flush=True)
    got, stats = sol_attention_indexed(qn, kn, vn, plan, beta=1.0, return_stats=True)
    out = torch.zeros_like(qn)
    sol_attention_indexed(qn, kn, vn, plan, beta=1.0, out=out)
    assert torch.equal(out[rows.reshape(-1).cuda()], got.reshape(-1, h, d))
    _native.WORKGROUP_FORM = 1
    try:
        one, one_stats = sol_attention_indexed(qn, kn, vn, plan, beta=1.0, return_stats=True)
    finally:
        _native.WORKGROUP_FORM = 0
    assert torch.equal(stats.exact_blocks, one_stats.exact_blocks)
    assert_close(got.cpu(), one.cpu())
