"""Parity at the headline size: 84,672 tokens (a 21 x 48 x 84 smooth field),
24 heads, D = 128, beta 1, kv and query sinks of 128 tokens, local band 1.

The oracle runs on a sample of query blocks (the first, a query sink that
selects every key block; one from the middle; the last) x all 24 heads:
routing decisions within the stated band, proxies, cutoffs, counts, and the
outputs under identical routing.  Whole-size properties: the exact-block
counts equal the decision masks' popcounts (checked on the sample above), a
repeated call is bit-identical, and beta = -inf equals the dense kernel
within the BF16 tolerance.
"""

import math

import pytest
import torch

import bench
from sol_attn_amd import dense_attention, sol_attention
from sol_testlib import HAS_GPU, assert_close
from test_kernels import check_routing

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
