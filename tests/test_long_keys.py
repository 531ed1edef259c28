"""Key sequences longer than one routing segment.

The SOL kernel keeps each query block's routing bitmask in LDS for 8,192 key
blocks (524,288 tokens) and routes and attends longer key sequences one
segment of 8,192 blocks at a time, carrying one softmax state across the
segments.  The reference has no such bound (kernels.py:129 loops over every
key-block group), so these calls must agree with the oracle exactly as the
short ones do.

Workload: cross-attention, B = 1, 128 queries (two query blocks), 1,049,640
keys = 16,401 key blocks (segments of 8,192, 8,192 and 17 blocks; the last
block holds 40 valid tokens), one head, D = 128, random N(0, 1) inputs drawn
from one seeded CPU generator.  Query block 0 is a query sink (it selects
every key block, so its exact stream crosses every segment); query block 1 is
routed by the cutoff, beta = 0 selecting about half the blocks of every
segment.  Checked in both workgroup forms: routing decisions within the
band, exact-block counts, the output under identical routing, beta = +inf
(sinks and local band only) against the oracle, and beta = -inf through the
SOL kernel against the dense kernel.
"""

import math

import pytest
import torch

from sol_attn_amd import _native, dense_attention, sol_attention
from sol_testlib import HAS_GPU, assert_close
from test_kernels import check_routing

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]

TQ, TK, H, D = 128, 2 * 8192 * 64 + 16 * 64 + 40, 1, 128


@pytest.fixture(scope="module")
def long_keys():
    gen = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, t, H, D, generator=gen).to(torch.bfloat16).cuda() for t in (TQ, TK, TK))
    return q, k, v


@pytest.mark.parametrize("group", [1, 2])
@pytest.mark.parametrize("beta", [0.0, math.inf])
def test_long_keys_against_oracle(long_keys, group, beta, monkeypatch):
    monkeypatch.setattr(_native, "WORKGROUP_FORM", group)
    q, k, v = long_keys
    print(f"long keys: Tq {TQ} Tk {TK} H {H} D {D} form {group} beta {beta}", flush=True)
    actual, ref, _ = check_routing(q, k, v, beta, local=1, kv_sink=128, q_sink=64,
                                   label=f"long keys form {group}")
    assert_close(actual, ref)


@pytest.mark.parametrize("group", [1, 2])
def test_long_keys_every_block_exact_equals_dense(long_keys, group, monkeypatch):
    # A forced workgroup form keeps beta = -inf on the SOL kernel (its
    # every-block-exact segments) instead of the dense shortcut.
    monkeypatch.setattr(_native, "WORKGROUP_FORM", group)
    q, k, v = long_keys
    print(f"long keys beta -inf form {group}", flush=True)
    out, stats = sol_attention(q, k, v, beta=-math.inf, return_stats=True)
    assert stats.exact_blocks.eq(-(-TK // 64)).all()
    assert_close(out.cpu(), dense_attention(q, k, v).cpu())
