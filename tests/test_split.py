"""Query-sink tiles split by key range.

A query-sink block selects every key block.  In short launches (at most
8,192 query blocks over all (entry, head) pairs) its workgroup would end long
after the others, so the key blocks of sink blocks [0, 2 floor(sinks / 2))
are split over up to 8 workgroups, and a second kernel merges their partial
softmax states.  The split calls must satisfy four properties:
- they match the oracle as unsplit calls do (routing, counts, outputs under
  identical routing);
- they agree with the unsplit kernel to rounding, with equal counts;
- the two workgroup forms stay bit-identical, because whether a query block
  is split depends on its index alone;
- repeat calls are bitwise equal.
"""

import math

import pytest
import torch

from sol_attn_amd import _native, sol_attention
from sol_testlib import HAS_GPU, assert_close, block_smooth, tensors
from test_kernels import check_routing

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]

# (batch, query tokens, key tokens, heads, head_dim, query sink tokens, inputs):
# 64 query blocks x 4 heads with two sink blocks (4 parts of 16 key blocks);
# three sink blocks (block 2 stays whole), tails, four parts, random inputs.
CASES = [(1, 4096, 4096, 4, 128, 128, "smooth"),
         (2, 1000, 5000, 3, 64, 192, "random")]


def inputs(case):
    b, tq, tk, h, d, _, kind = case
    if kind == "smooth":
        return tuple(block_smooth(b, t, h, d, seed, device="cuda") for t, seed in ((tq, 61), (tk, 62), (tk, 63)))
    return tensors(nq=tq, nk=tk, d=d, b=b, h=h, device="cuda", seed=64)


def split_bytes(case, beta):
    b, tq, tk, h, d, qs, _ = case
    return _native.library().sol_split_workspace_size(b, tq, tk, h, d, beta, qs)


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("beta", [1.0, 0.0, math.inf])
def test_split_sinks_against_oracle(case, beta):
    c = CASES[case]
    assert split_bytes(c, beta) > 0
    q, k, v = inputs(c)
    print(f"split case {case} beta {beta}", flush=True)
    actual, ref, _ = check_routing(q, k, v, beta, local=1, kv_sink=64, q_sink=c[5], label=f"split {case}")
    assert_close(actual, ref)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_split_agrees_with_unsplit_and_forms_are_identical(case, monkeypatch):
    c = CASES[case]
    q, k, v = inputs(c)
    kw = dict(beta=1.0, kv_sink_tokens=64, query_sink_tokens=c[5], return_stats=True)
    print(f"split case {case}: split vs unsplit, forms", flush=True)
    split, split_stats = sol_attention(q, k, v, **kw)
    assert torch.equal(split, sol_attention(q, k, v, **kw)[0])  # deterministic
    monkeypatch.setattr(_native, "SPLIT_SINKS", False)
    whole, whole_stats = sol_attention(q, k, v, **kw)
    assert torch.equal(split_stats.exact_blocks, whole_stats.exact_blocks)
    assert_close(split.cpu(), whole.cpu())
    assert split_bytes(c, 1.0) > 0  # the split path ran (outputs may still agree bit for bit)
    monkeypatch.setattr(_native, "SPLIT_SINKS", True)
    forms = {}
    for g in (1, 2):
        monkeypatch.setattr(_native, "WORKGROUP_FORM", g)
        forms[g] = sol_attention(q, k, v, **kw)
    assert torch.equal(forms[1][0], forms[2][0])
    assert torch.equal(forms[1][1].exact_blocks, forms[2][1].exact_blocks)
    assert torch.equal(forms[1][1].exact_blocks, split_stats.exact_blocks)

