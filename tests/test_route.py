"""The routing kernel (sol_attention_fwd with a route_workspace): cutoffs and
every (query block, key block) decision formed before attention, against the
oracle within the routing band, with the query-block means taken from the
pairing pass or formed from Q, for plain, strided, ragged-tail and indexed
inputs; and the attention kernel's own tile-by-tile routing gives the same
outputs wherever the decisions agree."""

import math

import numpy as np
import pytest
import torch

from oracle import sol_oracle as orc
from sol_attn_amd import IndexedPlan, _native, sol_attention, sol_attention_indexed
from sol_testlib import HAS_GPU, assert_close, block_smooth, tensors, to_np
from test_kernels import check_routing, run_debug

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


@pytest.fixture
def prepass(monkeypatch):
    monkeypatch.setattr(_native, "ROUTE_PREPASS", "always")
    return monkeypatch


@pytest.mark.parametrize("means", ["pairing", "from_q"])
@pytest.mark.parametrize("beta", [0.0, 1.0, math.inf])
@pytest.mark.parametrize("case", [dict(nq=300, nk=517, d=128, b=1, h=2, strided=True),
                                  dict(nq=777, nk=1500, d=64, b=2, h=3),
                                  dict(nq=1024, nk=4000, d=128, b=1, h=2),
                                  # 782 key blocks = 25 chunks of 32: two key ranges per query-block group
                                  dict(nq=640, nk=50000, d=64, b=1, h=2)])
def test_routing_kernel_against_oracle(prepass, case, beta, means):
    if means == "pairing":
        prepass.setattr(_native, "PAIR_MIN_QUERY_BLOCKS", 1)   # pairing also writes the query means
    else:
        prepass.setattr(_native, "PAIRING", False)             # the routing kernel forms them from Q
    q, k, v = tensors(device="cuda", seed=11, **case)
    actual, ref, _ = check_routing(q, k, v, beta, kv_sink=64, q_sink=64, local=1,
                                   label=f"route kernel {means}")
    assert_close(actual, ref)


def test_routing_kernel_smooth_input_and_full_covariance(prepass):
    prepass.setattr(_native, "PAIR_MIN_QUERY_BLOCKS", 1)
    q, k, v = (block_smooth(1, 2000, 4, 128, seed=s, device="cuda") for s in (1, 2, 3))
    for est in ("diagonal_covariance", "full_covariance"):
        actual, ref, _ = check_routing(q, k, v, 1.0, kv_sink=128, q_sink=128, estimator=est,
                                       label=f"route kernel {est}")
        assert_close(actual, ref)


def test_routing_kernel_indexed_windows_with_protection(prepass):
    g = torch.Generator().manual_seed(5)
    n, h, d = 3000, 2, 64
    q, k, v = (torch.randn((n, h, d), generator=g).to(torch.bfloat16) for _ in range(3))
    rows = torch.stack([torch.arange(0, 700), torch.arange(1500, 2200)])
    keys = torch.stack([torch.arange(0, 1400), torch.arange(1000, 2400)])
    plan = IndexedPlan.create(rows, keys, n, protected_ranges=((0, 100),), local_tokens=64)
    dev = plan.to("cuda")
    out, stats = sol_attention_indexed(q.cuda(), k.cuda(), v.cuda(), dev, beta=1.0, return_stats=True)
    for w in range(2):
        nkb = -(-keys.shape[1] // 64)
        ref, counts, _ = orc.sol_oracle(to_np(q[rows[w]])[None], to_np(k[keys[w]])[None], to_np(v[keys[w]])[None],
                                        beta=1.0, local_blocks=-1,
                                        protected_blocks=plan.protected_blocks[w:w + 1, :, :nkb].numpy())
        assert_close(out[w:w + 1].cpu(), ref)
        np.testing.assert_array_equal(stats.exact_blocks[w:w + 1].cpu().numpy(), counts)


@pytest.mark.parametrize("beta", [0.5, math.inf])
def test_routing_kernel_equals_in_kernel_routing_where_decisions_agree(monkeypatch, beta):
    q, k, v = (block_smooth(2, 3000, 3, 128, seed=s, device="cuda") for s in (7, 8, 9))
    monkeypatch.setattr(_native, "ROUTE_PREPASS", False)
    a, ca, da = run_debug(q, k, v, beta, kv_sink=64, q_sink=64)
    monkeypatch.setattr(_native, "ROUTE_PREPASS", "always")
    b, cb, db = run_debug(q, k, v, beta, kv_sink=64, q_sink=64)
    same = (da["selected"] == db["selected"]).all(-1)          # [B, NQB, H]: every decision equal
    assert same.float().mean().item() > 0.99
    rows = same.repeat_interleave(64, 1)[:, :q.shape[1]]       # [B, Tq, H]
    assert torch.equal(a[rows], b[rows])
    assert torch.equal(ca[same], cb[same])
    if math.isinf(beta):
        assert torch.equal(da["selected"], db["selected"])
