"""Full-covariance thresholds (the reference roadmap's experiment; not in the reference).

GPU: the key covariance (sol_key_covariance) against the oracle's float64
estimator, and its exact symmetry; routing decisions, cutoffs and outputs against the oracle under
the full-covariance cutoff (the same band and tolerances as the diagonal
path); beta = 0 makes both estimators identical; ragged indexed windows.
"""

import math

import numpy as np
import pytest
import torch

from oracle import sol_oracle as orc
from sol_attn_amd import IndexedPlan, _native, sol_attention, sol_attention_indexed
from sol_testlib import HAS_GPU, assert_close, block_smooth, tensors, to_np
from test_kernels import check_routing

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


def correlated(b, t, h, d, seed):
    """BF16 [B, T, H, D] whose block means have strongly correlated features."""
    g = torch.Generator().manual_seed(seed)
    nb = -(-t // 64)
    mix = torch.randn((d, d), generator=g) * (0.6 / math.sqrt(d))
    centres = torch.randn((b, nb, h, d), generator=g) @ (torch.eye(d) + mix) + 0.2
    x = centres.repeat_interleave(64, 1)[:, :t] + 0.1 * torch.randn((b, t, h, d), generator=g)
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("shape", [(1, 317, 2, 64), (2, 1089, 3, 128), (1, 4096, 4, 128)])
def test_key_covariance_matches_oracle(shape):
    b, t, h, d = shape
    k, v = correlated(b, t, h, d, 1), correlated(b, t, h, d, 2)
    pooled = _native.key_covariance(_native.pool_kv(k.cuda(), v.cuda()))
    cov = to_np(pooled["cov"].cpu())
    kc = orc.block_means(to_np(k), True)
    ref = orc.key_covariance(kc)
    np.testing.assert_allclose(cov, ref, rtol=0, atol=2e-6 * np.abs(ref).max() + 1e-7)
    # Symmetric bit for bit: the cutoff stages read column d for row d.
    np.testing.assert_array_equal(cov, np.swapaxes(cov, -1, -2))
    # Its diagonal is the diagonal estimator's variance before the clamp.
    _, var = orc.key_moments(kc)
    diag = np.diagonal(cov, axis1=-2, axis2=-1)
    np.testing.assert_allclose(np.maximum(diag, 0), var, rtol=0, atol=2e-6 * var.max() + 1e-7)


@pytest.mark.parametrize("beta", [0.5, 1.0, -1.0])
@pytest.mark.parametrize("d", [64, 128])
def test_full_covariance_routing_and_output(beta, d):
    q, k, v = (correlated(1, 4096, 4, d, s).cuda() for s in (3, 4, 5))
    got, ref, _ = check_routing(q, k, v, beta, estimator="full_covariance")
    assert_close(got, ref)


def test_full_covariance_differs_from_diagonal_and_beta_zero_matches():
    q, k, v = (correlated(1, 4096, 4, 128, s).cuda() for s in (6, 7, 8))
    _, diag = sol_attention(q, k, v, beta=1.0, return_stats=True)
    _, full = sol_attention(q, k, v, beta=1.0, return_stats=True, threshold_estimator="full_covariance")
    assert not torch.equal(diag.exact_blocks, full.exact_blocks)  # correlated features move the cutoff
    a = sol_attention(q, k, v, beta=0.0)
    b = sol_attention(q, k, v, beta=0.0, threshold_estimator="full_covariance")
    assert torch.equal(a, b)
    for beta in (-math.inf, math.inf):  # forced routing ignores the estimator
        assert torch.equal(sol_attention(q, k, v, beta=beta),
                           sol_attention(q, k, v, beta=beta, threshold_estimator="full_covariance"))


@pytest.mark.parametrize("group", ["1", "2"])  # one- and two-block workgroups
def test_full_covariance_ragged_windows_match_oracle(group, monkeypatch):
    monkeypatch.setattr(_native, "WORKGROUP_FORM", int(group))
    x = [correlated(1, 3000, 2, 64, s)[0].cuda() for s in (9, 10, 11)]
    rows = torch.stack((torch.arange(0, 700), torch.arange(1500, 2200)))
    keys = [torch.arange(0, 1200), torch.arange(900, 3000)]
    plan = IndexedPlan.create(rows, keys, 3000, protected_ranges=((0, 64),), local_tokens=64).to("cuda")
    out, stats = sol_attention_indexed(*x, plan, beta=1.0, return_stats=True, threshold_estimator="full_covariance")
    with torch.no_grad():
        _, _, dbg = _native.launch_sol(x[0], x[1], x[2], 64 ** -0.5, 1.0, -1, 0, 0, True, plan.protected_blocks,
                                       rows=plan.rows, keys=plan.keys, key_lengths=plan.key_lengths,
                                       debug=True, threshold_estimator="full_covariance")
    ksel = to_np(dbg["selected"].cpu()).astype(bool)
    for w in range(2):
        kv = keys[w]
        nkb = -(-len(kv) // 64)
        args = (to_np(x[0][rows[w]].cpu())[None], to_np(x[1][kv].cpu())[None], to_np(x[2][kv].cpu())[None])
        kw = dict(beta=1.0, local_blocks=-1, threshold_estimator="full_covariance",
                  protected_blocks=plan.protected_blocks[w:w + 1, :, :nkb].cpu())
        _, _, info = orc.sol_oracle(*args, **kw)
        sel = ksel[w:w + 1, :, :, :nkb]
        assert (sel != info["selected"]).mean() < 1e-3          # only near-tie decisions may differ
        np.testing.assert_allclose(to_np(dbg["cutoff"].cpu())[w:w + 1], info["cutoff"], rtol=1e-4,
                                   atol=1e-5 * np.abs(info["cutoff"]).max())
        ref, counts, _ = orc.sol_oracle(*args, **kw, selected=sel)    # outputs under identical routing
        assert_close(to_np(out[w].cpu())[None], ref)
        np.testing.assert_array_equal(stats.exact_blocks[w].cpu().numpy(), counts[0])


def test_invalid_estimator_is_rejected():
    q, k, v = (x.cuda() for x in tensors())
    with pytest.raises(ValueError, match="threshold_estimator"):
        sol_attention(q, k, v, threshold_estimator="banded")
