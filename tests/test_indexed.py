"""GPU parity of the indexed-window path, mirroring the reference's tests/test_indexed.py."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.sol_oracle import sol_oracle
from sol_attn_amd import IndexedPlan, sol_attention_indexed
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
