"""GPU parity tests of the BTHD API, mirroring the reference's tests/test_attention.py.

The HIP kernels are compared with the oracle (oracle/sol_oracle.py) on the
same BF16 inputs: outputs within the reference tolerance, exact-block counts
exactly equal, repeat calls bitwise equal.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.sol_oracle import sol_oracle
from sol_attn_amd import _native, dense_attention, sol_attention
from sol_testlib import HAS_GPU, assert_close, tensors

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


def sdpa(q, k, v):
    return F.scaled_dot_product_attention(q.float().cpu().transpose(1, 2), k.float().cpu().transpose(1, 2),
                                          v.float().cpu().transpose(1, 2)).transpose(1, 2)


# Both workgroup forms: one query block per workgroup (what these small
# launches use by default) and two blocks over their union (what large
# launches use).
GROUPS = ["1", "2"]


@pytest.mark.parametrize("group", GROUPS)
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("beta", [-math.inf, math.inf, 1.0])
@pytest.mark.parametrize("strided", [False, True])
def test_sol_ragged_cross_attention(d, beta, strided, group, monkeypatch):
    # test_attention.py:55-69
    monkeypatch.setattr(_native, "WORKGROUP_FORM", int(group))
    q, k, v = tensors(d=d, b=2, device="cuda", strided=strided)
    actual, stats = sol_attention(q, k, v, beta=beta, return_stats=True)
    ref, counts, _ = sol_oracle(q.cpu(), k.cpu(), v.cpu(), beta=beta)
    assert_close(actual.cpu(), ref)
    np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)
    repeated = sol_attention(q, k, v, beta=beta)
    assert torch.equal(actual, repeated)


@pytest.mark.parametrize("nq,nk", [(1, 1), (63, 65), (64, 64), (65, 63), (1025, 1089)])
def test_dense_tail(nq, nk):
    # test_attention.py:72-80
    q, k, v = tensors(nq=nq, nk=nk, d=128, device="cuda")
    actual = dense_attention(q, k, v)
    assert actual.shape == q.shape and actual.is_contiguous()
    assert_close(actual.cpu(), sdpa(q, k, v))


@pytest.mark.parametrize("d", [64, 128])
def test_dense_strided_and_repeatable(d):
    q, k, v = tensors(nq=300, nk=517, d=d, b=2, h=3, device="cuda", strided=True)
    actual = dense_attention(q, k, v)
    assert_close(actual.cpu(), sdpa(q, k, v))
    assert torch.equal(actual, dense_attention(q, k, v))


@pytest.mark.parametrize("shape", [(2, 193, 317, 2, 64), (1, 1025, 1089, 3, 128), (1, 70, 40, 2, 128)])
def test_all_exact_beta_takes_the_dense_kernel_bit_identically(shape, monkeypatch):
    # beta = -inf on plain inputs runs the dense kernel; the SOL kernel (a
    # forced workgroup form) gives the same bits and exact-block counts.
    b, nq, nk, h, d = shape
    q, k, v = tensors(nq=nq, nk=nk, d=d, b=b, h=h, device="cuda", strided=True)
    out, stats = sol_attention(q, k, v, beta=-math.inf, return_stats=True)
    assert torch.equal(out, dense_attention(q, k, v))
    for group in (1, 2):
        monkeypatch.setattr(_native, "WORKGROUP_FORM", group)
        sol, sol_stats = sol_attention(q, k, v, beta=-math.inf, return_stats=True)
        assert torch.equal(out, sol)
        assert torch.equal(stats.exact_blocks, sol_stats.exact_blocks)
    assert stats.density() == 1.0


def test_sol_zero_inputs_and_exact_sinks():
    # test_attention.py:83-93
    q, k, v = tensors(device="cuda")
    q.zero_(); k.zero_()
    actual, stats = sol_attention(q, k, v, beta=math.inf, local_blocks=0,
                                  kv_sink_tokens=65, query_sink_tokens=1, return_stats=True)
    ref, counts, _ = sol_oracle(q.cpu(), k.cpu(), v.cpu(), beta=math.inf, local_blocks=0,
                                kv_sink_tokens=65, query_sink_tokens=1)
    assert_close(actual.cpu(), ref)
    np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)


def test_sol_single_token_no_empty_mass_nan():
    # test_attention.py:96-101
    q, k, v = tensors(nq=1, nk=1, device="cuda")
    for beta in (-math.inf, math.inf, 1.0):
        assert torch.equal(sol_attention(q, k, v, beta=beta), v)


@pytest.mark.parametrize("group", GROUPS)
@pytest.mark.parametrize("beta", [-math.inf, math.inf, 1.0])
def test_sol_multiple_groups_and_tail(beta, group, monkeypatch):
    # test_attention.py:104-112; 17 query blocks: the last two-block
    # workgroup holds one live block.
    monkeypatch.setattr(_native, "WORKGROUP_FORM", int(group))
    q, k, v = tensors(nq=1025, nk=1089, h=1, device="cuda")
    actual, stats = sol_attention(q, k, v, beta=beta, return_stats=True)
    ref, counts, _ = sol_oracle(q.cpu(), k.cpu(), v.cpu(), beta=beta)
    assert_close(actual.cpu(), ref)
    np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)


def test_sol_rows_with_no_exact_blocks():
    # test_attention.py:115-123
    q, k, v = tensors(nq=321, nk=65, h=1, device="cuda")
    actual, stats = sol_attention(q, k, v, beta=math.inf, local_blocks=0, return_stats=True)
    ref, counts, _ = sol_oracle(q.cpu(), k.cpu(), v.cpu(), beta=math.inf, local_blocks=0)
    assert (stats.exact_blocks[:, 2:] == 0).all()
    assert_close(actual.cpu(), ref)
    np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)


def test_sol_preserves_inputs_and_rejects_masks():
    # test_attention.py:126-135
    q, k, v = tensors(device="cuda")
    copies = tuple(x.clone() for x in (q, k, v))
    sol_attention(q, k, v)
    for x, copy in zip((q, k, v), copies):
        assert torch.equal(x, copy)
    with pytest.raises(TypeError):
        sol_attention(q, k, v, attn_mask=torch.ones((193, 317), device="cuda"))


def test_sol_rejects_invalid_controls():
    # test_attention.py:138-146
    q, k, v = tensors(device="cuda")
    for controls in ({"beta": math.nan}, {"local_blocks": -1},
                     {"kv_sink_tokens": 318}, {"query_sink_tokens": 194},
                     {"scale": 0}, {"scale": math.inf}):
        with pytest.raises(ValueError):
            sol_attention(q, k, v, **controls)


def test_sol_misaligned_view_is_copied_not_written():
    # A view whose rows are not 16-byte aligned goes through one GPU copy.
    q, k, v = tensors(nq=200, nk=300, d=64, device="cuda")
    base = torch.zeros(1 + q.numel(), device="cuda", dtype=torch.bfloat16)
    qm = base[1:].view(q.shape)
    qm.copy_(q)
    assert qm.data_ptr() % 16 != 0
    actual = sol_attention(qm, k, v, beta=1.0)
    assert torch.equal(actual, sol_attention(q, k, v, beta=1.0))
    assert torch.equal(qm, q)
