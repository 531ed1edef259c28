"""GPU tests of the opt-in INT8-QK variant (``qk_precision="int8"``).

Not in the reference: its roadmap (ROADMAP.md:14-16) asks for a separately
measured INT8 QK beside a BF16 control.  The oracle's ``qk_precision="int8"``
quantises exactly as the kernels do (per query row and per 64-key block,
symmetric, round half to even), so the INT8 K tiles and scales must equal the
oracle's bit for bit, the integer dot products are exact on both sides, and
the outputs differ only by FP32 summation order: the same tolerance as the
BF16 parity tests, exact-block counts equal (routing stays BF16).
"""

import math

import numpy as np
import pytest
import torch

from oracle import sol_oracle as orc
from sol_attn_amd import _native, IndexedPlan, sol_attention, sol_attention_indexed
from sol_testlib import HAS_GPU, assert_close, block_smooth, tensors

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


def k8_rows(buf, d):
    """Undo the INT8 tile swizzle of one key block: 16-byte chunk c of row r
    sits at byte r * d + 16 * (c ^ swizzle(r)), swizzle(r) = (r >> 1) & 7 for
    d = 128 and (r >> 2) & 3 for d = 64.  Returns ``[64, d]`` int8."""
    buf = np.asarray(buf).reshape(64, d // 16, 16)
    rows = np.arange(64)
    swz = (rows >> 1) & 7 if d == 128 else (rows >> 2) & 3
    chunks = np.arange(d // 16)[None, :] ^ swz[:, None]
    return buf[rows[:, None], chunks].reshape(64, d)


@pytest.mark.parametrize("d,nk", [(64, 317), (128, 317), (128, 64), (64, 1), (128, 65)])
def test_quantised_key_tiles_equal_the_oracle(d, nk):
    q, k, v = tensors(nq=70, nk=nk, d=d, b=2, h=3, device="cuda", strided=True)
    k[0, :, 1] *= 40  # one head on a wider scale
    pooled = _native.pool_kv(k, v, moments=False, qk_int8=True)
    torch.cuda.synchronize()
    shifted = pooled["tiles"] is None  # rows mode: the partial last block holds the last 64 keys
    b, h, nkb = pooled["k8_scale"].shape
    k8 = pooled["workspace"][pooled["k8_ptr"] - pooled["workspace"].data_ptr():][:b * h * nkb * 64 * d]
    k8 = k8.view(torch.int8).view(b, h, nkb, 64 * d).cpu().numpy()
    kf = k.float().cpu().numpy()
    ref_q, ref_s = orc.quantize_keys(kf)
    np.testing.assert_array_equal(pooled["k8_scale"].cpu().numpy(), ref_s.transpose(0, 2, 1))
    for bi in range(b):
        for hi in range(h):
            for j in range(nkb):
                rows = min(64, nk - 64 * j)
                got = k8_rows(k8[bi, hi, j], d)
                if shifted and rows < 64:
                    # Keys nk - 64 .. nk - 1: the block's own are the last `rows`;
                    # the others (the previous block's) at this block's scale, clamped.
                    np.testing.assert_array_equal(got[64 - rows:], ref_q[bi, 64 * j:, hi])
                    inv = np.float32(127.0) / np.abs(kf[bi, 64 * j:, hi]).max()
                    prev = np.clip(np.rint(kf[bi, nk - 64:64 * j, hi] * inv), -127, 127)
                    np.testing.assert_array_equal(got[:64 - rows], prev)
                else:
                    np.testing.assert_array_equal(got[:rows], ref_q[bi, 64 * j:64 * j + rows, hi])
                    assert (got[rows:] == 0).all()


@pytest.mark.parametrize("group", ["1", "2"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("beta", [-math.inf, math.inf, 1.0])
def test_int8_qk_matches_the_int8_oracle(d, beta, group, monkeypatch):
    monkeypatch.setattr(_native, "WORKGROUP_FORM", int(group))
    q, k, v = tensors(d=d, b=2, device="cuda", strided=True)
    actual, stats = sol_attention(q, k, v, beta=beta, return_stats=True, qk_precision="int8")
    ref, counts, _ = orc.sol_oracle(q.cpu(), k.cpu(), v.cpu(), beta=beta, qk_precision="int8")
    assert_close(actual.cpu(), ref)
    np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)
    assert torch.equal(actual, sol_attention(q, k, v, beta=beta, qk_precision="int8"))
    assert counts.max() > 0
    assert not torch.equal(actual, sol_attention(q, k, v, beta=beta))  # the quantised products did run


@pytest.mark.parametrize("group", ["1", "2"])
def test_int8_qk_multiple_groups_tail_and_smooth_inputs(group, monkeypatch):
    # 17 query blocks, a 1-key tail block, block-smooth data (the routed regime).
    monkeypatch.setattr(_native, "WORKGROUP_FORM", int(group))
    q, k, v = (block_smooth(1, n, 2, 128, seed, device="cuda") for n, seed in ((1025, 1), (1089, 2), (1089, 3)))
    for beta in (1.0, 0.0):
        actual, stats = sol_attention(q, k, v, beta=beta, return_stats=True, qk_precision="int8")
        ref, counts, _ = orc.sol_oracle(q.cpu(), k.cpu(), v.cpu(), beta=beta, qk_precision="int8")
        assert_close(actual.cpu(), ref)
        np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)


def test_int8_qk_indexed_windows():
    g = torch.Generator().manual_seed(11)
    x = [torch.randn((700, 3, 64), generator=g, dtype=torch.bfloat16).cuda() for _ in range(3)]
    rows = torch.stack((torch.arange(0, 150), torch.arange(300, 450)))
    keys = torch.stack((torch.arange(100, 400), torch.arange(350, 650)))
    p = IndexedPlan.create(rows, keys, 700, protected_ranges=((100, 110),), local_tokens=64).to("cuda")
    out, stats = sol_attention_indexed(*x, p, beta=0.5, return_stats=True, qk_precision="int8")
    ref, counts, _ = orc.sol_oracle(x[0].cpu()[rows], x[1].cpu()[keys], x[2].cpu()[keys], beta=0.5,
                                    local_blocks=-1, protected_blocks=p.protected_blocks.cpu(),
                                    qk_precision="int8")
    assert_close(out.cpu(), ref)
    np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)


def test_int8_qk_rejects_unknown_precisions():
    q, k, v = tensors(device="cuda")
    with pytest.raises(ValueError):
        sol_attention(q, k, v, qk_precision="fp8")
