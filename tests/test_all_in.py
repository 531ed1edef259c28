"""One C-ABI call for pooling + attention (sol_attention_all_in), the path
plain BTHD calls without query-block pairing take.

CPU: the workspace-size query against the layout it promises (0 when the
attention launch pools its keys itself, the sol_pool_kv buffers 256-byte
aligned otherwise, the block tiles only outside rows mode, no moments at
beta = +inf, the split workspace) and its rejections; argument errors of the
entry point before any launch.
GPU: outputs and counts bit-identical to sol_pool_kv + sol_attention_fwd
(the same kernels and workspace layout, the moments from moments_kernel) on
every path the call can take -- keys pooled inside the launch, the
small-launch kernel after the pooling kernel, split query sinks, the
one-block kernel, block tiles for fewer than 64 keys, beta = +inf,
head-strided K / V, key moments folded inside the attention launch from 2 to
16 chunk sums, centroid tiles pooled alone (at most 16 key blocks) with the
moments formed from them in the attention launch -- and against the oracle
on one case.
"""

import ctypes
import math
import os

import pytest
import torch

from sol_attn_amd import _native, sol_attention
from sol_testlib import HAS_GPU, assert_close, block_smooth, tensors, to_np

gpu = pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")
built = pytest.mark.skipif(not os.path.exists(_native.LIB_PATH), reason="libsol_attn_amd.so not built")


def _aligned(n):
    return -(-n // 256) * 256


@built
def test_workspace_size_follows_the_pooling_layout():
    lib = _native.library()
    size = lib.sol_attention_workspace_size
    # Keys pooled inside the attention launch: no workspace.
    assert size(1, 1024, 1024, 8, 64, 1.0, 128, 512, 512) == 0
    assert bool(lib.sol_attention_pools_keys(1, 1024, 1024, 8, 64))
    # 1,024 keys x 4 heads at D = 128 (rows mode): centroid tiles, chunk sums,
    # mean and variance, each 256-byte aligned; no split (small kernel).
    sizes = (ctypes.c_int64 * 4)()
    assert lib.sol_pool_sizes(1, 1024, 4, 128, sizes) == 0
    moments = _aligned(sizes[0]) + _aligned(sizes[2]) + 2 * _aligned(sizes[3])
    assert size(1, 1024, 1024, 4, 128, 1.0, 0, 512, 512) == moments
    # beta = +inf: no moments; beta = -inf: no moments either.
    assert size(1, 1024, 1024, 4, 128, math.inf, 0, 512, 512) == _aligned(sizes[0])
    assert size(1, 1024, 1024, 4, 128, -math.inf, 0, 512, 512) == _aligned(sizes[0])
    # Fewer than 64 keys, or a token stride of 2^24 elements: block tiles too.
    assert lib.sol_pool_sizes(1, 40, 2, 64, sizes) == 0
    tiles = _aligned(sizes[0]) + _aligned(sizes[1]) + _aligned(sizes[2]) + 2 * _aligned(sizes[3])
    assert size(1, 300, 40, 2, 64, 1.0, 0, 128, 128) == tiles
    assert lib.sol_pool_sizes(1, 2000, 2, 64, sizes) == 0
    assert size(1, 300, 2000, 2, 64, 1.0, 0, 1 << 24, 128) == \
        _aligned(sizes[0]) + _aligned(sizes[1]) + _aligned(sizes[2]) + 2 * _aligned(sizes[3])
    # Split query sinks: the split workspace follows the pooled buffers.
    split = lib.sol_split_workspace_size(1, 4096, 4096, 4, 128, 1.0, 128)
    assert split > 0
    assert lib.sol_pool_sizes(1, 4096, 4, 128, sizes) == 0
    assert size(1, 4096, 4096, 4, 128, 1.0, 128, 512, 512) == \
        _aligned(sizes[0]) + _aligned(sizes[2]) + 2 * _aligned(sizes[3]) + _aligned(split)
    # Invalid sizes.
    assert size(1, 1024, 1024, 4, 96, 1.0, 0, 512, 512) == -1
    assert size(1, 1024, 1024, 4, 128, math.nan, 0, 512, 512) == -1
    assert size(1, 1024, 1024, 4, 128, 1.0, -1, 512, 512) == -1
    assert size(1, 1024, 1024, 4, 128, 1.0, 0, 0, 512) == -1


@built
def test_all_in_rejects_bad_arguments_before_any_launch():
    lib = _native.library()
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call fails its checks
    st = (ctypes.c_int64 * 3)(128 * 4 * 1024, 128 * 4, 128)
    call = lambda *a: lib.sol_attention_all_in(fake, st, fake, st, fake, st, 1, 1024, 1024, 4, 128, *a)
    assert call(0.088, 1.0, 1, 0, 0, None, 0, fake, None, None) == -1   # needs a workspace
    assert b"sol_attention_workspace_size" in lib.sol_last_error()
    assert call(0.088, 1.0, 1, 0, 0, fake, -8, fake, None, None) == -1
    assert call(0.088, 1.0, 1, 0, 0, None, 64, fake, None, None) == -1
    assert call(-1.0, 1.0, 1, 0, 0, fake, 1 << 30, fake, None, None) == -1
    assert b"scale" in lib.sol_last_error()
    assert call(0.088, 1.0, 1, 0, 0, ctypes.c_void_p((1 << 20) + 8), 1 << 30, fake, None, None) == -1
    assert b"workspace" in lib.sol_last_error()


def _two_calls(q, k, v, kw, monkeypatch):
    monkeypatch.setattr(_native, "ALL_IN", False)
    try:
        return sol_attention(q, k, v, **kw)
    finally:
        monkeypatch.setattr(_native, "ALL_IN", True)


# (batch, query tokens, key tokens, heads, head_dim, beta, kv sink, q sink, inputs)
CASES = [(1, 1024, 1024, 8, 64, 1.0, 128, 128, "smooth"),    # keys pooled inside the launch
         (1, 1024, 1024, 4, 128, 1.0, 0, 0, "smooth"),       # pooling kernel + small-launch kernel
         (1, 4096, 4096, 4, 128, 1.0, 64, 128, "smooth"),    # split query sinks, one-block kernel
         (2, 4096, 4096, 16, 128, 0.5, 64, 0, "random"),     # two-block workgroups, moments fold
         (1, 300, 40, 2, 64, 1.0, 0, 0, "random"),           # fewer keys than a block: block tiles
         (2, 700, 1000, 3, 128, math.inf, 64, 64, "random"),  # beta = +inf: no moments
         (1, 2000, 1500, 2, 64, 1.0, 0, 64, "strided"),     # head-strided K / V views, moments folded
         (1, 1024, 2000, 4, 128, 1.0, 64, 0, "random"),     # small-launch kernel folding 2 chunks
         (1, 512, 16000, 2, 64, 0.5, 0, 64, "random"),      # 250 key blocks: 15 whole chunks + a partial
         (1, 4096, 1000, 8, 64, 1.0, 64, 64, "random"),     # centroid tiles only, moments from tile 0 (D 64)
         (2, 4096, 900, 8, 128, 0.0, 0, 128, "smooth")]     # the same in two-block workgroups (D 128)


def _inputs(case):
    b, tq, tk, h, d, _, _, _, kind = case
    if kind == "smooth":
        return tuple(block_smooth(b, t, h, d, seed, device="cuda") for t, seed in ((tq, 1), (tk, 2), (tk, 3)))
    if kind == "strided":
        q = block_smooth(b, tq, h, d, 4, device="cuda")
        k = block_smooth(b, tk, 2 * h, d, 5, device="cuda")[:, :, ::2]
        v = block_smooth(b, tk, 2 * h, d, 6, device="cuda")[:, :, 1::2]
        return q, k, v
    return tensors(nq=tq, nk=tk, d=d, b=b, h=h, device="cuda", seed=7)


@pytest.mark.gpu
@gpu
@pytest.mark.parametrize("case", range(len(CASES)))
def test_all_in_equals_the_two_calls(case, monkeypatch):
    c = CASES[case]
    q, k, v = _inputs(c)
    kw = dict(beta=c[5], kv_sink_tokens=c[6], query_sink_tokens=c[7], return_stats=True)
    print(f"all-in case {case}: B{c[0]} Tq{c[1]} Tk{c[2]} H{c[3]} D{c[4]} beta {c[5]}", flush=True)
    one, one_stats = sol_attention(q, k, v, **kw)
    two, two_stats = _two_calls(q, k, v, kw, monkeypatch)
    assert torch.equal(one, two)
    assert torch.equal(one_stats.exact_blocks, two_stats.exact_blocks)
    again = sol_attention(q, k, v, beta=c[5], kv_sink_tokens=c[6], query_sink_tokens=c[7])
    assert torch.equal(one, again)


@pytest.mark.gpu
@gpu
def test_all_in_against_the_oracle():
    # check_routing runs the debug launch (two calls, decisions written out)
    # and the oracle under its routing; the all-in call must match both.
    from test_kernels import check_routing
    q, k, v = _inputs(CASES[1])
    print("all-in case 1 against the oracle", flush=True)
    debug_out, ref, _ = check_routing(q, k, v, 1.0, local=1, kv_sink=0, q_sink=0, label="all-in")
    one = to_np(sol_attention(q, k, v, beta=1.0).cpu())
    assert (one == debug_out).all()
    assert_close(one, ref)
