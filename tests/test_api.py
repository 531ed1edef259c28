"""CPU tests of the host contract: validation, plan builder, C-ABI exports."""

import ctypes
import math
import os
import re

import numpy as np
import pytest
import torch

from sol_attn_amd import IndexedPlan, SolStats, dense_attention, sol_attention, sol_attention_indexed
from sol_attn_amd import _native
from sol_testlib import tensors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sol_attn_amd.h")


def test_api_rejects_unsupported_input():
    # test_attention.py:149-156 (dtype and grad checks precede the device check)
    q, k, v = tensors()
    with pytest.raises(ValueError, match="AMD ROCm GPU"):
        sol_attention(q, k, v)
    with pytest.raises(ValueError, match="Only BF16"):
        sol_attention(q.float(), k.float(), v.float())
    with pytest.raises(ValueError, match="Inference only"):
        sol_attention(q.requires_grad_(), k, v)


@pytest.mark.parametrize("bad,match", [
    (lambda q, k, v: (q[0], k, v), "BTHD rank-4"),
    (lambda q, k, v: (q, k[:, :, :1], v), "must agree and be nonempty"),
    (lambda q, k, v: (q[..., :32], k[..., :32], v[..., :32]), "head dimensions 64 and 128"),
    (lambda q, k, v: (q.transpose(2, 3), k, v), None),
])
def test_api_validation_messages(bad, match):
    q, k, v = tensors()
    args = bad(q, k, v)
    with pytest.raises(ValueError, match=match):
        sol_attention(*args)
    with pytest.raises(ValueError, match=match):
        dense_attention(*args)


def test_api_keyword_only_and_no_masks():
    q, k, v = tensors()
    with pytest.raises(TypeError):
        sol_attention(q, k, v, 1.0)
    with pytest.raises(TypeError):
        sol_attention(q, k, v, attn_mask=None)
    with pytest.raises(TypeError):
        sol_attention_indexed(q[0], k[0], v[0], None, 1.0)


@pytest.mark.parametrize("kind", ["unsorted", "duplicate", "negative", "outside", "dtype", "batch"])
def test_indexed_rejects_invalid_metadata(kind):
    # test_indexed.py:45-56
    rows = torch.tensor([[1, 2]], dtype=torch.int64)
    keys = torch.arange(8).reshape(1, -1)
    if kind == "unsorted": keys = keys.flip(1)
    if kind == "duplicate": keys[0, 1] = 0
    if kind == "negative": rows[0, 0] = -1
    if kind == "outside": keys[0, -1] = 20
    if kind == "dtype": keys = keys.int()
    if kind == "batch": rows = rows.repeat(2, 1)
    with pytest.raises(ValueError):
        IndexedPlan.create(rows, keys, 20)


def test_indexed_protection_uses_original_indices():
    # test_indexed.py:20-29
    rows = torch.stack((torch.arange(87, 152), torch.arange(300, 365)))
    keys = torch.stack((torch.cat((torch.arange(0, 23), torch.arange(70, 198), torch.arange(500, 509))),
                        torch.cat((torch.arange(0, 23), torch.arange(283, 411), torch.arange(500, 509)))))
    p = IndexedPlan.create(rows, keys, 509, protected_ranges=((0, 23), (500, 509)), local_tokens=0)
    assert p.protected_blocks.shape == (2, 2, 3)
    assert p.protected_blocks.all()
    p = IndexedPlan.create(torch.tensor([[400]], dtype=torch.int64), torch.arange(128).reshape(1, -1),
                           509, local_tokens=0)
    assert not p.protected_blocks.any()


def test_indexed_plan_matches_oracle_on_random_windows():
    from oracle.sol_oracle import plan_protection
    rng = np.random.default_rng(12)
    for trial in range(20):
        w, seq = int(rng.integers(1, 4)), int(rng.integers(200, 3000))
        nq, nk = int(rng.integers(1, min(seq, 300))), int(rng.integers(1, min(seq, 400)))
        rows = np.stack([np.sort(rng.choice(seq, nq, replace=False)) for _ in range(w)])
        keys = np.stack([np.sort(rng.choice(seq, nk, replace=False)) for _ in range(w)])
        a = int(rng.integers(0, seq - 1))
        ranges = ((a, int(rng.integers(a + 1, seq + 1))),)
        local = int(rng.integers(0, 100))
        p = IndexedPlan.create(torch.from_numpy(rows), torch.from_numpy(keys), seq,
                               protected_ranges=ranges, local_tokens=local)
        np.testing.assert_array_equal(p.protected_blocks.numpy(),
                                      plan_protection(rows, keys, seq, ranges, local))


def test_indexed_api_rejects_cpu_inputs():
    p = IndexedPlan.create(torch.tensor([[1, 2]]), torch.arange(8).reshape(1, -1), 20)
    x = torch.randn((20, 2, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="AMD ROCm GPU"):
        sol_attention_indexed(x, x, x, p)
    with pytest.raises(ValueError, match="matching NHD"):
        sol_attention_indexed(x, x[:10], x, p)


def test_plan_records_whether_windows_share_rows():
    keys = torch.arange(100).reshape(1, -1).expand(2, -1).contiguous()
    apart = IndexedPlan.create(torch.tensor([[1, 2], [3, 4]]), keys, 200)
    shared = IndexedPlan.create(torch.tensor([[1, 2], [2, 4]]), keys, 200)
    assert apart.rows_distinct is True and apart.to("cpu").rows_distinct is True
    assert shared.rows_distinct is False and shared.to("cpu").rows_distinct is False
    direct = IndexedPlan(apart.rows, apart.keys, apart.protected_blocks, 200)
    assert direct.rows_distinct is None  # checked on first use with out=


def test_key_length_cap_is_a_value_error():
    from sol_attn_amd import attention
    attention._key_length(attention.MAX_KEY_TOKENS)
    with pytest.raises(ValueError, match="Key sequences longer than 33554432 tokens"):
        attention._key_length(attention.MAX_KEY_TOKENS + 1)


def test_stats_density():
    s = SolStats(torch.tensor([[[2, 4]]], dtype=torch.int32), 4)
    assert s.density() == 0.75


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int64_t|int|const char\*)\s+(sol_\w+)\(", text, re.M)))


def test_c_abi_library_exports_every_declared_symbol():
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("libsol_attn_amd.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_native.LIB_PATH)
    names = _declared_functions()
    assert set(names) >= {"sol_abi_version", "sol_last_error", "sol_pool_kv", "sol_attention_fwd",
                          "sol_dense_fwd", "sol_pool_sizes"}
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_native._SIGNATURES)
    native = _native.library()
    assert native.sol_abi_version() == _native.ABI_VERSION == 14
    sizes = (ctypes.c_int64 * 4)()
    assert native.sol_pool_sizes(1, 317, 2, 64, sizes) == 0
    tile = 2 * 64 * 64 * 2
    assert list(sizes) == [1 * 2 * 1 * tile, 1 * 2 * 5 * tile, 1 * 2 * 1 * 2 * 64 * 4, 2 * 64 * 4]
    assert native.sol_pool_sizes(1, 317, 2, 96, sizes) == -1
    assert b"invalid shape" in native.sol_last_error()
    # Pairing workspace: [B, H, D, NQB + 256] fp32; none below 4 query blocks.
    assert native.sol_pair_workspace_size(1, 193, 2, 64) == 2 * 64 * (4 + 256) * 4
    assert native.sol_pair_workspace_size(1, 192, 2, 64) == 0
    assert native.sol_pair_workspace_size(1, 193, 2, 96) == 0


def test_c_abi_rejects_bad_arguments_without_launching():
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("libsol_attn_amd.so not built")
    native = _native.library()
    strides = (ctypes.c_int64 * 3)(64 * 2 * 317, 128, 64)
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced: validation fails first
    rc = native.sol_dense_fwd(fake, strides, None, 0, fake, strides, fake, strides, 1, 193, 317, 2, 64,
                              float("nan"), fake, fake, None, None)
    assert rc == -1 and b"scale" in native.sol_last_error()
    # A query or output index needs the sequence length it addresses.
    for qi, oi in ((fake, None), (None, fake)):
        rc = native.sol_dense_fwd(fake, strides, qi, 0, fake, strides, fake, strides, 1, 193, 317, 2, 64,
                                  0.125, fake, fake, oi, None)
        assert rc == -1 and b"sequence_length" in native.sol_last_error()
    attn = lambda index, n, form: native.sol_attention_fwd(  # noqa: E731
        fake, strides, index, n, 1, 193, 317, None, 2, 64, None, None, None, None, fake, fake, fake, fake,
        None, None, None, None, None, None, 0.125, 1.0, 1, 0, 0, fake, None, None, None, None, None, None, None, form, None)
    rc = native.sol_attention_fwd(fake, strides, None, 0, 1, 193, 317, None, 2, 64, None, None, None, None,
                                  fake, fake, None, None, None, None, None, None, None, None, 0.125, 1.0, 1, 0, 0, fake,
                                  None, None, None, None, None, None, None, 0, None)
    assert rc == -1 and b"key_mean" in native.sol_last_error()
    rc = native.sol_attention_fwd(fake, strides, None, 0, 1, 193, 317, None, 2, 64, None, None, None, None,
                                  fake, fake, fake, fake, None, None, None, None, None, fake, 0.125, 1.0, 1, 0, 0,
                                  fake, None, None, None, None, None, None, None, 0, None)
    assert rc == -1 and b"query_means" in native.sol_last_error()
    assert native.sol_route_workspace_size(1, 193, 317, 2, float("-inf")) == 0
    # Decision words [B, H, NQB, ceil(NKB / 32)], then, 256-byte aligned, the
    # int32 tile order [B, H, NQB].
    mask_bytes = 2 * 3 * 4 * 1 * 4
    assert native.sol_route_workspace_size(2, 193, 317, 3, 1.0) == -(-mask_bytes // 256) * 256 + 2 * 3 * 4 * 4
    assert native.sol_route_workspace_size(1, 64 * 100, 64 * 70, 2, 0.5) == \
        -(-(1 * 2 * 100 * 3 * 4) // 256) * 256 + 1 * 2 * 100 * 4
    assert attn(None, 0, 3) == -1 and b"workgroup_form" in native.sol_last_error()
    assert attn(fake, 0, 0) == -1 and b"sequence_length" in native.sol_last_error()
    # Without tiles the keys must qualify for rows mode.
    rows = lambda nk, lengths: native.sol_attention_fwd(  # noqa: E731
        fake, strides, None, 0, 1, 193, nk, lengths, 2, 64, fake, strides, fake, strides, None, fake,
        fake, fake, None, None, None, None, None, None, 0.125, 1.0, 1, 0, 0, fake, None, None, None, None, None, None, None,
        0, None)
    assert rows(63, None) == -1 and b"without tiles" in native.sol_last_error()
    assert rows(317, fake) == -1 and b"without tiles" in native.sol_last_error()
    rc = native.sol_quantize_keys(fake, strides, None, None, 0, 1, 40, 2, 64, 1, fake, fake, None)
    assert rc == -1 and b"rows_mode" in native.sol_last_error()
    rc = native.sol_pair_strides(fake, strides, None, 0, 1, 192, 2, 64, fake, fake, None, None)
    assert rc == -2 and b"4 .. 8192 query blocks" in native.sol_last_error()
    rc = native.sol_pair_strides(fake, strides, None, 0, 1, 193, 2, 64, None, fake, None, None)
    assert rc == -1 and b"workspace" in native.sol_last_error()
    rc = native.sol_pair_strides(fake, strides, fake, 0, 1, 193, 2, 64, fake, fake, None, None)
    assert rc == -1 and b"sequence_length" in native.sol_last_error()
    bad = (ctypes.c_int64 * 3)(64 * 2 * 317, 127, 64)
    rc = native.sol_pool_kv(fake, bad, fake, strides, None, None, 0, 1, 317, 2, 64, fake, fake,
                            None, None, None, None)
    assert rc == -1 and b"aligned" in native.sol_last_error()
    rc = native.sol_pool_kv(fake, strides, fake, strides, None, None, 0, 1, 317, 2, 64, None, None,
                            None, None, None, None)
    assert rc == -1 and b"nothing to write" in native.sol_last_error()
    rc = native.sol_pool_kv(fake, strides, fake, strides, fake, None, 0, 1, 317, 2, 64, fake, fake,
                            None, None, None, None)
    assert rc == -1 and b"sequence_length" in native.sol_last_error()
    assert native.sol_key_covariance_workspace_size(2, 3, 64) == 2 * 3 * 16 * 64 * 64 * 4
    assert native.sol_key_covariance_workspace_size(2, 3, 96) == 0
    rc = native.sol_key_covariance(fake, fake, None, 1, 317, 2, 96, fake, fake, None)
    assert rc == -1 and b"invalid shape" in native.sol_last_error()
    rc = native.sol_key_covariance(fake, None, None, 1, 317, 2, 64, fake, fake, None)
    assert rc == -1 and b"required" in native.sol_last_error()
    rc = native.sol_plan_protection(fake, fake, None, 2, 0, 300, 64, None, 0, fake, None)
    assert rc == -1 and b"invalid shape" in native.sol_last_error()
    rc = native.sol_plan_protection(fake, fake, None, 2, 100, 300, -1, None, 0, fake, None)
    assert rc == -1 and b"invalid shape" in native.sol_last_error()
    rc = native.sol_plan_protection(fake, fake, None, 2, 100, 300, 64, None, 1, fake, None)
    assert rc == -1 and b"required" in native.sol_last_error()
    rc = native.sol_plan_protection(fake, None, None, 2, 100, 300, 64, None, 0, fake, None)
    assert rc == -1 and b"required" in native.sol_last_error()


def test_split_workspace_only_where_sinks_set_the_launch_end():
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("libsol_attn_amd.so not built")
    size = _native.library().sol_split_workspace_size
    # 4,096 tokens x 4 heads, D 128, two sink blocks: 4 parts of 16 key
    # blocks; rows of 128 + 4 floats for sink blocks 0, 1 of 4 (entry, head) pairs.
    assert size(1, 4096, 4096, 4, 128, 1.0, 128) == 4 * 2 * 64 * 4 * 132 * 4
    assert size(1, 8192, 8192, 4, 64, 1.0, 192) == 4 * 2 * 64 * 8 * 68 * 4  # 8 parts; block 2 whole
    # 2 x 4,096 x 16 heads (1,024 query-block pairs): split at beta = +inf only.
    assert size(2, 4096, 4096, 16, 128, math.inf, 128) == 32 * 2 * 64 * 4 * 132 * 4
    assert size(2, 4096, 4096, 16, 128, 1.0, 128) == 0
    assert size(1, 4096, 4096, 4, 128, -math.inf, 128) == 0   # every block exact
    assert size(1, 4096, 4096, 4, 128, 1.0, 64) == 0          # one sink block
    assert size(1, 4096, 4096, 4, 128, 1.0, 0) == 0           # no sinks
    assert size(1, 1024, 1024, 8, 64, 1.0, 128) == 0          # 16 key blocks (small-launch kernel)
    assert size(1, 84672, 84672, 24, 128, 1.0, 128) == 0      # many rounds of workgroups
    assert size(1, 4096, 4096, 4, 128, 1.0, 1100) == 0        # sinks over a quarter of the blocks
    assert size(1, 4096, 600000, 1, 128, 1.0, 128) == 0       # more than one routing segment


def test_self_pooling_sizes_and_null_centroid_tiles():
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("libsol_attn_amd.so not built")
    native = _native.library()
    pools = native.sol_attention_pools_keys
    assert pools(1, 1024, 1024, 8, 64) == 1
    assert pools(1, 1024, 1024, 8, 128) == 0       # head_dim 128: the pooling kernel first
    assert pools(1, 1024, 1025, 8, 64) == 0        # 17 key blocks: more than one pooling chunk
    assert pools(1, 1024, 40, 8, 64) == 0          # fewer than 64 keys: pooled block tiles
    assert pools(1, 4096, 1024, 16, 64) == 0       # 1,024 query blocks: not a small launch
    assert pools(1, 1024, 1024, 8, 96) == 0        # unsupported head_dim
    # NULL centroid tiles where the launch cannot pool its keys itself.
    strides = (ctypes.c_int64 * 3)(64 * 8 * 4096, 64 * 8, 64)
    fake = ctypes.c_void_p(1 << 20)
    rc = native.sol_attention_fwd(fake, strides, None, 0, 1, 4096, 4096, None, 8, 64, fake, strides, fake, strides,
                                  None, None, None, None, None, None, None, None, None, None, 0.125, 1.0, 1, 0, 0,
                                  fake, None, None, None, None, None, None, None, 0, None)
    assert rc == -1 and b"sol_attention_pools_keys" in native.sol_last_error()


def test_noalloc_rejects_problems_beyond_its_workspace_without_launching():
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("libsol_attn_amd.so not built")
    native = _native.library()
    tk = 64 * 8192
    strides = (ctypes.c_int64 * 3)(64 * 128 * tk, 64 * 128, 128)
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced: the size check fails first
    # 524,288 keys x 64 heads at D = 128: 256 MiB of centroid tiles.
    rc = native.sol_attention_noalloc(fake, strides, fake, strides, fake, strides, 1, 200, tk, 64, 128,
                                      0.088, 1.0, 1, 0, 0, fake, None, None)
    assert rc == -2 and b"SOL_NOALLOC_SCRATCH_BYTES" in native.sol_last_error()
    rc = native.sol_attention_noalloc(fake, strides, fake, strides, fake, strides, 1, 200, 200, 16, 96,
                                      0.088, 1.0, 1, 0, 0, fake, None, None)
    assert rc == -1 and b"head_dim" in native.sol_last_error()
    # Arguments the attention launch would reject are rejected before the
    # pooling launch (nothing runs, no device is touched).
    small = (ctypes.c_int64 * 3)(64 * 128 * 200, 64 * 128, 128)
    for args, what in (((-0.1, 1.0, 1, 0, 0, fake), b"scale"),
                       ((0.088, math.nan, 1, 0, 0, fake), b"beta"),
                       ((0.088, 1.0, 1, -1, 0, fake), b"sink"),
                       ((0.088, 1.0, 1, 0, 0, ctypes.c_void_p((1 << 20) + 2)), b"out")):
        rc = native.sol_attention_noalloc(fake, small, fake, small, fake, small, 1, 200, 200, 64, 128,
                                          *args, None, None)
        msg = native.sol_last_error()
        assert rc == -1 and msg.startswith(b"sol_attention_noalloc") and what in msg, msg


def test_ragged_plan_matches_oracle_per_window():
    from oracle.sol_oracle import plan_protection
    rng = np.random.default_rng(21)
    for trial in range(12):
        w, seq = int(rng.integers(2, 5)), int(rng.integers(400, 3000))
        nq = int(rng.integers(1, 200))
        rows = np.stack([np.sort(rng.choice(seq, nq, replace=False)) for _ in range(w)])
        keys = [np.sort(rng.choice(seq, int(rng.integers(1, 400)), replace=False)) for _ in range(w)]
        a = int(rng.integers(0, seq - 1))
        ranges = ((a, int(rng.integers(a + 1, seq + 1))),)
        local = int(rng.integers(0, 100))
        p = IndexedPlan.create(torch.from_numpy(rows), [torch.from_numpy(x) for x in keys], seq,
                               protected_ranges=ranges, local_tokens=local)
        nk = max(len(x) for x in keys)
        assert p.keys.shape == (w, nk) and p.key_lengths.tolist() == [len(x) for x in keys]
        assert p.protected_blocks.shape == (w, -(-nq // 64), -(-nk // 64))
        for i, x in enumerate(keys):
            nkb = -(-len(x) // 64)
            np.testing.assert_array_equal(p.keys[i, :len(x)].numpy(), x)
            expect = plan_protection(rows[i:i + 1], x[None], seq, ranges, local)[0]
            np.testing.assert_array_equal(p.protected_blocks[i, :, :nkb].numpy(), expect)
            assert not p.protected_blocks[i, :, nkb:].any()
        # An equal-length plan built from the same window agrees.
        q = IndexedPlan.create(torch.from_numpy(rows[:1]), torch.from_numpy(keys[0][None]), seq,
                               protected_ranges=ranges, local_tokens=local)
        assert q.key_lengths is None
        np.testing.assert_array_equal(q.protected_blocks[0].numpy(),
                                      p.protected_blocks[0, :, :q.protected_blocks.shape[2]].numpy())


@pytest.mark.parametrize("kind", ["empty", "unsorted", "outside", "count", "matrix", "dtype"])
def test_ragged_plan_rejects_invalid_keys(kind):
    rows = torch.tensor([[1, 2], [5, 6]], dtype=torch.int64)
    keys = [torch.arange(8), torch.arange(3, 12)]
    if kind == "empty": keys[1] = keys[1][:0]
    if kind == "unsorted": keys[0] = keys[0].flip(0)
    if kind == "outside": keys[1] = torch.arange(15, 25)
    if kind == "count": keys = keys[:1]
    if kind == "matrix": keys[0] = keys[0].reshape(2, 4)
    if kind == "dtype": keys[1] = keys[1].int()
    with pytest.raises(ValueError):
        IndexedPlan.create(rows, keys, 20)


def test_stats_density_ragged_windows():
    exact = torch.tensor([[[2], [4]], [[1], [1]]], dtype=torch.int32)
    assert SolStats(exact, torch.tensor([4, 2])).density() == pytest.approx((0.5 + 1 + 0.5 + 0.5) / 4)


def test_frame_window_plan_protection_floor():
    # 21 frame windows of 4,032 (= 63 x 64) queries, keys = frames
    # {0, f-1, f, f+1}, frame 0 protected, local 64.  Frame 0 fills key blocks
    # 0..62 of every window: 63 x 63 = 3969 protected (q-block, key-block)
    # pairs.  The local band of q-block qb touches token blocks qb-1, qb, qb+1
    # of frame f (block -1 / 63 = the neighbouring frame's edge block):
    #   f = 0:  keys are frames {0, 1}; only q-block 62 reaches past frame 0
    #           (block 63, frame 1's first)                       -> 3969 + 1
    #   f = 1:  keys {0, 1, 2}; q-block 0 adds 2 (block 62 is frame 0),
    #           q-blocks 1..62 add 3 each                         -> 3969 + 188
    #   f = 20: keys {0, 19, 20}; q-block 62 adds 2 (no frame 21),
    #           q-blocks 0..61 add 3 each                         -> 3969 + 188
    #   f = 2..19: 3 each for all 63 q-blocks                     -> 3969 + 189
    tpf = 4032
    rows = torch.stack([torch.arange(f * tpf, (f + 1) * tpf) for f in range(21)])
    keys = [torch.cat([torch.arange(x * tpf, (x + 1) * tpf)
                       for x in sorted({0, f - 1, f, f + 1} & set(range(21)))]) for f in range(21)]
    p = IndexedPlan.create(rows, keys, 21 * tpf, protected_ranges=((0, tpf),), local_tokens=64)
    assert sorted(set(p.key_lengths.tolist())) == [8064, 12096, 16128]
    for f, expect in ((0, 3970), (1, 4157), (10, 4158), (19, 4158), (20, 4157)):
        nkb = -(-len(keys[f]) // 64)
        assert int(p.protected_blocks[f, :, :nkb].sum()) == expect
        assert not p.protected_blocks[f, :, nkb:].any()


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits with a message before any GPU work."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 2
    assert "one GPU only" in res.stderr
