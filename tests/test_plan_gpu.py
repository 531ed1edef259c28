"""Indexed plans built on the GPU (sol_plan_protection) against the CPU builder and the oracle.

The CPU builder is itself pinned to the oracle's restatement of
`indexed.py:27-62` (test_api.py) and to the reference's known answers; here
the GPU kernel must reproduce it bit for bit on random equal-length and
ragged windows, on the frame-window plan, and in attention results.
"""

import numpy as np
import pytest
import torch

from oracle.sol_oracle import plan_protection
from sol_attn_amd import IndexedPlan, sol_attention_indexed
from sol_testlib import HAS_GPU

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


def random_windows(rng, ragged):
    w, seq = int(rng.integers(1, 5)), int(rng.integers(200, 3000))
    nq = int(rng.integers(1, min(seq, 300)))
    rows = np.stack([np.sort(rng.choice(seq, nq, replace=False)) for _ in range(w)])
    if ragged:
        keys = [np.sort(rng.choice(seq, int(rng.integers(1, min(seq, 400))), replace=False)) for _ in range(w)]
    else:
        nk = int(rng.integers(1, min(seq, 400)))
        keys = np.stack([np.sort(rng.choice(seq, nk, replace=False)) for _ in range(w)])
    ranges = []
    for _ in range(int(rng.integers(0, 3))):
        a = int(rng.integers(0, seq - 1))
        ranges.append((a, int(rng.integers(a + 1, seq + 1))))
    return rows, keys, seq, tuple(ranges), int(rng.integers(0, 100))


@pytest.mark.parametrize("ragged", [False, True])
def test_gpu_plan_equals_cpu_plan_and_oracle(ragged):
    rng = np.random.default_rng(31 + ragged)
    for _ in range(25):
        rows, keys, seq, ranges, local = random_windows(rng, ragged)
        cpu_keys = [torch.from_numpy(x) for x in keys] if ragged else torch.from_numpy(keys)
        gpu_keys = [x.cuda() for x in cpu_keys] if ragged else cpu_keys.cuda()
        cpu = IndexedPlan.create(torch.from_numpy(rows), cpu_keys, seq, protected_ranges=ranges, local_tokens=local)
        gpu = IndexedPlan.create(torch.from_numpy(rows).cuda(), gpu_keys, seq, protected_ranges=ranges,
                                 local_tokens=local)
        assert gpu.protected_blocks.device.type == "cuda" and gpu.protected_blocks.dtype == torch.bool
        assert torch.equal(gpu.protected_blocks.cpu(), cpu.protected_blocks)
        assert torch.equal(gpu.rows.cpu(), cpu.rows) and torch.equal(gpu.keys.cpu(), cpu.keys)
        if ragged:
            assert torch.equal(gpu.key_lengths.cpu(), cpu.key_lengths)
            for i, x in enumerate(keys):
                nkb = -(-len(x) // 64)
                np.testing.assert_array_equal(gpu.protected_blocks[i, :, :nkb].cpu().numpy(),
                                              plan_protection(rows[i:i + 1], x[None], seq, ranges, local)[0])
        else:
            assert gpu.key_lengths is None
            np.testing.assert_array_equal(gpu.protected_blocks.cpu().numpy(),
                                          plan_protection(rows, keys, seq, ranges, local))


def test_gpu_plan_known_answers():
    # test_indexed.py:20-29 on the device
    rows = torch.stack((torch.arange(87, 152), torch.arange(300, 365))).cuda()
    keys = torch.stack((torch.cat((torch.arange(0, 23), torch.arange(70, 198), torch.arange(500, 509))),
                        torch.cat((torch.arange(0, 23), torch.arange(283, 411), torch.arange(500, 509))))).cuda()
    p = IndexedPlan.create(rows, keys, 509, protected_ranges=((0, 23), (500, 509)), local_tokens=0)
    assert p.protected_blocks.shape == (2, 2, 3) and bool(p.protected_blocks.all())
    p = IndexedPlan.create(torch.tensor([[400]]).cuda(), torch.arange(128).reshape(1, -1).cuda(), 509,
                           local_tokens=0)
    assert not bool(p.protected_blocks.any())


def test_gpu_frame_window_plan():
    tpf = 4032
    rows = torch.stack([torch.arange(f * tpf, (f + 1) * tpf) for f in range(21)])
    keys = [torch.cat([torch.arange(x * tpf, (x + 1) * tpf)
                       for x in sorted({0, f - 1, f, f + 1} & set(range(21)))]) for f in range(21)]
    cpu = IndexedPlan.create(rows, keys, 21 * tpf, protected_ranges=((0, tpf),), local_tokens=64)
    gpu = IndexedPlan.create(rows.cuda(), [x.cuda() for x in keys], 21 * tpf, protected_ranges=((0, tpf),),
                             local_tokens=64)
    assert torch.equal(gpu.protected_blocks.cpu(), cpu.protected_blocks)
    for f, expect in ((0, 3970), (1, 4157), (10, 4158), (20, 4157)):
        assert int(gpu.protected_blocks[f].sum()) == expect


@pytest.mark.parametrize("kind", ["unsorted", "duplicate", "negative", "outside", "dtype", "batch", "mixed"])
def test_gpu_plan_rejects_invalid_metadata(kind):
    rows = torch.tensor([[1, 2]], dtype=torch.int64)
    keys = torch.arange(8).reshape(1, -1)
    if kind == "unsorted": keys = keys.flip(1)
    if kind == "duplicate": keys[0, 1] = 0
    if kind == "negative": rows[0, 0] = -1
    if kind == "outside": keys[0, -1] = 20
    if kind == "dtype": keys = keys.int()
    if kind == "batch": rows = rows.repeat(2, 1)
    rows = rows.cuda()
    keys = keys if kind == "mixed" else keys.cuda()
    with pytest.raises(ValueError):
        IndexedPlan.create(rows, keys, 20)


def test_gpu_plan_gives_identical_attention():
    g = torch.Generator().manual_seed(5)
    x = [torch.randn((1000, 2, 64), generator=g).to(torch.bfloat16).cuda() for _ in range(3)]
    rows = torch.stack((torch.arange(0, 300), torch.arange(500, 800)))
    keys = [torch.cat((torch.arange(0, 100), torch.arange(250, 600))), torch.arange(300, 1000)]
    cpu = IndexedPlan.create(rows, keys, 1000, protected_ranges=((0, 64),), local_tokens=32).to("cuda")
    gpu = IndexedPlan.create(rows.cuda(), [k.cuda() for k in keys], 1000, protected_ranges=((0, 64),),
                             local_tokens=32)
    a = sol_attention_indexed(*x, cpu, beta=0.5)
    b = sol_attention_indexed(*x, gpu, beta=0.5)
    assert torch.equal(a, b)
