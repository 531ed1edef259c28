"""Query-block pairing (sol_pair_strides): a schedule choice that never changes results.

No counterpart in the reference (one Triton program per query block).  The
checks: outputs and exact-block counts are bit-identical with and without
pairing and for forced strides; the chosen stride recovers the frame period of
a frame-structured sequence; and it maximises the pairing score restated here
in numpy from the query-block means.
"""

import math

import numpy as np
import pytest
import torch

from sol_attn_amd import IndexedPlan, _native, sol_attention, sol_attention_indexed
from sol_testlib import HAS_GPU

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


def frames(n_frames, blocks_per_frame, heads=2, d=128, seed=0, noise=0.1):
    """[1, T, H, D] BF16 laid out frame by frame: block i of frame f is a
    per-position pattern that drifts slowly with f, plus per-block noise, so
    block i is most alike block i + blocks_per_frame (one frame later)."""
    g = torch.Generator().manual_seed(seed)
    pos = torch.randn((1, blocks_per_frame, heads, d), generator=g)
    drift = torch.randn((1, blocks_per_frame, heads, d), generator=g)
    f = torch.arange(n_frames, dtype=torch.float32).view(-1, 1, 1, 1)
    x = (pos + 0.15 * f * drift).reshape(-1, heads, d)
    x = x + noise * torch.randn(x.shape, generator=g)
    x = x.repeat_interleave(64, 0) + 0.05 * torch.randn((x.shape[0] * 64, heads, d), generator=g)
    return x[None].to(torch.bfloat16)


def pairing_scores(q):
    """numpy restatement of pair_pick_kernel's score per stride 1..256 for [T, H, D] rows."""
    x = q.float().numpy()
    t, h, d = x.shape
    n = -(-t // 64)
    m = np.stack([x[64 * i:64 * (i + 1)].mean(0) for i in range(n)])          # [n, H, D]
    m = m / np.maximum(np.linalg.norm(m, axis=-1, keepdims=True), 1e-30)
    scores = np.full((h, 256), -2.0)
    c = np.zeros((h, 257))
    for s in range(1, 257):
        if s < n:
            c[:, s] = (m[:-s] * m[s:]).sum(-1).sum(0) / (n - s)
    for s in range(1, 257):
        covered = (n // (2 * s)) * (2 * s)
        if covered > 0:
            scores[:, s - 1] = (covered * c[:, s] + (n - covered) * c[:, 1]) / n
    return scores


def test_chosen_stride_is_the_frame_period():
    q = frames(12, 7).cuda()
    strides = _native.pair_strides(q, min_blocks=4)
    assert strides.shape == (1, 2) and strides.dtype == torch.int32
    assert strides.cpu().tolist() == [[7, 7]]


@pytest.mark.parametrize("seed", [1, 2])
def test_chosen_stride_maximises_the_score(seed):
    q = frames(9, 11, heads=3, d=64, seed=seed, noise=1.5)
    got = _native.pair_strides(q.cuda(), min_blocks=4).cpu().numpy()[0]
    scores = pairing_scores(q[0])
    for h in range(3):
        assert scores[h, got[h] - 1] >= scores[h].max() - 1e-5, (h, got[h], scores[h].argmax() + 1)


def test_no_pairing_below_four_query_blocks():
    assert _native.pair_strides(frames(1, 3).cuda(), min_blocks=1) is None
    assert _native.pair_strides(frames(12, 7).cuda()) is None  # below the default minimum


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("beta", [1.0, -math.inf, 0.0])
def test_pairing_never_changes_results(beta, d, monkeypatch):
    monkeypatch.setattr(_native, "PAIR_MIN_QUERY_BLOCKS", 4)  # pair these 72 query blocks
    monkeypatch.setattr(_native, "WORKGROUP_FORM", 2)  # two-block workgroups (this launch is small)
    q, k, v = (frames(8, 9, d=d, seed=s).cuda() for s in (3, 4, 5))
    ref, ref_stats = sol_attention(q, k, v, beta=beta, kv_sink_tokens=64, return_stats=True)
    monkeypatch.setattr(_native, "PAIRING", False)
    plain, plain_stats = sol_attention(q, k, v, beta=beta, kv_sink_tokens=64, return_stats=True)
    assert torch.equal(ref, plain)
    assert torch.equal(ref_stats.exact_blocks, plain_stats.exact_blocks)
    # Forced strides (including ones past the query blocks) are valid pairings too.
    pooled = _native.pool_kv(k, v, moments=not math.isinf(beta))
    for s in (1, 2, 5, 9, 40, 1 << 30):
        monkeypatch.setattr(_native, "_pairing", lambda q, rows=None, stream=None, s=s: (torch.full(
            (1, 2), s, device=q.device, dtype=torch.int32), None))
        monkeypatch.setattr(_native, "PAIRING", True)
        out, counts, _ = _native.attend(q, pooled, d ** -0.5, beta, 1, 64, 0)
        assert torch.equal(out, ref), s
        assert torch.equal(counts, ref_stats.exact_blocks), s


def test_pairing_on_the_side_stream_matches_the_caller_stream(monkeypatch):
    """The pairing kernels run on a second stream of the device, concurrently
    with pooling, and join the caller's stream before attention
    (OVERLAP_PAIRING).  Run on the caller's stream instead, or called from a
    non-default caller stream, the results are bit-identical."""
    monkeypatch.setattr(_native, "PAIR_MIN_QUERY_BLOCKS", 4)
    monkeypatch.setattr(_native, "WORKGROUP_FORM", 2)
    q, k, v = (frames(8, 9, seed=s).cuda() for s in (3, 4, 5))
    x = [frames(10, 6, seed=s)[0].cuda() for s in (6, 7, 8)]
    t = x[0].shape[0]
    rows = torch.stack((torch.arange(0, t // 2), torch.arange(t // 2, t)))
    keys = [torch.arange(0, t - 64), torch.arange(64, t - 128)]
    plan = IndexedPlan.create(rows, keys, t, protected_ranges=((0, 64),), local_tokens=64).to("cuda")
    assert _native.pair_strides(q) is not None and _native.pair_strides(x[0], plan.rows) is not None

    def run():
        out, stats = sol_attention(q, k, v, beta=1.0, kv_sink_tokens=64, return_stats=True)
        win, win_stats = sol_attention_indexed(*x, plan, beta=1.0, return_stats=True)
        return out, stats.exact_blocks, win, win_stats.exact_blocks

    ref = run()
    monkeypatch.setattr(_native, "OVERLAP_PAIRING", False)
    serial = run()
    monkeypatch.setattr(_native, "OVERLAP_PAIRING", True)
    caller = torch.cuda.Stream()
    caller.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(caller):
        on_caller = run()
    torch.cuda.current_stream().wait_stream(caller)
    torch.cuda.synchronize()
    for a, b, c in zip(ref, serial, on_caller):
        assert torch.equal(a, b) and torch.equal(a, c)


def test_indexed_windows_pair_per_window(monkeypatch):
    monkeypatch.setattr(_native, "PAIR_MIN_QUERY_BLOCKS", 4)
    monkeypatch.setattr(_native, "WORKGROUP_FORM", 2)  # two-block workgroups (this launch is small)
    x = [frames(10, 6, seed=s)[0].cuda() for s in (6, 7, 8)]      # [T, H, D] NHD
    t = x[0].shape[0]
    rows = torch.stack((torch.arange(0, t // 2), torch.arange(t // 2, t)))
    keys = torch.stack((torch.arange(0, t - 64), torch.arange(64, t)))
    plan = IndexedPlan.create(rows, keys, t, protected_ranges=((0, 64),), local_tokens=64).to("cuda")
    strides = _native.pair_strides(x[0], plan.rows, min_blocks=4)
    assert strides.shape == (2, 2)
    ref = sol_attention_indexed(*x, plan, beta=1.0)
    monkeypatch.setattr(_native, "PAIRING", False)
    assert torch.equal(ref, sol_attention_indexed(*x, plan, beta=1.0))


@pytest.mark.parametrize("shape", [(1, 4096, 4, 128), (2, 1000, 3, 64), (1, 20000, 2, 128)])
def test_one_and_two_block_workgroups_are_identical(shape, monkeypatch):
    """Small launches run one query block per workgroup; both forms must give
    bit-identical outputs and counts (a wave's tiles and their order do not
    depend on its partner block)."""
    b, t, h, d = shape
    q, k, v = (frames(-(-t // 576), 9, heads=h, d=d, seed=s)[:, :t].repeat(b, 1, 1, 1).cuda() for s in (12, 13, 14))
    res = {}
    for g in ("1", "2"):
        monkeypatch.setattr(_native, "WORKGROUP_FORM", int(g))
        res[g] = sol_attention(q, k, v, beta=1.0, kv_sink_tokens=64, return_stats=True)
    assert torch.equal(res["1"][0], res["2"][0])
    assert torch.equal(res["1"][1].exact_blocks, res["2"][1].exact_blocks)
