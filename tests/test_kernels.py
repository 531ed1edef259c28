"""GPU kernel-level parity: pooling bit-exactness, routing decisions within the
stated band, outputs under identical routing, and the dense limit.

Routing band (stated here and used by every decision check): a kernel decision
may differ from the oracle's only for blocks with
``|proxy - cutoff| <= 1e-5 * max(|cutoff|, scale * |Qc| * |Kc_j|)``
(oracle values, natural-log units); ``|.|`` are Euclidean norms.  The second
term is the magnitude the FP32 proxy dot product is rounded against.
"""

import math

import numpy as np
import pytest
import torch

import bench
from oracle import sol_oracle as orc
from sol_attn_amd import _native, dense_attention, sol_attention
from sol_testlib import HAS_GPU, assert_close, block_smooth, tensors, to_np

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]

BAND = 1e-5


def kernel_pool(k, v, moments=True):
    with torch.no_grad():
        return _native.pool_kv(k, v, moments=moments)


def unswizzle(tiles):
    """Tile pairs ``[B, H, N, 2, 64 D]`` -> K and V rows ``[B, H, N, 64, D]``
    (uint16 BF16 bits), undoing the tile layouts: K chunk c (8 features) of
    row r sits at chunk c ^ (r & 15) (D = 128) or c ^ ((r >> 1) & 7) (D = 64)
    of the row; V chunk c of row r at chunk (r >> 2) 4 CPR + (c >> 2) 16 +
    (r & 3) 4 + (c & 3) of the tile (CPR = D / 8 chunks per row)."""
    t = tiles.cpu().view(torch.int16).numpy().view(np.uint16)
    b, h, n, _, e = t.shape
    d = e // 64
    rows = np.arange(64)[:, None]
    chunks = np.arange(d // 8)[None, :]
    kswz = (rows & 15) if d == 128 else ((rows >> 1) & 7)
    kt = t[:, :, :, 0].reshape(b, h, n, 64, d // 8, 8)
    vt = t[:, :, :, 1].reshape(b, h, n, 64 * d // 8, 8)
    k_rows = kt[:, :, :, rows, chunks ^ kswz].reshape(b, h, n, 64, d)
    vpos = (rows >> 2) * (4 * (d // 8)) + (chunks >> 2) * 16 + (rows & 3) * 4 + (chunks & 3)
    v_rows = vt[:, :, :, vpos].reshape(b, h, n, 64, d)
    return k_rows, v_rows


def check_tiles(tiles, k, v):
    """The attention tiles hold K / V of every key block, zero past the end."""
    kb = k.contiguous().view(torch.int16).numpy().view(np.uint16)
    vb = v.contiguous().view(torch.int16).numpy().view(np.uint16)
    k_rows, v_rows = unswizzle(tiles)
    b, h, nkb, d = k_rows.shape[0], k_rows.shape[1], k_rows.shape[2], k_rows.shape[4]
    pad = nkb * 64 - kb.shape[1]
    kp = np.concatenate([kb, np.zeros((b, pad) + kb.shape[2:], np.uint16)], 1)
    vp = np.concatenate([vb, np.zeros((b, pad) + vb.shape[2:], np.uint16)], 1)
    np.testing.assert_array_equal(k_rows, kp.reshape(b, nkb, 64, h, d).transpose(0, 3, 1, 2, 4))
    np.testing.assert_array_equal(v_rows, vp.reshape(b, nkb, 64, h, d).transpose(0, 3, 1, 2, 4))


def centroids(ctiles, nkb):
    """Centroid tiles -> K and V block centroids ``[B, NKB, H, D]`` float32 (+ padding check)."""
    k_rows, v_rows = unswizzle(ctiles)              # [B, H, NCT, 64, D] each
    b, h, nct, _, d = k_rows.shape
    kc = k_rows.reshape(b, h, nct * 64, d)
    vc = v_rows.reshape(b, h, nct * 64, d)
    assert (kc[:, :, nkb:] == 0).all() and (vc[:, :, nkb:] == 0).all()
    f = lambda x: orc.bf16_bits_to_f32(x[:, :, :nkb]).transpose(0, 2, 1, 3)
    return f(kc), f(vc)


# Grids of up to 512 chunk workgroups (2 B H ceil(NKB / 64) 4) take the wide
# pooling form, larger ones the four-wave form: the last two shapes (ragged
# last block) are the four-wave form's, for D = 64 and 128.  Keys of at most
# 16 blocks (one pooling chunk: 317, 1 and exactly 1,024 tokens) get their
# moments from the pooling kernel itself, longer ones from moments_kernel;
# 40,000 and 17,000 tokens (625 and 266 blocks) take its 256-block groups.
# Large grids at D = 128 with heads in fours take the four-head workgroups:
# 4,033 tokens x 68 heads and 20,000 x 2 x 8 (313 blocks).
@pytest.mark.parametrize("shape", [(1, 317, 2, 64), (2, 1089, 3, 128), (1, 1, 1, 64), (1, 1024, 2, 64),
                                   (2, 4096, 16, 128), (1, 10000, 4, 128), (1, 4100, 72, 64),
                                   (1, 4033, 68, 128), (1, 40000, 2, 64), (2, 17000, 3, 128),
                                   (2, 20000, 8, 128)])
def test_pooling_and_moments_bit_exact(shape):
    b, t, h, d = shape
    g = torch.Generator().manual_seed(t)
    k = torch.randn(shape, generator=g, dtype=torch.bfloat16)
    v = torch.randn(shape, generator=g, dtype=torch.bfloat16)
    out = kernel_pool(k.cuda(), v.cuda())
    torch.cuda.synchronize()
    # Block tiles only where the attention kernels cannot read K / V rows
    # themselves (fewer than 64 keys here).
    assert (out["tiles"] is None) == (t >= 64)
    if out["tiles"] is not None:
        check_tiles(out["tiles"], k, v)
    kc = orc.block_means(to_np(k), True)          # [B, NKB, H, D]
    vc = orc.block_means(to_np(v), True)
    mean, var = orc.key_moments(kc)
    got_kc, got_vc = centroids(out["ctiles"], kc.shape[1])
    np.testing.assert_array_equal(got_kc, kc)
    np.testing.assert_array_equal(got_vc, vc)
    np.testing.assert_array_equal(to_np(out["mean"]), mean)
    np.testing.assert_array_equal(to_np(out["var"]), var)


def test_pooling_strided_and_indexed_gather():
    g = torch.Generator().manual_seed(9)
    base = torch.randn((900, 6, 64), generator=g, dtype=torch.bfloat16)
    keys = torch.stack((torch.arange(3, 503), torch.arange(350, 850)))
    k = base.cuda()[:, ::2]                     # NHD, head stride 128 elements
    v = (base.cuda() * 2)[:, 1::2]
    out = _native.pool_kv(k, v, key_index=keys.cuda())
    check_tiles(out["tiles"], k.cpu()[keys], v.cpu()[keys])
    kc = orc.block_means(to_np(k.cpu()[keys]), True)
    vc = orc.block_means(to_np(v.cpu()[keys]), True)
    got_kc, got_vc = centroids(out["ctiles"], kc.shape[1])
    np.testing.assert_array_equal(got_kc, kc)
    np.testing.assert_array_equal(got_vc, vc)
    mean, var = orc.key_moments(kc)
    np.testing.assert_array_equal(to_np(out["mean"]), mean)
    np.testing.assert_array_equal(to_np(out["var"]), var)


def run_debug(q, k, v, beta, scale=None, local=1, kv_sink=0, q_sink=0, estimator="diagonal_covariance"):
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    with torch.no_grad():
        out, counts, dbg = _native.launch_sol(q, k, v, scale, beta, local, kv_sink, q_sink, True,
                                              debug=True, threshold_estimator=estimator)
    torch.cuda.synchronize()
    return out, counts, dbg


# In-band mismatches allowed per decision (a stated cap on top of the band).
MAX_BAND_MISMATCH_RATE = 1e-4


def check_routing(q, k, v, beta, scale=None, local=1, kv_sink=0, q_sink=0, query_blocks=None,
                  max_band_mismatch=None, estimator="diagonal_covariance", label=""):
    """Decisions vs oracle (band), outputs under identical routing, counts.

    Every mismatch must lie inside the band, and their number may not exceed
    ``max_band_mismatch`` (default: MAX_BAND_MISMATCH_RATE of the decisions);
    the count and the band population are printed.  Returns
    ``(kernel_out, oracle_out_under_kernel_routing, mismatch_mask)``."""
    qn, kn, vn = to_np(q.cpu()), to_np(k.cpu()), to_np(v.cpu())
    d = qn.shape[-1]
    s = d ** -0.5 if scale is None else scale
    out, counts, dbg = run_debug(q, k, v, beta, s, local, kv_sink, q_sink, estimator)
    qm = orc.block_means(qn, False)
    kc = orc.block_means(kn, True)
    mean, var = orc.key_moments(kc)
    if estimator == "full_covariance":
        cut = orc.cutoffs_full(qm, mean, orc.key_covariance(kc), beta, s)
    else:
        cut = orc.cutoffs(qm, mean, var, beta, s)
    sel, proxy = orc.route(qn, kc, cut, beta=beta, scale=s, local_blocks=local,
                           kv_sink_tokens=kv_sink, query_sink_tokens=q_sink, query_blocks=query_blocks)
    ksel = to_np(dbg["selected"]).astype(bool)
    qbs = np.arange(qm.shape[1]) if query_blocks is None else np.asarray(query_blocks)
    ksel_s, sel_s = ksel[:, qbs], sel[:, qbs]
    mismatch = ksel_s != sel_s
    in_band = 0
    if math.isfinite(beta):
        c = cut[:, qbs][..., None]
        qn_norm = np.linalg.norm(qm[:, qbs], axis=-1)[..., None]            # [B, n, H, 1]
        kn_norm = np.linalg.norm(kc, axis=-1).transpose(0, 2, 1)[:, None]   # [B, 1, H, NKB]
        band = BAND * np.maximum(np.abs(c), s * qn_norm * kn_norm)
        gap = np.abs(proxy[:, qbs] - c)
        in_band = int((gap <= band).sum())
        outside = mismatch & (gap > band)
        assert not outside.any(), f"{int(outside.sum())} routing decisions differ outside the band"
    else:
        assert not mismatch.any(), "infinite beta routing must match exactly"
    cap = (max_band_mismatch if max_band_mismatch is not None
           else int(MAX_BAND_MISMATCH_RATE * mismatch.size))
    print(f"routing {label} beta={beta}: {mismatch.size} decisions, {int(mismatch.sum())} in-band "
          f"mismatches (cap {cap}), {in_band} decisions inside the band", flush=True)
    assert mismatch.sum() <= cap, f"{int(mismatch.sum())} in-band mismatches exceed the cap {cap}"
    # Kernel proxies and cutoffs agree with the oracle's to FP32 rounding.
    if math.isfinite(beta):
        kp = to_np(dbg["proxy"])[:, qbs]
        np.testing.assert_allclose(kp, proxy[:, qbs], rtol=1e-4, atol=1e-5 * np.abs(proxy[:, qbs]).max())
        np.testing.assert_allclose(to_np(dbg["cutoff"])[:, qbs], cut[:, qbs], rtol=1e-4,
                                   atol=1e-5 * np.abs(cut).max())
    kcounts = counts.cpu().numpy()[:, qbs]
    np.testing.assert_array_equal(kcounts, ksel_s.sum(-1))
    # (b) output under identical routing: the oracle evaluated with the kernel's decisions.
    ref, _, _ = orc.sol_oracle(qn, kn, vn, beta=beta, scale=s, local_blocks=local,
                               kv_sink_tokens=kv_sink, query_sink_tokens=q_sink,
                               query_blocks=list(qbs), selected=ksel)
    rows = np.concatenate([np.arange(64 * x, min(qn.shape[1], 64 * x + 64)) for x in qbs])
    return to_np(out.cpu())[:, rows], ref[:, rows], mismatch


def workload(name):
    """A bench workload's inputs (seed 0, one CPU generator, draw order Q, K, V)."""
    cfg = bench.WORKLOADS[name]
    q, k, v = bench.make_inputs(cfg, torch.device("cuda"))
    return cfg, q, k, v


@pytest.mark.parametrize("group", [1, 2])
def test_c1_whole_call_against_oracle(group, monkeypatch):
    # B=1, T=1024, H=8, D=64, block-smooth (noise 0.1), seed 0, beta 1, sinks
    # 128, local 1: every query block of the call against the oracle.
    monkeypatch.setattr(_native, "WORKGROUP_FORM", group)
    cfg, q, k, v = workload("selfattn-1024-smooth")
    assert q.shape == (1, 1024, 8, 64)
    actual, ref, _ = check_routing(q, k, v, cfg["beta"], local=cfg["local_blocks"],
                                   kv_sink=cfg["kv_sink_tokens"], q_sink=cfg["query_sink_tokens"],
                                   label=f"C1 form {group}")
    assert_close(actual, ref)
    out, stats = sol_attention(q, k, v, beta=cfg["beta"], local_blocks=cfg["local_blocks"],
                               kv_sink_tokens=cfg["kv_sink_tokens"],
                               query_sink_tokens=cfg["query_sink_tokens"], return_stats=True)
    ref_all, counts, _ = orc.sol_oracle(to_np(q.cpu()), to_np(k.cpu()), to_np(v.cpu()), beta=cfg["beta"],
                                        local_blocks=cfg["local_blocks"], kv_sink_tokens=cfg["kv_sink_tokens"],
                                        query_sink_tokens=cfg["query_sink_tokens"])
    assert_close(out.cpu(), ref_all)
    np.testing.assert_array_equal(stats.exact_blocks.cpu().numpy(), counts)


@pytest.mark.parametrize("beta", [-math.inf, 0.0, 1.0, math.inf])
@pytest.mark.parametrize("kind", ["smooth", "random"])
def test_c2_shape_routing_and_output(beta, kind):
    # B=2, T=4096, H=16, D=128, sinks 128, local 1, seed 0; oracle on 6 query blocks.
    cfg, q, k, v = workload(f"selfattn-4096-{kind}")
    qbs = [0, 1, 2, 31, 32, 63]
    actual, ref, _ = check_routing(q, k, v, beta, kv_sink=cfg["kv_sink_tokens"],
                                   q_sink=cfg["query_sink_tokens"], local=cfg["local_blocks"],
                                   query_blocks=qbs, label=f"C2 {kind}")
    assert_close(actual, ref)


@pytest.mark.parametrize("beta", [-math.inf, 0.0, 1.0, math.inf])
@pytest.mark.parametrize("name", ["selfattn-4096-smooth", "selfattn-4096-random", "crossattn-4096x10000-random"])
def test_routing_every_decision(name, beta):
    # Every (query block, key block, head) decision of the configuration's
    # call against the oracle's (float64 Qc . Kc_j): none outside the band.
    cfg, q, k, v = workload(name)
    if name.startswith("cross") and beta != 1.0:
        pytest.skip("the cross-attention configuration runs at beta 1")
    kw = dict(local_blocks=cfg["local_blocks"], kv_sink_tokens=cfg["kv_sink_tokens"],
              query_sink_tokens=cfg["query_sink_tokens"])
    _, counts, dbg = run_debug(q, k, v, beta, local=kw["local_blocks"], kv_sink=kw["kv_sink_tokens"],
                               q_sink=kw["query_sink_tokens"])
    res = orc.routing_check(q.cpu(), k.cpu(), dbg["selected"].cpu(), beta=beta, **kw)
    print(f"routing every decision {name} beta={beta}: {res}", flush=True)
    assert res["decisions"] == dbg["selected"].numel()
    assert res["outside_band"] == 0
    assert res["mismatches"] <= MAX_BAND_MISMATCH_RATE * res["decisions"]
    np.testing.assert_array_equal(counts.cpu().numpy(), dbg["selected"].sum(-1).cpu().numpy())


def test_c3_ragged_cross_attention_strided_query():
    # B=1, H=24, D=128, Tq=4096, Tk=10000, Q head-strided view, random, seed 0;
    # beta 1, kv sink 64, q sink 0, local 0.
    cfg, q, k, v = workload("crossattn-4096x10000-random")
    assert q.stride(2) == 256 and k.shape[1] == 10000
    actual, ref, _ = check_routing(q, k, v, cfg["beta"], local=cfg["local_blocks"],
                                   kv_sink=cfg["kv_sink_tokens"], q_sink=cfg["query_sink_tokens"],
                                   query_blocks=[0, 17, 40, 63], label="C3")
    assert_close(actual, ref)


@pytest.mark.parametrize("d", [64, 128])
def test_dense_limit_matches_dense_kernel(d):
    # (c) beta=-inf reproduces dense attention within BF16 tolerance.
    q, k, v = tensors(nq=777, nk=1500, d=d, b=2, h=3, device="cuda", seed=4)
    sol = sol_attention(q, k, v, beta=-math.inf)
    dense = dense_attention(q, k, v)
    assert_close(sol.cpu(), dense.cpu())
    assert_close(dense.cpu(), orc.dense_oracle(q.cpu(), k.cpu(), v.cpu()))


def test_repeat_calls_are_bitwise_deterministic():
    q, k, v = (block_smooth(1, 3000, 8, 128, seed=s, device="cuda") for s in (5, 6, 7))
    a, sa = sol_attention(q, k, v, beta=1.0, kv_sink_tokens=128, query_sink_tokens=128, return_stats=True)
    for _ in range(3):
        b, sb = sol_attention(q, k, v, beta=1.0, kv_sink_tokens=128, query_sink_tokens=128,
                              return_stats=True)
        assert torch.equal(a, b) and torch.equal(sa.exact_blocks, sb.exact_blocks)
