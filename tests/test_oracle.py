"""CPU pins of the oracle (oracle/sol_oracle.py) -- no GPU needed.

Each oracle function is checked against something it does not share code
with: torch's own BF16 cast / mean / SDPA, NumPy's variance, golden vectors
written from the reference's oracle (tests/golden/make_golden.py), the
reference tests' known answers, and a float64 brute force of the
virtual-token definition.
"""

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import sol_oracle as orc
from sol_testlib import tensors, to_np

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz")


def sdpa(q, k, v, scale=None):
    return F.scaled_dot_product_attention(q.float().transpose(1, 2), k.float().transpose(1, 2),
                                          v.float().transpose(1, 2), scale=scale).transpose(1, 2)


# --- BF16 rounding, block means, moments -------------------------------------

def test_bf16_round_matches_torch_cast():
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(100000, generator=g) * 10.0 ** torch.randint(-30, 30, (100000,), generator=g),
                   torch.tensor([0.0, -0.0, 1.0, 1.00390625, 1.01171875, -1.00390625, 3.0e38, -3.0e38,
                                 1e-40, float("inf"), -float("inf")])])
    # 1.00390625 = 1 + 2^-8 is an exact tie (rounds to even 1.0); 1.01171875 ties up.
    expected = x.to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(orc.bf16_round(x.numpy()), expected)


@pytest.mark.parametrize("shape", [(1, 317, 2, 64), (2, 1089, 3, 128), (1, 64, 1, 64), (1, 1, 2, 128),
                                   (1, 4100, 4, 64)])
def test_block_means_bit_exact_with_torch_mean(shape):
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(shape, generator=g, dtype=torch.bfloat16)
    t = shape[1]
    ref = torch.stack([x[:, i:i + 64].float().mean(1) for i in range(0, t, 64)], 1)
    np.testing.assert_array_equal(orc.block_means(to_np(x), round_bf16=False), ref.numpy())
    np.testing.assert_array_equal(orc.block_means(to_np(x), round_bf16=True),
                                  ref.to(torch.bfloat16).float().numpy())


@pytest.mark.parametrize("nkb", [1, 5, 16, 17, 255, 256, 257, 1323, 4097])
def test_key_moments_bit_exact_and_population(nkb):
    g = torch.Generator().manual_seed(nkb)
    kc = torch.randn((2, nkb, 3, 64), generator=g).to(torch.bfloat16).float()
    mean, var = orc.key_moments(kc.numpy())
    ref_mean = kc.mean(1)
    ref_var = (kc.square().mean(1) - ref_mean.square()).clamp_min(0)
    np.testing.assert_array_equal(mean, ref_mean.numpy())
    np.testing.assert_array_equal(var, ref_var.numpy())
    # Population (ddof=0) variance, not the sample estimator.
    np.testing.assert_allclose(var, np.var(kc.double().numpy(), axis=1), rtol=2e-3, atol=1e-5)


# --- golden vectors from the reference oracle --------------------------------

GOLDEN_A = {
    "b1": dict(beta=1.0), "b0": dict(beta=0.0), "bhalf_l0": dict(beta=0.5, local_blocks=0),
    "bneg_l2": dict(beta=-0.75, local_blocks=2),
    "b1_sinks": dict(beta=1.0, kv_sink_tokens=65, query_sink_tokens=1, local_blocks=0),
    "binf_sinks": dict(beta=math.inf, kv_sink_tokens=65, query_sink_tokens=1, local_blocks=0),
    "b2_scale": dict(beta=2.0, scale=0.05),
}


def _golden():
    return np.load(GOLDEN)


@pytest.mark.parametrize("name", sorted(GOLDEN_A))
def test_oracle_matches_reference_vectors_fixture_a(name):
    z = _golden()
    q, k, v = (orc.bf16_bits_to_f32(z["A_" + n]) for n in "qkv")
    out, counts, _ = orc.sol_oracle(q, k, v, **GOLDEN_A[name])
    np.testing.assert_array_equal(counts, z[f"A_{name}_counts"])
    np.testing.assert_allclose(out, z[f"A_{name}_out"], atol=5e-6, rtol=1e-5)


@pytest.mark.parametrize("name,beta", [("b1", 1.0), ("b0", 0.0)])
def test_oracle_matches_reference_vectors_fixture_b(name, beta):
    z = _golden()
    q, k, v = (orc.bf16_bits_to_f32(z["B_" + n]) for n in "qkv")
    out, counts, _ = orc.sol_oracle(q, k, v, beta=beta)
    np.testing.assert_array_equal(counts, z[f"B_{name}_counts"])
    np.testing.assert_allclose(out, z[f"B_{name}_out"], atol=5e-6, rtol=1e-5)


def test_oracle_matches_reference_vectors_protected_smooth():
    z = _golden()
    q, k, v = (orc.bf16_bits_to_f32(z["C_" + n]) for n in "qkv")
    out, counts, _ = orc.sol_oracle(q, k, v, beta=1.0, local_blocks=-1, protected_blocks=z["C_prot"])
    np.testing.assert_array_equal(counts, z["C_b1_counts"])
    np.testing.assert_allclose(out, z["C_b1_out"], atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("i", [0, 1, 2])
def test_plan_protection_matches_reference_vectors(i):
    z = _golden()
    meta = [int(x) for x in z[f"D{i}_meta"]]
    ranges = ((meta[2], meta[3]), (meta[4], meta[5]))
    prot = orc.plan_protection(z[f"D{i}_rows"], z[f"D{i}_keys"], meta[0], ranges, meta[1])
    np.testing.assert_array_equal(prot, z[f"D{i}_prot"])


# --- known answers of the reference tests ------------------------------------

@pytest.mark.parametrize("d", [64, 128])
def test_reference_dense_limit(d):
    # test_attention.py:27-34
    q, k, v = tensors(d=d)
    out, counts, _ = orc.sol_oracle(q, k, v, beta=-math.inf)
    torch.testing.assert_close(torch.from_numpy(out), sdpa(q, k, v), atol=1e-6, rtol=2e-5)
    assert (counts == 5).all()
    np.testing.assert_allclose(orc.dense_oracle(q, k, v), sdpa(q, k, v).numpy(), atol=1e-6, rtol=2e-5)


def test_reference_constant_keys_correction():
    # test_attention.py:37-43
    q, k, v = tensors()
    k[:] = k[:, :1].clone()
    sparse, _, _ = orc.sol_oracle(q, k, v, beta=math.inf)
    dense, _, _ = orc.sol_oracle(q, k, v, beta=-math.inf)
    np.testing.assert_allclose(sparse, dense, atol=0.001, rtol=0.04)


def test_reference_prefix_protection_rounds_outward():
    # test_attention.py:46-52
    q, k, v = tensors()
    _, counts, _ = orc.sol_oracle(q, k, v, beta=math.inf, kv_sink_tokens=65,
                                  query_sink_tokens=1, local_blocks=0)
    assert (counts[:, 0] == 5).all()
    assert (counts[:, 1] == 2).all()
    assert (counts[:, 2:] == 3).all()


def test_reference_query_subset_preserves_full_key_moments():
    # test_indexed.py:32-42
    g = torch.Generator().manual_seed(7)
    q = torch.randn((1, 129, 1, 64), generator=g, dtype=torch.bfloat16)
    k, v = [torch.randn((1, 205, 1, 64), generator=g, dtype=torch.bfloat16) for _ in range(2)]
    full, full_counts, _ = orc.sol_oracle(q, k, v, beta=0.0)
    part, counts, _ = orc.sol_oracle(q, k, v, beta=0.0, query_blocks=[0, 2])
    np.testing.assert_array_equal(part[:, :64], full[:, :64])
    np.testing.assert_array_equal(part[:, 128:], full[:, 128:])
    assert np.isnan(part[:, 64:128]).all()
    assert (counts[:, 1] == -1).all()
    np.testing.assert_array_equal(counts[:, [0, 2]], full_counts[:, [0, 2]])


def test_plan_protection_known_answers():
    # test_indexed.py:20-29
    rows = np.stack((np.arange(87, 152), np.arange(300, 365)))
    keys = np.stack((np.concatenate((np.arange(0, 23), np.arange(70, 198), np.arange(500, 509))),
                     np.concatenate((np.arange(0, 23), np.arange(283, 411), np.arange(500, 509)))))
    prot = orc.plan_protection(rows, keys, 509, ((0, 23), (500, 509)), 0)
    assert prot.shape == (2, 2, 3) and prot.all()
    assert not orc.plan_protection(np.array([[400]]), np.arange(128)[None], 509, (), 0).any()


# --- closed forms and brute force --------------------------------------------

def test_zero_query_key_gives_length_weighted_mean_of_values():
    # All logits 0: exact tokens weigh 1 each, a centroid weighs its valid length,
    # so the output is the mean of V with approximated blocks replaced by their
    # BF16-rounded means.
    q, k, v = tensors()
    q.zero_(); k.zero_()
    out, counts, info = orc.sol_oracle(q, k, v, beta=math.inf, local_blocks=0,
                                       kv_sink_tokens=65, query_sink_tokens=1)
    vv = to_np(v)[0]
    lengths = np.minimum(64, 317 - 64 * np.arange(5))
    for qb in range(4):
        for h in range(2):
            sel = info["selected"][0, qb, h]
            parts = [vv[64 * j:64 * j + lengths[j], h] if sel[j]
                     else np.repeat(info["vc"][0, j, h][None], lengths[j], 0) for j in range(5)]
            expect = np.concatenate(parts).mean(0)
            rows = slice(64 * qb, min(193, 64 * qb + 64))
            np.testing.assert_allclose(out[0, rows, h], np.broadcast_to(expect, out[0, rows, h].shape),
                                       atol=2e-6)


def test_single_token_returns_value():
    q, k, v = tensors(nq=1, nk=1)
    for beta in (-math.inf, math.inf, 1.0):
        out, _, _ = orc.sol_oracle(q, k, v, beta=beta)
        np.testing.assert_array_equal(out, to_np(v))


def _virtual_token_bruteforce(q, k, v, sel, scale):
    """float64 restatement with an explicit virtual-token list per query block."""
    b, tq, h, d = q.shape
    tk = k.shape[1]
    out = np.zeros(q.shape)
    kc = orc.block_means(k, True).astype(np.float64)
    vc = orc.block_means(v, True).astype(np.float64)
    for bi in range(b):
        for hi in range(h):
            for qb in range(sel.shape[1]):
                keys, vals, bias = [], [], []
                for j in range(sel.shape[3]):
                    a, e = 64 * j, min(64 * j + 64, tk)
                    if sel[bi, qb, hi, j]:
                        keys += list(k[bi, a:e, hi]); vals += list(v[bi, a:e, hi]); bias += [0.0] * (e - a)
                    else:
                        keys.append(kc[bi, j, hi]); vals.append(vc[bi, j, hi]); bias.append(math.log(e - a))
                kk, vv, bb = np.array(keys, np.float64), np.array(vals, np.float64), np.array(bias)
                for r in range(64 * qb, min(tq, 64 * qb + 64)):
                    z = q[bi, r, hi].astype(np.float64) @ kk.T * scale + bb
                    p = np.exp(z - z.max())
                    out[bi, r, hi] = p @ vv / p.sum()
    return out


@pytest.mark.parametrize("beta", [1.0, 0.0])
def test_oracle_matches_float64_virtual_token_bruteforce(beta):
    q, k, v = (to_np(x) for x in tensors(nq=130, nk=200, d=64, h=2, seed=3))
    out, _, info = orc.sol_oracle(q, k, v, beta=beta, kv_sink_tokens=1)
    brute = _virtual_token_bruteforce(q, k, v, info["selected"], 64 ** -0.5)
    np.testing.assert_allclose(out, brute, atol=2e-6, rtol=1e-5)
    out64, _, _ = orc.sol_oracle(q, k, v, beta=beta, kv_sink_tokens=1, dtype=np.float64)
    np.testing.assert_allclose(out64, brute, atol=1e-6, rtol=1e-6)


def test_forced_routing_reproduces_given_decisions():
    q, k, v = (to_np(x) for x in tensors())
    rng = np.random.default_rng(0)
    forced = rng.random((1, 4, 2, 5)) < 0.4
    out, counts, info = orc.sol_oracle(q, k, v, beta=1.0, selected=forced)
    np.testing.assert_array_equal(counts, forced.sum(-1))
    brute = _virtual_token_bruteforce(q, k, v, forced, 64 ** -0.5)
    np.testing.assert_allclose(out, brute, atol=2e-6, rtol=1e-5)


# Full-covariance thresholds (roadmap item 4 of the reference; no reference
# implementation exists, so the estimator is pinned by independent identities).

def _smooth_keys(seed, nkb=37, h=2, d=16):
    rng = np.random.default_rng(seed)
    base = rng.standard_normal((1, nkb, h, d))
    mix = rng.standard_normal((d, d)) * 0.4                 # correlated features
    return orc.bf16_round((base @ mix + 0.3).astype(np.float32))


def test_full_covariance_quadratic_form_identity():
    kc = _smooth_keys(3)
    cov = orc.key_covariance(kc)
    assert cov.shape == (1, 2, 16, 16)
    np.testing.assert_allclose(cov, np.swapaxes(cov, -1, -2), rtol=0, atol=1e-6)
    rng = np.random.default_rng(4)
    qm = rng.standard_normal((1, 5, 2, 16)).astype(np.float32)
    k64 = kc.astype(np.float64)
    proj = np.einsum("bqhd,bjhd->bqhj", qm.astype(np.float64), k64)      # Qc . Kc_j
    mu = proj.mean(-1)
    quad = (proj ** 2).mean(-1) - mu ** 2                                 # E[(Qc.Kc)^2] - (Qc.mu)^2
    mean, _ = orc.key_moments(kc)
    got = orc.cutoffs_full(qm, mean, cov, beta=1.0, scale=1.0) - orc.cutoffs_full(qm, mean, cov, 0.0, 1.0)
    np.testing.assert_allclose(got, np.sqrt(np.maximum(quad, 0)), rtol=2e-5, atol=1e-5)


def test_full_covariance_equals_diagonal_when_one_feature_varies():
    rng = np.random.default_rng(5)
    kc = np.tile(rng.standard_normal((1, 1, 2, 16)), (1, 29, 1, 1))
    kc[..., 3] += rng.standard_normal((1, 29, 2))
    kc = orc.bf16_round(kc.astype(np.float32))
    qm = rng.standard_normal((1, 4, 2, 16)).astype(np.float32)
    mean, var = orc.key_moments(kc)
    full = orc.cutoffs_full(qm, mean, orc.key_covariance(kc), 1.5, 0.125)
    diag = orc.cutoffs(qm, mean, var, 1.5, 0.125)
    np.testing.assert_allclose(full, diag, rtol=1e-5, atol=1e-6)


def test_full_covariance_beta_zero_and_oracle_option():
    rng = np.random.default_rng(6)
    q, k, v = (orc.bf16_round(rng.standard_normal((1, 200, 2, 64)).astype(np.float32)) for _ in range(3))
    a, ca, ia = orc.sol_oracle(q, k, v, beta=0.0)
    b, cb, ib = orc.sol_oracle(q, k, v, beta=0.0, threshold_estimator="full_covariance")
    np.testing.assert_allclose(ia["cutoff"], ib["cutoff"], rtol=1e-5, atol=1e-6)
    assert ib["cov"].shape == (1, 2, 64, 64) and ia["cov"] is None
    with pytest.raises(ValueError):
        orc.sol_oracle(q, k, v, threshold_estimator="banded")


def test_int8_quantisation_closed_forms():
    # Round half to even, clamp, the scale, and an all-zero group.
    x = np.array([[0.5, 1.5, -2.5, 127.0], [0.0, 0.0, 0.0, 0.0], [254.0, -1.0, 63.5, 127.5]], np.float32)
    q, sc = orc.quantize_sym(x, axes=1)
    np.testing.assert_array_equal(q[0], [0, 2, -2, 127])       # amax 127: q = rint(x)
    np.testing.assert_array_equal(q[1], [0, 0, 0, 0])
    np.testing.assert_array_equal(sc[:, 0], np.float32([1.0, 0.0, 2.0]))
    np.testing.assert_array_equal(q[2], [127, -0, 32, 64])      # x / 2: 31.75 -> 32, 63.75 -> 64
    k = np.zeros((1, 70, 1, 16), np.float32)
    k[0, 3, 0, 5] = -4.0                                        # block 0's max; block 1 is 6 rows
    k[0, 64:, 0, :] = 1.0
    k8, sk = orc.quantize_keys(k)
    assert k8.shape == k.shape and sk.shape == (1, 2, 1)
    np.testing.assert_array_equal(sk[0, :, 0], np.float32([4.0 / 127, 1.0 / 127]))
    assert k8[0, 3, 0, 5] == -127 and (k8[0, 64:] == 127).all()


def test_int8_oracle_equals_bf16_oracle_on_the_int8_grid():
    # Integer-valued Q and K whose every row / key block reaches |127| quantise
    # exactly (scale 1), so the INT8-QK oracle must reproduce the BF16 one bit
    # for bit; any other input it must not (pins the quantised path).
    rng = np.random.default_rng(8)
    q = rng.integers(-126, 127, (1, 150, 2, 64)).astype(np.float32)
    k = rng.integers(-126, 127, (1, 200, 2, 64)).astype(np.float32)
    q[..., 0] = 127.0
    k[..., 0] = -127.0
    v = orc.bf16_round(rng.standard_normal((1, 200, 2, 64)).astype(np.float32))
    scale = 1.0 / 4096
    for beta in (1.0, -math.inf, 0.0):
        a, ca, _ = orc.sol_oracle(q, k, v, beta=beta, scale=scale)
        b, cb, _ = orc.sol_oracle(q, k, v, beta=beta, scale=scale, qk_precision="int8")
        np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(ca, cb)
    c, _, _ = orc.sol_oracle(q * 1.37, k, v, beta=1.0, scale=scale, qk_precision="int8")
    d, _, _ = orc.sol_oracle(q * 1.37, k, v, beta=1.0, scale=scale)
    assert not np.array_equal(c, d)


def test_quantised_pv_accuracy_against_bf16_control():
    """The FP8 P V half of the roadmap experiment, in simulation: the
    probabilities rounded to FP8-e4m3 (with V kept BF16, or V also FP8)
    instead of BF16, float64 elsewhere, against the BF16-P control.  On
    random inputs FP8 P leaves the parity bar (rel-L2 0.8%); on block-smooth
    inputs it stays inside it."""
    rng = np.random.default_rng(1)
    t, d = 1024, 128

    def fp8(x):
        return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).float().numpy()

    def attn(q, k, v, pq, pv):
        s = q.astype(np.float64) @ k.T.astype(np.float64) / math.sqrt(d)
        p = np.exp(s - s.max(1, keepdims=True))
        return (pq(p) @ pv(v)) / p.sum(1, keepdims=True)

    bf = lambda x: orc.bf16_round(np.asarray(x, np.float32))  # noqa: E731
    ident = lambda x: x  # noqa: E731

    def smooth():
        c = rng.standard_normal((t // 64, d))
        return bf(np.repeat(c, 64, 0) + 0.1 * rng.standard_normal((t, d)))

    errs = {}
    for name, make in (("random", lambda: bf(rng.standard_normal((t, d)))), ("smooth", smooth)):
        q, k, v = make(), make(), make()
        ref = attn(q, k, v, bf, ident)
        for label, pq, pv in (("fp8p_bf16v", fp8, ident), ("fp8p_fp8v", fp8, fp8)):
            o = attn(q, k, v, pq, pv)
            errs[(name, label)] = np.linalg.norm(o - ref) / np.linalg.norm(ref)
    assert 0.015 < errs[("random", "fp8p_bf16v")] < 0.04, errs
    assert errs[("random", "fp8p_fp8v")] > errs[("random", "fp8p_bf16v")], errs
    assert errs[("smooth", "fp8p_bf16v")] < 0.006 and errs[("smooth", "fp8p_fp8v")] < 0.008, errs


def test_quantised_qk_accuracy_against_bf16_control():
    """The INT8 / FP8 QK half of the reference roadmap's experiment row, in
    simulation: attention with Q and K rounded to FP8-e4m3, or to INT8 with one
    symmetric scale per row, against the same attention on the BF16 inputs
    (float64 softmax).  FP8 QK lands far outside the parity bar (rel-L2 0.8%);
    per-row INT8 sits at it."""
    rng = np.random.default_rng(0)
    t, d = 1024, 128

    def fp8(x):
        return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).float().numpy()

    def int8_rows(x):
        s = np.abs(x).max(1, keepdims=True) / 127.0
        return np.clip(np.round(x / s), -127, 127) * s

    def attn(q, k, v):
        s = q.astype(np.float64) @ k.T.astype(np.float64) / math.sqrt(d)
        p = np.exp(s - s.max(1, keepdims=True))
        return (p / p.sum(1, keepdims=True)) @ v

    q, k, v = (orc.bf16_round(rng.standard_normal((t, d)).astype(np.float32)) for _ in range(3))
    ref = attn(q, k, v)
    err = {name: np.linalg.norm(attn(f(q), f(k), v) - ref) / np.linalg.norm(ref)
           for name, f in (("fp8", fp8), ("int8", int8_rows))}
    assert 0.02 < err["fp8"] < 0.06, err
    assert 0.004 < err["int8"] < 0.012, err


# --- routing_check: every decision at any size (float64 Qc . Kc_j) ------------

@pytest.mark.parametrize("name", sorted(GOLDEN_A))
def test_routing_check_agrees_with_reference_routing(name):
    # The reference's own routing (per-row products, mean; `route`, whose
    # counts equal the reference oracle's golden counts) passes the check
    # with no decision outside the band, on every golden fixture.
    z = _golden()
    q, k, v = (orc.bf16_bits_to_f32(z["A_" + n]) for n in "qkv")
    kw = dict(GOLDEN_A[name])
    _, counts, info = orc.sol_oracle(q, k, v, **kw)
    np.testing.assert_array_equal(counts, z[f"A_{name}_counts"])
    beta = kw.pop("beta")
    res = orc.routing_check(q, k, info["selected"], beta=beta, **kw)
    assert res["outside_band"] == 0 and res["decisions"] == info["selected"].size
    assert res["mismatches"] == 0  # no fixture decision sits inside the 1e-5 band


def test_routing_check_protected_plan_and_full_covariance():
    z = _golden()
    q, k, v = (orc.bf16_bits_to_f32(z["C_" + n]) for n in "qkv")
    _, counts, info = orc.sol_oracle(q, k, v, beta=1.0, local_blocks=-1, protected_blocks=z["C_prot"])
    np.testing.assert_array_equal(counts, z["C_b1_counts"])
    res = orc.routing_check(q, k, info["selected"], beta=1.0, local_blocks=-1, protected_blocks=z["C_prot"])
    assert res["outside_band"] == 0 and res["mismatches"] == 0
    _, _, full = orc.sol_oracle(q, k, v, beta=1.0, threshold_estimator="full_covariance")
    res = orc.routing_check(q, k, full["selected"], beta=1.0, threshold_estimator="full_covariance")
    assert res["outside_band"] == 0


def test_routing_check_flags_planted_mistakes():
    z = _golden()
    q, k, v = (orc.bf16_bits_to_f32(z["A_" + n]) for n in "qkv")
    _, _, info = orc.sol_oracle(q, k, v, beta=1.0, local_blocks=0)
    sel = info["selected"]
    # The decision farthest from its cutoff, flipped: outside the band.
    gap = np.abs(info["proxy"] - info["cutoff"][..., None])
    gap[sel & ~(info["proxy"] > info["cutoff"][..., None])] = -1.0  # protected blocks aside
    far = np.unravel_index(np.argmax(gap), gap.shape)
    bad = sel.copy()
    bad[far] = ~bad[far]
    res = orc.routing_check(q, k, bad, beta=1.0, local_blocks=0)
    assert res["outside_band"] == 1 and res["mismatches"] == 1 and res["max_rel_gap"] > 1.0
    # A protected block left unselected, and forced routing: exact agreement is required.
    bad = sel.copy()
    bad[0, 0, 0, 0] = False                     # the local band always holds (qb 0, kb 0)
    assert orc.routing_check(q, k, bad, beta=1.0, local_blocks=0)["outside_band"] == 1
    _, _, inf = orc.sol_oracle(q, k, v, beta=math.inf, kv_sink_tokens=65, local_blocks=0)
    bad = inf["selected"].copy()
    bad[0, -1, 0, -1] = ~bad[0, -1, 0, -1]
    assert orc.routing_check(q, k, inf["selected"], beta=math.inf, kv_sink_tokens=65,
                             local_blocks=0)["outside_band"] == 0
    assert orc.routing_check(q, k, bad, beta=math.inf, kv_sink_tokens=65, local_blocks=0)["outside_band"] == 1
