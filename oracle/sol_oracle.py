"""CPU oracle for SOL routed attention -- TEST INFRASTRUCTURE ONLY.

This module checks the product and is never part of it.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it.
The shipped package (``sol_attn_amd``) never imports it and has no CPU path.

It restates, in NumPy float32, the algorithm of the reference oracle
``src/sol_attn_amd/reference.py:13-66`` and the protection builder
``src/sol_attn_amd/indexed.py:27-62``.  The formulation is our own:

* Block means and key moments follow torch's CPU outer-dimension summation
  order (16-row sequential chunks folded through four accumulator levels), so
  centroids, query means and key moments are bit-identical to the reference
  oracle's ``Tensor.mean`` results (checked by ``tests/test_oracle.py``).
* Attention is evaluated as ONE masked softmax over the exact-token logits and
  the centroid logits (``+ ln(valid_len)``) instead of the reference's
  concatenated virtual-token list; the two are the same mathematics.

Pinning status (each function's check lives in ``tests/test_oracle.py``):
``bf16_round`` vs torch's BF16 cast; ``block_means`` and ``key_moments`` vs
torch ``mean`` (bit-exact) and NumPy ``var``; ``cutoffs``/``route``/``sol_oracle``
vs golden vectors written from the reference oracle, the dense limit (FP32
SDPA), the prefix-protection known answer ``[5, 2, 3, 3]`` and a float64
brute force of the virtual-token definition; ``plan_protection`` vs the
reference's known answers and golden vectors; ``key_covariance`` /
``cutoffs_full`` (the full-covariance threshold experiment of the reference's
roadmap, which the reference does not implement) vs the identity
``Qc^T cov Qc = mean_j (Qc . Kc_j)^2 - (Qc . mu)^2``, the diagonal estimator
when only one feature varies, and beta = 0.  No function is parity unpinned.
"""

from __future__ import annotations

import math
from typing import Iterable, Optional, Sequence

import numpy as np

BLOCK = 64  # physical block size, src/sol_attn_amd/kernels.py:12
_LEVELS = 4  # accumulator levels of torch's cascade sum


# ----------------------------------------------------------------------------
# BF16 helpers
# ----------------------------------------------------------------------------

def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest BF16 (ties to even); float32 out.

    Matches ``Tensor.to(torch.bfloat16)`` for finite values
    (``reference.py:14-15`` rounds K/V block means this way).
    """
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    r = (u + np.uint32(0x7FFF) + lsb) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def bf16_bits_to_f32(bits) -> np.ndarray:
    """uint16 BF16 bit patterns -> float32 values (exact)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 (already BF16-representable or not) -> uint16 RNE bit patterns."""
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


# ----------------------------------------------------------------------------
# Summation order of torch's CPU outer reduction
# ----------------------------------------------------------------------------

def _level_power(n: int) -> int:
    ceil_log2 = 0 if n <= 1 else int(math.ceil(math.log2(n)))
    return max(4, ceil_log2 // _LEVELS)


def cascade_sum(x: np.ndarray, axis: int = 1) -> np.ndarray:
    """Sum ``x`` over ``axis`` in float32 with torch's outer-reduction order.

    Rows are added sequentially into level 0 in chunks of ``2**lp`` rows
    (``lp = max(4, ceil(log2 n) // 4)``); each full chunk is carried into
    level 1, level 1 into level 2 every ``2**(2 lp)`` rows, and so on; finally
    ``((acc0 + acc1) + acc2) + acc3``.  This is the order ``Tensor.mean``
    uses for ``x[:, i:i + 64].float().mean(1)`` and ``km.mean(1)`` in
    ``reference.py:14,27-28``.
    """
    x = np.moveaxis(np.asarray(x, dtype=np.float32), axis, 0)
    n = x.shape[0]
    lp = _level_power(n)
    step = 1 << lp
    mask = step - 1
    acc = [np.zeros(x.shape[1:], np.float32) for _ in range(_LEVELS)]
    i = 0
    while i + step <= n:
        for _ in range(step):
            acc[0] = acc[0] + x[i]
            i += 1
        for j in range(1, _LEVELS):
            acc[j] = acc[j] + acc[j - 1]
            acc[j - 1] = np.zeros_like(acc[j - 1])
            if i & (mask << (j * lp)):
                break
    while i < n:
        acc[0] = acc[0] + x[i]
        i += 1
    out = acc[0]
    for j in range(1, _LEVELS):
        out = out + acc[j]
    return out


def block_means(x: np.ndarray, round_bf16: bool, block: int = BLOCK) -> np.ndarray:
    """Per-block means ``[B, T, H, D] -> [B, ceil(T/block), H, D]``.

    ``reference.py:13-15`` / ``kernels.py:16-27``: FP32 sum of the valid rows
    of each 64-token block divided by the valid length; BF16-rounded for K/V,
    FP32 for Q.  Tail blocks pad with zero rows, which leaves torch's cascade
    order unchanged (adding +0.0 is exact).
    """
    x = np.asarray(x, dtype=np.float32)
    b, t, h, d = x.shape
    nb = (t + block - 1) // block
    pad = nb * block - t
    if pad:
        x = np.concatenate([x, np.zeros((b, pad, h, d), np.float32)], 1)
    xs = x.reshape(b, nb, block, h, d)
    sums = cascade_sum(xs, axis=2) if block == BLOCK else xs.sum(2, dtype=np.float32)
    lengths = np.minimum(block, t - block * np.arange(nb)).astype(np.float32)
    means = (sums / lengths[None, :, None, None]).astype(np.float32)
    return bf16_round(means) if round_bf16 else means


def key_moments(kc: np.ndarray):
    """Diagonal population moments of pooled keys over the block axis.

    ``reference.py:27-28`` / ``kernels.py:30-49``: ``mu = mean_j Kc_j``,
    ``var = max(mean_j Kc_j^2 - mu^2, 0)``, unweighted by ragged length.
    ``kc``: ``[B, NKB, H, D]`` -> ``mean, var``: ``[B, H, D]``.
    """
    kc = np.asarray(kc, dtype=np.float32)
    n = np.float32(kc.shape[1])
    mean = (cascade_sum(kc, axis=1) / n).astype(np.float32)
    sq = (cascade_sum(kc * kc, axis=1) / n).astype(np.float32)
    var = np.maximum(sq - (mean * mean).astype(np.float32), np.float32(0))
    return mean, var.astype(np.float32)


def cutoffs(qm: np.ndarray, mean: np.ndarray, var: np.ndarray, beta: float,
            scale: float) -> np.ndarray:
    """Eq. 15 cutoff per (batch, query block, head), natural-log units.

    ``reference.py:29-30`` / ``kernels.py:52-64``:
    ``scale * (Qc . mu + beta * sqrt(sum Qc^2 var))``.
    ``qm``: ``[B, NQB, H, D]``; ``mean``/``var``: ``[B, H, D]``.
    """
    mu = (qm * mean[:, None]).sum(-1, dtype=np.float32)
    sig = np.sqrt((qm * qm * var[:, None]).sum(-1, dtype=np.float32))
    with np.errstate(invalid="ignore", over="ignore"):
        c = (mu + np.float32(beta) * sig) * np.float32(scale)
    return c.astype(np.float32)


def key_covariance(kc: np.ndarray) -> np.ndarray:
    """Full population covariance of pooled keys over the block axis.

    Roadmap item 4 of the reference (``ROADMAP.md:14-16``, "full covariance
    thresholds"); the reference implements only the diagonal.  The same
    estimator as ``key_moments`` without discarding the off-diagonal terms:
    ``cov = mean_j Kc_j Kc_j^T - mu mu^T``, unweighted by ragged length,
    evaluated in float64.  ``kc``: ``[B, NKB, H, D]`` -> ``[B, H, D, D]``.
    """
    kc = np.asarray(kc, dtype=np.float64)
    n = kc.shape[1]
    mu = kc.mean(1)                                             # [B, H, D]
    second = np.einsum("bjhd,bjhe->bhde", kc, kc) / n
    return (second - mu[..., :, None] * mu[..., None, :]).astype(np.float32)


def cutoffs_full(qm: np.ndarray, mean: np.ndarray, cov: np.ndarray, beta: float,
                 scale: float) -> np.ndarray:
    """Eq. 15 cutoff with the full covariance, natural-log units:
    ``scale * (Qc . mu + beta * sqrt(max(Qc^T cov Qc, 0)))`` (float64
    quadratic form; the clamp absorbs rounding below zero).
    ``qm``: ``[B, NQB, H, D]``; ``mean``: ``[B, H, D]``; ``cov``: ``[B, H, D, D]``.
    """
    q64 = np.asarray(qm, dtype=np.float64)
    mu = (q64 * np.asarray(mean, dtype=np.float64)[:, None]).sum(-1)
    quad = np.einsum("bqhd,bhde,bqhe->bqh", q64, np.asarray(cov, dtype=np.float64), q64)
    with np.errstate(invalid="ignore", over="ignore"):
        c = (mu + beta * np.sqrt(np.maximum(quad, 0.0))) * scale
    return c.astype(np.float32)


THRESHOLD_ESTIMATORS = ("diagonal_covariance", "full_covariance")


# ----------------------------------------------------------------------------
# INT8 QK (the quantised-score experiment of the reference's roadmap,
# ROADMAP.md:14-16; the reference does not implement it)
# ----------------------------------------------------------------------------

def quantize_sym(x: np.ndarray, axes) -> tuple:
    """Symmetric INT8 quantisation over ``axes``: ``amax = max|x|``,
    ``q = clip(rint(x * float32(127 / amax)), -127, 127)`` (round half to
    even), ``scale = amax / 127`` (float32 arithmetic; an all-zero group gets
    scale 0 and zeros).  Returns ``(q as float32 integers, scale)`` with the
    scale keeping ``axes`` as size-1 dimensions."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=axes, keepdims=True)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint((x * inv).astype(np.float32)), -127, 127).astype(np.float32)
    return q, (amax / np.float32(127.0)).astype(np.float32)


def quantize_keys(k: np.ndarray) -> tuple:
    """Per 64-key block and head one scale: ``k`` ``[B, Tk, H, D]`` ->
    ``(k8 [B, Tk, H, D], scale [B, NKB, H])`` (the tail block's absent rows
    count as zeros)."""
    b, tk, h, d = k.shape
    nkb = -(-tk // BLOCK)
    pad = np.zeros((b, nkb * BLOCK, h, d), np.float32)
    pad[:, :tk] = k
    q, sc = quantize_sym(pad.reshape(b, nkb, BLOCK, h, d), axes=(2, 4))
    return q.reshape(b, nkb * BLOCK, h, d)[:, :tk], sc.reshape(b, nkb, h)


# ----------------------------------------------------------------------------
# Routing
# ----------------------------------------------------------------------------

def _protection_mask(nqb: int, nkb: int, local_blocks: int, kv_sink_tokens: int,
                     query_sink_tokens: int, block: int = BLOCK) -> np.ndarray:
    """Static protection ``[NQB, NKB]`` (``reference.py:46-51``).

    Local band ``|qb - kb| <= local_blocks`` (never when ``local_blocks < 0``),
    key-prefix sink ``kb * 64 < kv_sink_tokens`` and query-prefix sink
    ``qb * 64 < query_sink_tokens``; prefixes round outward to whole blocks.
    """
    qb = np.arange(nqb)[:, None]
    kb = np.arange(nkb)[None, :]
    prot = np.abs(qb - kb) <= local_blocks
    prot |= (kb * block) < kv_sink_tokens
    prot |= (qb * block) < query_sink_tokens
    return prot


def route(q: np.ndarray, kc: np.ndarray, cut: np.ndarray, *, beta: float, scale: float,
          local_blocks: int, kv_sink_tokens: int, query_sink_tokens: int,
          protected_blocks: Optional[np.ndarray] = None, block: int = BLOCK,
          query_blocks: Optional[Sequence[int]] = None):
    """Per-(batch, query block, head, key block) routing decisions.

    ``reference.py:39-51``: ``proxy = scale * mean_r (Q_r . Kc_j)``;
    selected when ``proxy > cutoff`` (strict); beta=-inf selects all,
    beta=+inf none; then OR with the static and plan protection.
    Returns ``selected`` (bool) and ``proxy`` (float32), both
    ``[B, NQB, H, NKB]``.  With ``query_blocks`` only those query blocks get
    proxies (the rest hold NaN and are not selected unless protected).
    """
    b, tq, h, d = q.shape
    nqb, nkb = cut.shape[1], kc.shape[1]
    pad = nqb * block - tq
    qp = np.concatenate([q, np.zeros((b, pad, h, d), np.float32)], 1) if pad else q
    lengths = np.minimum(block, tq - block * np.arange(nqb)).astype(np.float32)
    qbs = np.arange(nqb) if query_blocks is None else np.asarray(list(query_blocks), np.int64)
    rows = (qbs[:, None] * block + np.arange(block)[None, :]).reshape(-1)
    proxy = np.full((b, nqb, h, nkb), np.nan, np.float32)
    for bi in range(b):
        for hi in range(h):
            dots = qp[bi, rows, hi] @ kc[bi, :, hi].T          # [len(qbs)*64, NKB]
            dots = dots.reshape(len(qbs), block, nkb)
            proxy[bi, qbs, hi] = cascade_sum(dots, axis=1) / lengths[qbs, None] * np.float32(scale)
    if beta == -math.inf:
        selected = np.ones(proxy.shape, bool)
    elif beta == math.inf:
        selected = np.zeros(proxy.shape, bool)
    else:
        with np.errstate(invalid="ignore"):
            selected = proxy > cut[..., None]
    selected |= _protection_mask(nqb, nkb, local_blocks, kv_sink_tokens,
                                 query_sink_tokens, block)[None, :, None, :]
    if protected_blocks is not None:
        selected |= np.asarray(protected_blocks, bool)[:, :, None, :]
    return selected, proxy


def routing_check(q, k, kernel_selected, *, beta: float, scale: Optional[float] = None,
                  local_blocks: int = 1, kv_sink_tokens: int = 0, query_sink_tokens: int = 0,
                  protected_blocks=None, threshold_estimator: str = "diagonal_covariance",
                  band: float = 1e-5) -> dict:
    """Every (batch, query block, head, key block) decision of a kernel against
    the oracle's, at any size.

    The proxy ``scale * mean_r (Q_r . Kc_j)`` (``reference.py:39``) equals
    ``scale * Qc . Kc_j`` in exact arithmetic (``Qc`` the query block's mean),
    so it is formed as one float64 product per head, ``Qc Kc^T``, from the
    oracle's bit-exact FP32 ``Qc`` and BF16 ``Kc``; the cutoff
    (``reference.py:29-30``) likewise in float64 from the oracle's FP32
    moments.  Decisions: ``proxy > cutoff`` (strict), forced for beta = +-inf,
    OR the local band, sinks and plan protection (``reference.py:40-51``).
    A kernel decision may differ only where
    ``|proxy - cutoff| <= band * max(|cutoff|, scale |Qc| |Kc_j|)`` (the
    magnitudes an FP32 evaluation rounds against).  ``kernel_selected``:
    bool ``[B, NQB, H, NKB]``.  Returns counts: ``decisions``, ``mismatches``,
    ``outside_band`` (must be 0), ``in_band`` (decisions inside the band) and
    ``max_rel_gap`` (largest ``|proxy - cutoff|`` over the band's scale among
    the mismatches; at most 1 when none lies outside).
    """
    q, k = _as_f32(q), _as_f32(k)
    ksel = _as_bool(kernel_selected)
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else float(scale)
    qm = block_means(q, round_bf16=False)
    kc = block_means(k, round_bf16=True)
    mean, var = key_moments(kc)
    b, nqb, h, _ = qm.shape
    nkb = kc.shape[1]
    prot_static = _protection_mask(nqb, nkb, local_blocks, kv_sink_tokens, query_sink_tokens)
    prot = None if protected_blocks is None else _as_bool(protected_blocks)
    cov = key_covariance(kc) if threshold_estimator == "full_covariance" else None
    res = dict(decisions=0, mismatches=0, outside_band=0, in_band=0, max_rel_gap=0.0)
    for bi in range(b):
        for hi in range(h):
            q64 = qm[bi, :, hi].astype(np.float64)                    # [NQB, D]
            k64 = kc[bi, :, hi].astype(np.float64)                    # [NKB, D]
            if beta == -math.inf:
                sel = np.ones((nqb, nkb), bool)
                gap = rel = None
            elif beta == math.inf:
                sel = np.zeros((nqb, nkb), bool)
                gap = rel = None
            else:
                mu = q64 @ mean[bi, hi].astype(np.float64)
                if cov is None:
                    quad = (q64 * q64) @ var[bi, hi].astype(np.float64)
                else:
                    quad = np.maximum(np.einsum("qd,de,qe->q", q64, cov[bi, hi].astype(np.float64), q64), 0.0)
                cut = scale * (mu + beta * np.sqrt(quad))                 # [NQB]
                proxy = scale * (q64 @ k64.T)                             # [NQB, NKB]
                sel = proxy > cut[:, None]
                width = band * np.maximum(np.abs(cut)[:, None],
                                          scale * np.linalg.norm(q64, axis=1)[:, None]
                                          * np.linalg.norm(k64, axis=1)[None, :])
                gap = np.abs(proxy - cut[:, None])
                rel = gap / np.maximum(width, np.finfo(np.float64).tiny)
            sel |= prot_static
            if prot is not None:
                sel |= prot[bi]
            got = ksel[bi, :, hi]
            diff = got != sel
            res["decisions"] += sel.size
            res["mismatches"] += int(diff.sum())
            if rel is None:
                res["outside_band"] += int(diff.sum())
            else:
                inside = rel <= 1.0
                res["in_band"] += int(inside.sum())
                res["outside_band"] += int((diff & ~inside).sum())
                if diff.any():
                    res["max_rel_gap"] = max(res["max_rel_gap"], float(rel[diff].max()))
    return res


# ----------------------------------------------------------------------------
# Attention
# ----------------------------------------------------------------------------

def _attend(qrows, k, v, kc, vc, sel_rows, lengths, scale, dtype, exact_scores=None):
    """One masked softmax over exact tokens and centroid virtual tokens.

    ``qrows``: ``[R, D]``; ``sel_rows``: ``[R, NKB]`` routing of each row's
    query block.  Selected blocks contribute every valid token
    (``reference.py:54-57``); the rest contribute ``Kc_j`` with logit
    ``+ ln(len_j)`` and value ``Vc_j`` (``reference.py:58-61``).
    ``exact_scores`` (``[R, Tk]``, natural-log units) replaces ``Q K^T * scale``
    for the exact tokens (the INT8-QK experiment).
    """
    tk = k.shape[0]
    nkb = kc.shape[0]
    token_block = np.arange(tk) // BLOCK
    qrows = qrows.astype(dtype)
    if exact_scores is None:
        s_exact = (qrows @ k.astype(dtype).T) * dtype(scale)                  # [R, Tk]
    else:
        s_exact = exact_scores.astype(dtype)
    s_cent = (qrows @ kc.astype(dtype).T) * dtype(scale) + np.log(lengths.astype(dtype))  # [R, NKB]
    m_exact = sel_rows[:, token_block]
    m_cent = ~sel_rows
    neg = dtype(-np.inf)
    s_exact = np.where(m_exact, s_exact, neg)
    s_cent = np.where(m_cent, s_cent, neg)
    peak = np.maximum(s_exact.max(1), s_cent.max(1) if nkb else neg)[:, None]
    p_exact = np.exp(s_exact - peak)
    p_cent = np.exp(s_cent - peak)
    num = p_exact @ v.astype(dtype) + p_cent @ vc.astype(dtype)
    den = p_exact.sum(1) + p_cent.sum(1)
    return num / den[:, None]


def sol_oracle(q, k, v, *, beta: float = 1.0, scale: Optional[float] = None,
               local_blocks: int = 1, kv_sink_tokens: int = 0, query_sink_tokens: int = 0,
               protected_blocks=None, query_blocks: Optional[Iterable[int]] = None,
               selected: Optional[np.ndarray] = None, dtype=np.float32,
               threshold_estimator: str = "diagonal_covariance", qk_precision: str = "bf16"):
    """FP32 SOL oracle, ``reference.py:18-66`` restated.

    ``q``: ``[B, Tq, H, D]``; ``k``/``v``: ``[B, Tk, H, D]``; BF16 values held
    in float32 (or torch tensors).  ``protected_blocks``: bool
    ``[B, NQB, NKB]`` plan protection (no head axis, ``reference.py:50``).
    ``query_blocks`` restricts the evaluated query blocks; moments always use
    every key block (``reference.py:33-35``).  ``selected``, when given,
    forces the routing (``[B, NQB, H, NKB]``) so outputs can be compared
    under identical routing.  ``dtype=np.float64`` evaluates the same
    definition in double precision (brute-force check).
    ``threshold_estimator="full_covariance"`` replaces the diagonal variance
    of the cutoff with the full key covariance (``cutoffs_full``).
    ``qk_precision="int8"`` scores the exact tokens as ``s_q s_k (Q8 . K8)``
    (``quantize_sym`` per query row, ``quantize_keys`` per key block); routing,
    centroid terms and values are unchanged.

    Returns ``out`` (float32, NaN outside ``query_blocks``), ``counts``
    (int32 ``[B, NQB, H]``, -1 outside ``query_blocks``) and an ``info`` dict
    with ``selected``, ``proxy``, ``cutoff``, ``kc``, ``vc``, ``qm``,
    ``mean``, ``var``.
    """
    q, k, v = (_as_f32(x) for x in (q, k, v))
    b, tq, h, d = q.shape
    tk = k.shape[1]
    scale = d ** -0.5 if scale is None else float(scale)
    qm = block_means(q, round_bf16=False)
    kc = block_means(k, round_bf16=True)
    vc = block_means(v, round_bf16=True)
    mean, var = key_moments(kc)
    if threshold_estimator not in THRESHOLD_ESTIMATORS:
        raise ValueError(f"threshold_estimator must be one of {THRESHOLD_ESTIMATORS}")
    cov = None
    if threshold_estimator == "full_covariance":
        cov = key_covariance(kc)
        cut = cutoffs_full(qm, mean, cov, beta, scale)
    else:
        cut = cutoffs(qm, mean, var, beta, scale)
    nqb, nkb = qm.shape[1], kc.shape[1]
    prot = None if protected_blocks is None else _as_bool(protected_blocks)
    sel, proxy = route(q, kc, cut, beta=beta, scale=scale, local_blocks=local_blocks,
                       kv_sink_tokens=kv_sink_tokens, query_sink_tokens=query_sink_tokens,
                       protected_blocks=prot, query_blocks=query_blocks)
    if selected is not None:
        sel = _as_bool(selected).copy()
    lengths = np.minimum(BLOCK, tk - BLOCK * np.arange(nkb)).astype(np.float32)
    if qk_precision not in ("bf16", "int8"):
        raise ValueError("qk_precision must be 'bf16' or 'int8'")
    if qk_precision == "int8":
        q8, sq = quantize_sym(q, axes=3)                  # [B, Tq, H, D], [B, Tq, H, 1]
        k8, sk = quantize_keys(k)                         # [B, Tk, H, D], [B, NKB, H]
        sk_tok = np.repeat(sk, BLOCK, axis=1)[:, :tk]     # [B, Tk, H]
    blocks = list(range(nqb)) if query_blocks is None else [int(x) for x in query_blocks]
    out = np.full(q.shape, np.nan, np.float32)
    counts = np.full((b, nqb, h), -1, np.int32)
    for bi in range(b):
        for hi in range(h):
            for chunk in _chunks(blocks, max(1, min(32, (1 << 26) // max(tk, 1) // BLOCK))):
                rows = np.concatenate([np.arange(qb * BLOCK, min(tq, (qb + 1) * BLOCK))
                                       for qb in chunk])
                sel_rows = sel[bi, rows // BLOCK, hi]
                exact = None
                if qk_precision == "int8":
                    ints = q8[bi, rows, hi] @ k8[bi, :, hi].T           # exact integers in float32
                    exact = (ints.astype(np.float64) * sq[bi, rows, hi] * sk_tok[bi, :, hi][None, :]
                             * scale)
                res = _attend(q[bi, rows, hi], k[bi, :, hi], v[bi, :, hi], kc[bi, :, hi],
                              vc[bi, :, hi], sel_rows, lengths, scale, dtype, exact)
                out[bi, rows, hi] = res.astype(np.float32)
                for qb in chunk:
                    counts[bi, qb, hi] = int(sel[bi, qb, hi].sum())
    info = dict(selected=sel, proxy=proxy, cutoff=cut, kc=kc, vc=vc, qm=qm, mean=mean, var=var, cov=cov)
    return out, counts, info


def dense_oracle(q, k, v, *, scale: Optional[float] = None, dtype=np.float32):
    """Non-causal softmax attention over all keys (FP32), BTHD."""
    q, k, v = (_as_f32(x) for x in (q, k, v))
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else float(scale)
    out = np.empty(q.shape, np.float32)
    for bi in range(q.shape[0]):
        for hi in range(q.shape[2]):
            s = (q[bi, :, hi].astype(dtype) @ k[bi, :, hi].astype(dtype).T) * dtype(scale)
            s = np.exp(s - s.max(1, keepdims=True))
            out[bi, :, hi] = ((s @ v[bi, :, hi].astype(dtype)) / s.sum(1, keepdims=True))
    return out


# ----------------------------------------------------------------------------
# Indexed windows
# ----------------------------------------------------------------------------

def plan_protection(rows, keys, sequence_length: int, protected_ranges: Sequence = (),
                    local_tokens: int = 64) -> np.ndarray:
    """Protection of packed key blocks for indexed windows (``indexed.py:50-61``).

    Block ``(w, qb, kb)`` is protected when its packed keys touch any
    ``[a, b)`` in ``protected_ranges`` or touch the original-index
    neighbourhood ``[rows[w, 64 qb] - local_tokens, rows[w, last] + local_tokens]``
    of the query block (rows and keys are strictly increasing per window).
    """
    rows = np.asarray(rows, dtype=np.int64)
    keys = np.asarray(keys, dtype=np.int64)
    w, nq = rows.shape
    nk = keys.shape[1]
    nqb, nkb = (nq + BLOCK - 1) // BLOCK, (nk + BLOCK - 1) // BLOCK
    out = np.zeros((w, nqb, nkb), bool)
    first = np.arange(nqb) * BLOCK
    last = np.minimum(first + BLOCK, nq) - 1
    kstart = np.arange(nkb) * BLOCK
    kend = np.minimum(kstart + BLOCK, nk)  # exclusive
    for wi in range(w):
        kk = keys[wi]
        sink = np.zeros(nkb, bool)
        for a, bnd in protected_ranges:
            # first packed position whose key >= a; protected if it is < b and in the block
            pos = np.searchsorted(kk, a, side="left")
            for kb in range(nkb):
                p = max(pos, kstart[kb])
                sink[kb] |= bool(p < kend[kb] and kk[p] < bnd)
        lo = rows[wi, first] - local_tokens
        hi = rows[wi, last] + local_tokens
        for qb in range(nqb):
            pos = np.searchsorted(kk, lo[qb], side="left")
            p = np.maximum(pos, kstart)
            ok = p < kend
            hit = np.zeros(nkb, bool)
            hit[ok] = kk[p[ok]] <= hi[qb]
            out[wi, qb] = hit | sink
    return out


# ----------------------------------------------------------------------------
# Input helpers
# ----------------------------------------------------------------------------

def _as_f32(x) -> np.ndarray:
    if hasattr(x, "detach"):  # torch tensor (CPU); BF16 -> float32 is exact
        return x.detach().cpu().float().numpy()
    return np.asarray(x, dtype=np.float32)


def _as_bool(x) -> np.ndarray:
    if hasattr(x, "detach"):
        return x.detach().cpu().numpy().astype(bool)
    return np.asarray(x, dtype=bool)


def _chunks(seq, n):
    for i in range(0, len(seq), n):
        yield seq[i:i + n]
