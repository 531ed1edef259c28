"""Explicit indexed windows (mirrors src/sol_attn_amd/indexed.py:1-104).

``IndexedPlan.create`` builds the packed-block protection on the CPU with a
vectorised sorted-key search (O(W * blocks * log nk) instead of the
reference's per-block Python loop); ``sol_attention_indexed`` hands the plan's
row and key indices straight to the HIP kernels, which gather Q/K/V token rows
inside pooling and attention -- no gathered copies are materialised.

Beyond the reference's equal-length windows, a plan may hold windows with
different key counts (a list of key index vectors), which then run in one
call, and ``sol_attention_indexed(..., out=)`` stores each window's rows
straight into a full-sequence output (the scatter of a window adapter,
``integrations/vdn.py:67-74``).
"""

from dataclasses import dataclass
import math

import torch

from .attention import (SolStats, _key_length, _validate, _nonnegative_integer, _qk_precision,
                        _threshold_estimator)

BLOCK = 64


def _touches(keys, lo, hi_inclusive, lengths):
    """``[W, Q, NKB]`` bool: packed key block touches ``[lo, hi]`` (keys sorted per row).

    ``keys``: ``[W, nk]`` int64, non-decreasing, strictly increasing over each
    window's first ``lengths[w]`` entries (the rest repeat its last key);
    ``lo``/``hi_inclusive``: ``[W, Q]`` int64; blocks past a window's own keys
    never touch.
    """
    nk = keys.shape[1]
    nkb = (nk + BLOCK - 1) // BLOCK
    start = torch.arange(nkb, dtype=torch.int64) * BLOCK
    end = torch.minimum((start + BLOCK)[None, :], lengths[:, None])    # [W, NKB]
    first = torch.searchsorted(keys, lo.contiguous())                # first key >= lo
    pos = torch.maximum(first[..., None], start)                      # [W, Q, NKB]
    inside = pos < end[:, None, :]
    val = torch.gather(keys[:, None, :].expand(-1, pos.shape[1], -1), 2,
                       pos.clamp(max=nk - 1))
    return inside & (val <= hi_inclusive[..., None])


def _distinct(rows):
    """No row index appears twice in the plan (rows are sorted per window, so
    only different windows can share one)."""
    return bool(torch.unique(rows).numel() == rows.numel())


def _key_range(keys, lengths):
    """``(start, count)`` when every window's keys are one and the same
    contiguous token range (keys are strictly increasing over each window's
    first ``lengths[w]`` entries), else None."""
    if bool((lengths != lengths[0]).any()):
        return None
    count = int(lengths[0])
    ends = keys[:, [0, count - 1]].cpu()   # one transfer for a device plan
    start = int(ends[0, 0])
    if bool((ends[:, 0] != start).any()) or bool((ends[:, 1] - ends[:, 0] != count - 1).any()):
        return None
    return start, count


def _index_matrix(name, x, sequence_length, device=torch.device("cpu")):
    if (x.device != device or x.dtype != torch.int64 or x.ndim != 2
            or any(n == 0 for n in x.shape)):
        where = "CPU" if device.type == "cpu" else f"{device} (the rows' device)"
        raise ValueError(f"{name} must be a nonempty {where} int64 matrix")
    if bool((x < 0).any() or (x >= sequence_length).any()):
        raise ValueError(f"{name} index outside sequence")
    if bool((x[:, 1:] <= x[:, :-1]).any()):
        raise ValueError(f"{name} must be strictly increasing within each batch")


@dataclass(frozen=True)
class IndexedPlan:
    """Each window has independent, sorted Q rows and an identical allowed KV set.

    Build on the CPU and transfer once, outside repeated operator timing
    (``indexed.py:11-25``).  Holds indices and protection only, never
    activations.  No key outside ``keys`` enters pooling or attention.
    Blocks touching protected keys or the original-index local neighbourhood
    of a query block are exact; protection rounds outward to whole packed
    blocks.
    """

    rows: torch.Tensor
    keys: torch.Tensor
    protected_blocks: torch.Tensor
    sequence_length: int
    key_lengths: "torch.Tensor | None" = None  # int32 [W] for ragged windows, else None
    # Whether no query row appears in two windows (set by create(); None for a
    # plan built directly, checked on first use with out=).
    rows_distinct: "bool | None" = None
    # (start, count) when every window's keys are the same contiguous token
    # range start .. start + count - 1 (set by create(); None otherwise):
    # beta = -inf then runs the dense kernel on that range of K / V rows,
    # with no pooling pass and no block tiles.
    key_range: "tuple | None" = None

    @classmethod
    def create(cls, rows, keys, sequence_length, *, protected_ranges=(), local_tokens=64):
        """Validate indices and compute ``protected_blocks`` (``indexed.py:27-62``).

        ``keys`` is an int64 ``[W, nk]`` matrix (every window sees ``nk``
        keys, as in the reference) or a sequence of W int64 vectors of any
        nonzero lengths (ragged windows, run in one call): the plan then pads
        ``keys`` to the longest window with each window's last key and records
        ``key_lengths``; padded entries are never read.

        With ``rows`` and ``keys`` on the CPU (the reference's contract) the
        protection is computed on the CPU.  With both on one AMD GPU the plan
        is built there: the same checks run on the device, the protection
        comes from the ``sol_plan_protection`` kernel, and the plan is
        returned on that device (no transfer needed).
        """
        _nonnegative_integer("local_tokens", local_tokens)
        _nonnegative_integer("sequence_length", sequence_length)
        if sequence_length == 0:
            raise ValueError("sequence_length must be positive")
        ragged = isinstance(keys, (list, tuple))
        dev = rows.device if isinstance(rows, torch.Tensor) and rows.device.type == "cuda" \
            else torch.device("cpu")
        _index_matrix("rows", rows, sequence_length, dev)
        if ragged:
            if len(keys) != rows.shape[0]:
                raise ValueError("rows and keys must have the same batch size")
            for x in keys:
                if not isinstance(x, torch.Tensor) or x.ndim != 1:
                    raise ValueError("ragged keys must be 1-D int64 vectors on the rows' device")
                _index_matrix("keys", x[None], sequence_length, dev)
            lengths = torch.tensor([x.numel() for x in keys], dtype=torch.int64)
            nk = int(lengths.max())
            padded = torch.stack([torch.cat((x, x[-1:].expand(nk - x.numel()))) for x in keys])
        else:
            _index_matrix("keys", keys, sequence_length, dev)
            if rows.shape[0] != keys.shape[0]:
                raise ValueError("rows and keys must have the same batch size")
            padded = keys
            lengths = torch.full((keys.shape[0],), keys.shape[1], dtype=torch.int64)
        ranges = tuple(protected_ranges)
        for a, b in ranges:
            if not (isinstance(a, int) and isinstance(b, int)
                    and 0 <= a < b <= sequence_length):
                raise ValueError("Invalid protected key range")
        rows = rows.clone().contiguous()
        keys = padded.clone().contiguous()
        distinct = _distinct(rows)
        key_range = _key_range(keys, lengths)
        if dev.type == "cuda":
            from ._native import plan_protection
            key_lengths = lengths.to(torch.int32).to(dev) if ragged else None
            with torch.cuda.device(dev):
                protection = plan_protection(rows, keys, key_lengths, local_tokens, ranges)
            return cls(rows, keys, protection, sequence_length, key_lengths, distinct, key_range)
        w, nq = rows.shape
        nqb = (nq + BLOCK - 1) // BLOCK
        first = rows[:, ::BLOCK]                                        # [W, NQB]
        last = rows[:, torch.clamp(torch.arange(nqb) * BLOCK + BLOCK, max=nq) - 1]
        protection = _touches(keys, first - local_tokens, last + local_tokens, lengths)
        for a, b in ranges:
            lo = torch.full((w, 1), a, dtype=torch.int64)
            hi = torch.full((w, 1), b - 1, dtype=torch.int64)
            protection |= _touches(keys, lo, hi, lengths)
        return cls(rows, keys, protection.contiguous(), sequence_length,
                   lengths.to(torch.int32) if ragged else None, distinct, key_range)

    def to(self, device):
        return IndexedPlan(self.rows.to(device), self.keys.to(device),
                           self.protected_blocks.to(device), self.sequence_length,
                           None if self.key_lengths is None else self.key_lengths.to(device),
                           self.rows_distinct, self.key_range)


def sol_attention_indexed(q, k, v, plan, *, beta=1.0, scale=None, return_stats=False, out=None,
                          threshold_estimator="diagonal_covariance", qk_precision="bf16"):
    """BF16 NHD inputs -> ``[windows, query_rows, heads, D]`` (``indexed.py:69-104``).

    Window ``w`` attends its query rows ``plan.rows[w]`` to its keys
    ``plan.keys[w]`` (its first ``plan.key_lengths[w]`` for a ragged plan)
    with no local band and the plan's protection.  The row gathers run inside
    the HIP kernels.  Plan creation and transfer are one-time setup costs.

    ``out``: an optional contiguous BF16 ``[N, H, D]`` tensor on the Q device
    (N = sequence length).  Query row ``plan.rows[w, i]`` of the result is then
    stored directly at ``out[plan.rows[w, i]]`` -- the ``out[rows] = result``
    step of a window adapter fused into the kernel's store -- and ``out`` is
    returned; other rows of ``out`` are left as they were.  Rows shared by
    two windows of one plan would race, so ``out=`` is rejected for such a
    plan.  The kernels clamp index entries into the sequence and skip output
    rows outside it, so a plan whose tensors were changed after ``create``
    cannot make them access memory outside Q/K/V or ``out``.

    ``threshold_estimator``, ``qk_precision``: as in :func:`sol_attention`.
    """
    if any(t.ndim != 3 for t in (q, k, v)) or q.shape != k.shape or k.shape != v.shape:
        raise ValueError("Indexed Q/K/V must have matching NHD shapes")
    scale = _validate(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), scale)
    if not isinstance(plan, IndexedPlan):
        raise ValueError("An explicit IndexedPlan is required")
    if plan.sequence_length != q.shape[0]:
        raise ValueError("Plan sequence length does not match Q/K/V")
    lengths = plan.key_lengths
    if any(x.device != q.device for x in (plan.rows, plan.keys, plan.protected_blocks)) or (
            lengths is not None and lengths.device != q.device):
        raise ValueError("Transfer the plan to the Q/K/V device first")
    b, nq = plan.rows.shape
    if (plan.rows.ndim != 2 or plan.keys.ndim != 2 or plan.keys.shape[0] != b
            or b <= 0 or nq <= 0 or plan.keys.shape[1] <= 0
            or plan.rows.dtype != torch.int64 or plan.keys.dtype != torch.int64
            or plan.protected_blocks.dtype != torch.bool
            or plan.protected_blocks.shape != (b, (nq + 63) // 64, (plan.keys.shape[1] + 63) // 64)
            or any(not x.is_contiguous() for x in (plan.rows, plan.keys, plan.protected_blocks))
            or (lengths is not None and (lengths.dtype != torch.int32 or lengths.shape != (b,)
                                         or not lengths.is_contiguous()))):
        raise ValueError("Invalid indexed descriptor; use IndexedPlan.create")
    if out is not None and (out.dtype != torch.bfloat16 or out.shape != q.shape
                            or not out.is_contiguous() or out.device != q.device):
        raise ValueError("out must be a contiguous BF16 tensor shaped like Q on its device")
    if out is not None and not (plan.rows_distinct if plan.rows_distinct is not None
                                else _distinct(plan.rows)):
        raise ValueError("out= needs a plan whose windows share no query row")
    _key_length(plan.keys.shape[1])
    beta = float(beta)
    if math.isnan(beta):
        raise ValueError("beta must not be NaN")
    _threshold_estimator(threshold_estimator)
    _qk_precision(qk_precision)
    from ._native import launch_dense, launch_sol
    if beta == -math.inf and qk_precision == "bf16" and plan.key_range is not None:
        # Every block exact over one contiguous key range: the dense kernel on
        # those K / V rows, queries gathered and (with out=) results scattered
        # inside it -- no pooling pass, no block tiles, no protection needed.
        start, count = plan.key_range
        with torch.no_grad(), torch.cuda.device(q.device):
            result = launch_dense(q, k[start:start + count], v[start:start + count], scale,
                                  rows=plan.rows, out=out)
        if return_stats:
            nkb = (plan.keys.shape[1] + 63) // 64
            counts = torch.full((b, (nq + 63) // 64, q.shape[1]), nkb, device=q.device, dtype=torch.int32)
            return result, SolStats(counts, nkb)
        return result
    with torch.no_grad(), torch.cuda.device(q.device):
        result, counts = launch_sol(q, k, v, scale, beta, -1, 0, 0, return_stats,
                                    plan.protected_blocks, rows=plan.rows, keys=plan.keys,
                                    key_lengths=lengths, out=out,
                                    threshold_estimator=threshold_estimator, qk_precision=qk_precision)
    if return_stats:
        key_blocks = ((plan.keys.shape[1] + 63) // 64 if lengths is None
                      else (lengths.to(torch.int64) + 63) // 64)
        return result, SolStats(counts, key_blocks)
    return result
