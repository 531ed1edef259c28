"""Explicit equal-length indexed windows (mirrors src/sol_attn_amd/indexed.py:1-104).

``IndexedPlan.create`` builds the packed-block protection on the CPU with a
vectorised sorted-key search (O(W * blocks * log nk) instead of the
reference's per-block Python loop); ``sol_attention_indexed`` hands the plan's
row and key indices straight to the HIP kernels, which gather Q/K/V token rows
inside pooling and attention -- no gathered copies are materialised.
"""

from dataclasses import dataclass
import math

import torch

from .attention import SolStats, _validate, _nonnegative_integer

BLOCK = 64


def _touches(keys, lo, hi_inclusive, nk):
    """``[W, Q, NKB]`` bool: packed key block touches ``[lo, hi]`` (keys sorted per row).

    ``keys``: ``[W, nk]`` int64 strictly increasing; ``lo``/``hi_inclusive``:
    ``[W, Q]`` int64.
    """
    nkb = (nk + BLOCK - 1) // BLOCK
    start = torch.arange(nkb, dtype=torch.int64) * BLOCK
    end = torch.clamp(start + BLOCK, max=nk)
    first = torch.searchsorted(keys, lo.contiguous())                # first key >= lo
    pos = torch.maximum(first[..., None], start)                      # [W, Q, NKB]
    inside = pos < end
    val = torch.gather(keys[:, None, :].expand(-1, pos.shape[1], -1), 2,
                       pos.clamp(max=nk - 1))
    return inside & (val <= hi_inclusive[..., None])


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

    @classmethod
    def create(cls, rows, keys, sequence_length, *, protected_ranges=(), local_tokens=64):
        """Validate indices and compute ``protected_blocks`` (``indexed.py:27-62``)."""
        _nonnegative_integer("local_tokens", local_tokens)
        _nonnegative_integer("sequence_length", sequence_length)
        if sequence_length == 0:
            raise ValueError("sequence_length must be positive")
        for name, x in (("rows", rows), ("keys", keys)):
            if (x.device.type != "cpu" or x.dtype != torch.int64 or x.ndim != 2
                    or any(n == 0 for n in x.shape)):
                raise ValueError(f"{name} must be a nonempty CPU int64 matrix")
            if bool((x < 0).any() or (x >= sequence_length).any()):
                raise ValueError(f"{name} index outside sequence")
            if bool((x[:, 1:] <= x[:, :-1]).any()):
                raise ValueError(f"{name} must be strictly increasing within each batch")
        if rows.shape[0] != keys.shape[0]:
            raise ValueError("rows and keys must have the same batch size")
        ranges = tuple(protected_ranges)
        for a, b in ranges:
            if not (isinstance(a, int) and isinstance(b, int)
                    and 0 <= a < b <= sequence_length):
                raise ValueError("Invalid protected key range")
        rows = rows.clone().contiguous()
        keys = keys.clone().contiguous()
        w, nq = rows.shape
        nk = keys.shape[1]
        nqb = (nq + BLOCK - 1) // BLOCK
        first = rows[:, ::BLOCK]                                        # [W, NQB]
        last = rows[:, torch.clamp(torch.arange(nqb) * BLOCK + BLOCK, max=nq) - 1]
        protection = _touches(keys, first - local_tokens, last + local_tokens, nk)
        for a, b in ranges:
            lo = torch.full((w, 1), a, dtype=torch.int64)
            hi = torch.full((w, 1), b - 1, dtype=torch.int64)
            protection |= _touches(keys, lo, hi, nk)
        return cls(rows, keys, protection.contiguous(), sequence_length)

    def to(self, device):
        return IndexedPlan(self.rows.to(device), self.keys.to(device),
                           self.protected_blocks.to(device), self.sequence_length)


def sol_attention_indexed(q, k, v, plan, *, beta=1.0, scale=None, return_stats=False):
    """BF16 NHD inputs -> ``[windows, query_rows, heads, D]`` (``indexed.py:69-104``).

    Window ``w`` attends its query rows ``plan.rows[w]`` to its keys
    ``plan.keys[w]`` with no local band and the plan's protection.  The row
    gathers run inside the HIP kernels.  Plan creation and transfer are
    one-time setup costs.  Output is not scattered back.
    """
    if any(t.ndim != 3 for t in (q, k, v)) or q.shape != k.shape or k.shape != v.shape:
        raise ValueError("Indexed Q/K/V must have matching NHD shapes")
    scale = _validate(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), scale)
    if not isinstance(plan, IndexedPlan):
        raise ValueError("An explicit IndexedPlan is required")
    if plan.sequence_length != q.shape[0]:
        raise ValueError("Plan sequence length does not match Q/K/V")
    if any(x.device != q.device for x in (plan.rows, plan.keys, plan.protected_blocks)):
        raise ValueError("Transfer the plan to the Q/K/V device first")
    b, nq = plan.rows.shape
    if (plan.rows.ndim != 2 or plan.keys.ndim != 2 or plan.keys.shape[0] != b
            or b <= 0 or nq <= 0 or plan.keys.shape[1] <= 0
            or plan.rows.dtype != torch.int64 or plan.keys.dtype != torch.int64
            or plan.protected_blocks.dtype != torch.bool
            or plan.protected_blocks.shape != (b, (nq + 63) // 64, (plan.keys.shape[1] + 63) // 64)
            or any(not x.is_contiguous() for x in (plan.rows, plan.keys, plan.protected_blocks))):
        raise ValueError("Invalid indexed descriptor; use IndexedPlan.create")
    beta = float(beta)
    if math.isnan(beta):
        raise ValueError("beta must not be NaN")
    from ._native import launch_sol
    with torch.no_grad(), torch.cuda.device(q.device):
        out, counts = launch_sol(q, k, v, scale, beta, -1, 0, 0, return_stats,
                                 plan.protected_blocks, rows=plan.rows, keys=plan.keys)
    if return_stats:
        return out, SolStats(counts, (plan.keys.shape[1] + 63) // 64)
    return out
