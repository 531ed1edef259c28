"""Inference-only SOL-style BF16 routed attention, MI355X-native (gfx950 HIP kernels)."""

from .attention import SolStats, dense_attention, sol_attention
from .indexed import IndexedPlan, sol_attention_indexed

__all__ = ["SolStats", "dense_attention", "sol_attention", "IndexedPlan", "sol_attention_indexed"]
