"""Public BTHD interface (mirrors src/sol_attn_amd/attention.py:1-85).

Validation, keyword-only signatures, error messages and return types follow
the reference; the device work goes through the HIP C-ABI library
(``_native``).  There is no fallback: inputs off an AMD ROCm GPU are rejected.
"""

from dataclasses import dataclass
import math

import torch


@dataclass(frozen=True)
class SolStats:
    """Exact-block statistics (``attention.py:9-16``).

    ``exact_blocks`` is a device int32 tensor ``[batch, query_blocks, heads]``;
    ``density()`` synchronises to produce a Python float.  ``key_blocks`` is
    an int, or, for ragged indexed windows, a ``[batch]`` tensor of each
    window's key blocks; density is then the mean of exact / key blocks.
    """

    exact_blocks: torch.Tensor
    key_blocks: "int | torch.Tensor"

    def density(self) -> float:
        if isinstance(self.key_blocks, torch.Tensor):
            kb = self.key_blocks.to(self.exact_blocks.device, torch.float32).view(-1, 1, 1)
            return (self.exact_blocks.float() / kb).mean().item()
        return self.exact_blocks.float().mean().item() / self.key_blocks


def _validate(q, k, v, scale):
    """Input contract of ``attention.py:19-39``; returns the effective scale."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("Q/K/V must have BTHD rank-4 layout")
    if (k.shape != v.shape or q.shape[0] != k.shape[0]
            or q.shape[2:] != k.shape[2:] or min(q.shape + k.shape) <= 0):
        raise ValueError("Q/K/V batch, head and dimension shapes must agree and be nonempty")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError("Only BF16 Q/K/V are implemented")
    if q.shape[-1] not in (64, 128):
        raise ValueError("Only head dimensions 64 and 128 are implemented")
    if q.requires_grad or k.requires_grad or v.requires_grad:
        raise ValueError("Inference only: Q/K/V must not require gradients")
    for t in (q, k, v):
        strides = t.stride()
        if strides[-1] != 1 or min(strides) <= 0:
            raise ValueError("Q/K/V need positive strides and contiguous head dimension")
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("scale must be finite and positive")
    if (torch.version.hip is None or q.device.type != "cuda"
            or k.device != q.device or v.device != q.device):
        raise ValueError("The HIP backend requires Q/K/V on the same AMD ROCm GPU")
    return scale


# Key tokens one pooling call takes (SOL_MAX_KEY_TOKENS in
# include/sol_attn_amd.h, 2^19 key blocks).  The attention kernel routes longer
# key sequences in segments of 8,192 blocks, so this is the only bound.
MAX_KEY_TOKENS = 1 << 25


def _key_length(tokens):
    """Rejects key sequences beyond the pooling bound before any launch."""
    if tokens > MAX_KEY_TOKENS:
        raise ValueError(f"Key sequences longer than {MAX_KEY_TOKENS} tokens are not supported")


def _nonnegative_integer(name, value):
    if not isinstance(value, int) or isinstance(value, bool) or value < 0:
        raise ValueError(f"{name} must be a nonnegative integer")


def dense_attention(q, k, v, *, scale=None):
    """Noncausal BF16 attention over all keys, FP32 softmax/accumulation.

    Same-project dense control (``attention.py:47-55``), a CDNA4 flash-attention
    HIP kernel.
    """
    scale = _validate(q, k, v, scale)
    from ._native import launch_dense
    with torch.no_grad(), torch.cuda.device(q.device):
        return launch_dense(q, k, v, scale)


THRESHOLD_ESTIMATORS = ("diagonal_covariance", "full_covariance")


def _threshold_estimator(name):
    if name not in THRESHOLD_ESTIMATORS:
        raise ValueError("threshold_estimator must be 'diagonal_covariance' or 'full_covariance'")
    return name


QK_PRECISIONS = ("bf16", "int8")


def _qk_precision(name):
    if name not in QK_PRECISIONS:
        raise ValueError("qk_precision must be 'bf16' or 'int8'")
    return name


def sol_attention(q, k, v, *, beta=1.0, scale=None, local_blocks=1,
                  kv_sink_tokens=0, query_sink_tokens=0, return_stats=False,
                  threshold_estimator="diagonal_covariance", qk_precision="bf16"):
    """SOL-style noncausal attention (``attention.py:58-85``).

    Physical blocks hold 64 tokens.  Selected blocks use BF16 QK/PV with FP32
    softmax/accumulation; the others contribute their pooled key/value with
    weight ``exp(q . k_mean) * valid_len``.  Thresholds use the
    diagonal-covariance estimator (paper Eq. 15).  Prefix protection rounds
    outward to whole blocks.  beta=-inf forces every block exact; beta=+inf
    leaves only protected blocks exact.

    ``threshold_estimator="full_covariance"`` (not in the reference: the
    full-covariance threshold experiment of its roadmap) replaces
    ``sqrt(sum Qc^2 var)`` with ``sqrt(max(Qc^T cov Qc, 0))`` over the full
    covariance of the key centroids; the default keeps the reference's
    diagonal estimator.

    ``qk_precision="int8"`` (not in the reference: the INT8-QK experiment of
    its roadmap) computes the selected blocks' scores as ``s_q s_k (Q8 . K8)``
    on the INT8 matrix cores -- each query row quantised with one symmetric
    scale, each 64-key block of K with one -- while routing, the centroid
    terms and the P V product stay BF16.  The default keeps BF16 scores.
    """
    scale = _validate(q, k, v, scale)
    beta = float(beta)
    if math.isnan(beta):
        raise ValueError("beta must not be NaN")
    _threshold_estimator(threshold_estimator)
    _qk_precision(qk_precision)
    for name, value in (("local_blocks", local_blocks),
                        ("kv_sink_tokens", kv_sink_tokens),
                        ("query_sink_tokens", query_sink_tokens)):
        _nonnegative_integer(name, value)
    if kv_sink_tokens > k.shape[1] or query_sink_tokens > q.shape[1]:
        raise ValueError("Sink token counts must not exceed their sequence lengths")
    _key_length(k.shape[1])
    from ._native import launch_sol
    with torch.no_grad(), torch.cuda.device(q.device):
        out, counts = launch_sol(q, k, v, scale, beta, local_blocks,
                                 kv_sink_tokens, query_sink_tokens, return_stats,
                                 threshold_estimator=threshold_estimator, qk_precision=qk_precision)
    if return_stats:
        return out, SolStats(counts, (k.shape[1] + 63) // 64)
    return out
