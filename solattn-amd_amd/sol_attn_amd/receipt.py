"""Benchmark receipts in the reference's JSON format.

Mirrors the receipt that `benchmarks/bench_attention.py:48-117` writes, so
that results from this package line up field by field with the reference's
receipts: one JSON document per run, rewritten after every case, with the
state ("running" / "complete" / "failed"), the environment, the
configuration, SHA-256 hashes of the sources, and per case the timings
(median, samples, min, max, CV) of torch SDPA, the in-house dense kernel and
SOL all-in, the exact-block density, and the error of SOL against SDPA.

Differences, all additive or forced by the platform:
  * there is no Triton: "triton" is null and "backend" / "library_abi" name
    the HIP library; the hashed sources include the HIP kernels and the C
    header;
  * torch SDPA runs only on its fused backends (flash / memory-efficient).
    Its math fallback computes BF16 batched products on transposed views,
    which this package never launches; if no fused backend takes the shape,
    the case records "torch_sdpa_auto": null and the error fields compare
    against an FP32 SDPA of the same inputs instead ("error_reference").

Usage: python -m sol_attn_amd.receipt --out receipts/run.json [--tokens 1024 4096]
       [--heads 4] [--head-dim 128] [--beta 1.0] [--input block-smooth|random]
       [--seed 42] [--repeats 5] [--trials 5]
"""

import argparse
import hashlib
import json
import math
import os
from pathlib import Path
import statistics
import time

import torch
import torch.nn.functional as F

from . import _native
from .attention import dense_attention, sol_attention

_PACKAGE = Path(__file__).resolve().parent


def parse_args(argv=None):
    """The reference's command line (bench_attention.py:49-65), same checks and messages."""
    parser = argparse.ArgumentParser(description="All-in kernel benchmark receipt; synthetic inputs only.")
    parser.add_argument("--tokens", type=int, nargs="+", default=[1024, 4096])
    parser.add_argument("--heads", type=int, default=4)
    parser.add_argument("--head-dim", type=int, choices=[64, 128], default=128)
    parser.add_argument("--beta", type=float, default=1.0)
    parser.add_argument("--input", choices=["random", "block-smooth"], default="block-smooth")
    parser.add_argument("--seed", type=int, default=42)
    parser.add_argument("--repeats", type=int, default=5)
    parser.add_argument("--trials", type=int, default=5)
    parser.add_argument("--out", type=Path, required=True)
    args = parser.parse_args(argv)
    if min(*args.tokens, args.heads, args.repeats, args.trials) <= 0:
        parser.error("shape and repetition counts must be positive")
    if not math.isfinite(args.beta):
        parser.error("Benchmark beta must be finite; dense-limit cases are covered by tests")
    if args.out.exists():
        parser.error("Use a new output path to preserve experiment receipts")
    return args


def source_hashes():
    """SHA-256 of every source the measured path is built from, keyed by path."""
    root = _PACKAGE.parent
    files = sorted(_PACKAGE.glob("*.py")) + sorted((_PACKAGE / "csrc").glob("*.hip")) + \
        sorted((_PACKAGE / "csrc").glob("*.h"))
    header = root.parent / "include" / "sol_attn_amd.h"
    if header.exists():
        files.append(header)
    return {str(p.relative_to(root.parent) if header.exists() else p.relative_to(root)):
            hashlib.sha256(p.read_bytes()).hexdigest() for p in files}


def make_inputs(tokens, heads, dimension, seed, kind, device):
    """Seeded BF16 [1, T, H, D] Q, K, V drawn on the device: iid normal, or
    block-smooth (per-block centres repeated over the block's 64 tokens plus
    0.05 x the iid draw), in the reference's draw order."""
    gen = torch.Generator(device=device).manual_seed(seed)

    def draw(shape):
        return torch.randn(shape, device=device, dtype=torch.bfloat16, generator=gen)

    q, k, v = (draw((1, tokens, heads, dimension)) for _ in range(3))
    if kind == "block-smooth":
        for x in (q, k, v):
            centres = draw((1, -(-tokens // 64), heads, dimension))
            x.copy_(centres.repeat_interleave(64, dim=1)[:, :tokens] + 0.05 * x)
    return q, k, v


def _summary(samples):
    return {"median_ms": statistics.median(samples), "samples_ms": samples, "min_ms": min(samples),
            "max_ms": max(samples), "cv_percent": statistics.pstdev(samples) / statistics.mean(samples) * 100}


def _event_ms(fn, repeats):
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(repeats):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / repeats


def _fused_sdpa(q, k, v):
    """torch SDPA in [B, T, H, D] on its fused backends only (None if none takes the shape)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    qt, kt, vt = (x.transpose(1, 2) for x in (q, k, v))
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            F.scaled_dot_product_attention(qt, kt, vt)
    except RuntimeError:
        return None

    def run():
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(qt, kt, vt).transpose(1, 2)
    return run


def _fp32_sdpa(q, k, v):
    """FP32 attention as the error reference when no fused BF16 SDPA exists.
    Per head, on contiguous operands (no transposed-view batched products)."""
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    scale = q.shape[-1] ** -0.5
    for h in range(q.shape[2]):
        qh = q[0, :, h].float().contiguous()
        kh = k[0, :, h].float().t().contiguous()
        vh = v[0, :, h].float().contiguous()
        out[0, :, h] = torch.softmax((qh @ kh) * scale, dim=-1) @ vh
    return out


def run_case(args, n, device):
    q, k, v = make_inputs(n, args.heads, args.head_dim, args.seed, args.input, device)
    sdpa = _fused_sdpa(q, k, v)
    functions = {"project_dense": lambda: dense_attention(q, k, v),
                 "sol_all_in": lambda: sol_attention(q, k, v, beta=args.beta)}
    if sdpa is not None:
        functions = {"torch_sdpa_auto": sdpa, **functions}
    for fn in functions.values():  # warm-up
        for _ in range(3):
            fn()
    torch.cuda.synchronize()
    samples = {name: [] for name in functions}
    names = list(functions)
    for trial in range(args.trials):  # rotate the order between trials
        for name in names[trial % len(names):] + names[:trial % len(names)]:
            samples[name].append(_event_ms(functions[name], args.repeats))
    timings = {name: _summary(xs) for name, xs in samples.items()}
    actual, stats = sol_attention(q, k, v, beta=args.beta, return_stats=True)
    reference = sdpa().float() if sdpa is not None else _fp32_sdpa(q, k, v)
    delta = actual.float() - reference
    sol_ms = timings["sol_all_in"]["median_ms"]
    case = {"shape": list(q.shape), "timings": timings, "exact_block_density": stats.density(),
            "finite": bool(torch.isfinite(actual).all()),
            "relative_l2_vs_sdpa": (delta.norm() / reference.norm().clamp_min(1e-8)).item(),
            "max_abs_vs_sdpa": delta.abs().max().item(),
            "cosine_vs_sdpa": F.cosine_similarity(actual.float().flatten(), reference.flatten(), dim=0).item(),
            "speedup_vs_sdpa": (timings["torch_sdpa_auto"]["median_ms"] / sol_ms) if sdpa is not None else None,
            "speedup_vs_project_dense": timings["project_dense"]["median_ms"] / sol_ms,
            "error_reference": "torch_sdpa_auto" if sdpa is not None else "fp32_attention"}
    if sdpa is None:
        case["timings"]["torch_sdpa_auto"] = None
    return case


def main(argv=None):
    args = parse_args(argv)
    device = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(0)
    report = {"state": "running", "scope": "All-in GPU-event latency, warm; synthetic data only",
              "started_unix": time.time(), "torch": torch.__version__, "hip": torch.version.hip,
              "triton": None, "backend": "HIP (gfx950)", "library_abi": _native.library().sol_abi_version(),
              "device": str(props), "gpu_uuid": os.environ.get("ROCR_VISIBLE_DEVICES"),
              "image": os.environ.get("SOL_ROCM_IMAGE"), "configuration": vars(args).copy(),
              "threshold_estimator": "diagonal_covariance", "source_sha256": source_hashes(), "cases": []}
    report["configuration"]["out"] = str(args.out)
    args.out.parent.mkdir(parents=True, exist_ok=True)

    def save():
        args.out.write_text(json.dumps(report, indent=2, allow_nan=False) + "\n")

    save()
    try:
        with torch.no_grad():
            for n in args.tokens:
                case = run_case(args, n, device)
                report["cases"].append(case)
                save()
                print(json.dumps(case), flush=True)
        report["state"] = "complete"
        save()
    except Exception as exc:
        report.update(state="failed", error=repr(exc))
        save()
        raise
    return report


if __name__ == "__main__":
    main()
