"""Benchmark receipts in the reference's format (benchmarks/bench_attention.py:48-117).

CPU: the command-line contract (defaults, the three parser errors and their
messages) and the source hashes.  GPU: a two-case run whose JSON carries the
reference receipt's fields and a SOL result close to attention.
"""

import hashlib
import json
from pathlib import Path

import pytest

from sol_attn_amd import receipt
from sol_testlib import HAS_GPU

REFERENCE_CASE_FIELDS = {"shape", "timings", "exact_block_density", "finite", "relative_l2_vs_sdpa",
                         "max_abs_vs_sdpa", "cosine_vs_sdpa", "speedup_vs_sdpa", "speedup_vs_project_dense"}
REFERENCE_TOP_FIELDS = {"state", "scope", "started_unix", "torch", "hip", "triton", "device", "gpu_uuid",
                        "image", "configuration", "threshold_estimator", "source_sha256", "cases"}
TIMING_FIELDS = {"median_ms", "samples_ms", "min_ms", "max_ms", "cv_percent"}


def test_defaults_match_the_reference_command_line(tmp_path):
    args = receipt.parse_args(["--out", str(tmp_path / "r.json")])
    assert args.tokens == [1024, 4096] and args.heads == 4 and args.head_dim == 128
    assert args.beta == 1.0 and args.input == "block-smooth" and args.seed == 42
    assert args.repeats == 5 and args.trials == 5


@pytest.mark.parametrize("argv, message", [
    (["--tokens", "0"], "shape and repetition counts must be positive"),
    (["--trials", "0"], "shape and repetition counts must be positive"),
    (["--beta", "inf"], "Benchmark beta must be finite"),
])
def test_rejected_arguments(tmp_path, capsys, argv, message):
    with pytest.raises(SystemExit):
        receipt.parse_args(argv + ["--out", str(tmp_path / "r.json")])
    assert message in capsys.readouterr().err


def test_existing_receipt_is_never_overwritten(tmp_path, capsys):
    out = tmp_path / "r.json"
    out.write_text("{}")
    with pytest.raises(SystemExit):
        receipt.parse_args(["--out", str(out)])
    assert "Use a new output path" in capsys.readouterr().err
    assert out.read_text() == "{}"


def test_source_hashes_cover_kernels_and_header():
    hashes = receipt.source_hashes()
    names = {Path(k).name for k in hashes}
    assert {"attention.hip", "pool.hip", "capi.hip", "sol_attn_amd.h", "receipt.py"} <= names
    repo = Path(__file__).resolve().parents[1]
    for key, digest in hashes.items():
        assert hashlib.sha256((repo / key).read_bytes()).hexdigest() == digest


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")
def test_receipt_run(tmp_path):
    out = tmp_path / "receipt.json"
    report = receipt.main(["--tokens", "256", "300", "--heads", "2", "--repeats", "1", "--trials", "3",
                           "--out", str(out)])
    saved = json.loads(out.read_text())
    assert saved["state"] == "complete" == report["state"]
    assert REFERENCE_TOP_FIELDS <= set(saved)
    assert saved["configuration"]["tokens"] == [256, 300] and saved["library_abi"] >= 3
    assert len(saved["cases"]) == 2
    for case, n in zip(saved["cases"], (256, 300)):
        assert REFERENCE_CASE_FIELDS <= set(case)
        assert case["shape"] == [1, n, 2, 128]
        for name in ("project_dense", "sol_all_in"):
            assert TIMING_FIELDS <= set(case["timings"][name])
            assert len(case["timings"][name]["samples_ms"]) == 3
        assert case["finite"] and 0.0 < case["exact_block_density"] <= 1.0
        # Block-smooth inputs: SOL is close to full attention.
        assert case["relative_l2_vs_sdpa"] < 0.05 and case["cosine_vs_sdpa"] > 0.99
