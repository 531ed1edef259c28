"""The ctypes binding shown in INTEGRATION.md (the one a reference maintainer
would drop next to kernels.py) is executed as written: its declarations must
match the library's exports, and on the GPU its launch_sol / launch_dense must
give the package's results bit for bit."""

import ctypes
import math
import os
import re

import pytest
import torch

from sol_attn_amd import _native, dense_attention, sol_attention
from sol_testlib import HAS_GPU, tensors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def stub():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    code = re.search(r"```python\n(.*?)```", text, re.S).group(1)
    assert 'LIB_PATH = "libsol_attn_amd.so"' in code
    code = code.replace('LIB_PATH = "libsol_attn_amd.so"', f"LIB_PATH = {_native.LIB_PATH!r}")
    ns = {}
    exec(compile(code, "INTEGRATION.md", "exec"), ns)
    return ns


def test_stub_declarations_match_the_library():
    if not os.path.exists(_native.LIB_PATH):
        pytest.skip("libsol_attn_amd.so not built")
    lib = stub()["_lib"]
    for name in ("sol_pool_sizes", "sol_pool_kv", "sol_attention_fwd", "sol_dense_fwd",
                 "sol_pair_workspace_size", "sol_pair_strides"):
        ours = [t for t in _native._SIGNATURES[name][0]]
        theirs = list(getattr(lib, name).argtypes)
        assert theirs == ours, name


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")
@pytest.mark.parametrize("nq,nk,d", [(300, 517, 128), (193, 40, 64), (4096, 4096, 64)])
def test_stub_launches_equal_the_package(nq, nk, d):
    ns = stub()
    q, k, v = tensors(nq=nq, nk=nk, d=d, b=2, h=2, device="cuda", strided=True)
    scale = d ** -0.5
    sinks = min(64, nk)
    for beta in (1.0, 0.0, -math.inf, math.inf):
        ref, stats = sol_attention(q, k, v, beta=beta, kv_sink_tokens=sinks, return_stats=True)
        out, counts = ns["launch_sol"](q, k, v, scale, beta, 1, sinks, 0, True)
        assert torch.equal(out, ref), beta
        assert torch.equal(counts, stats.exact_blocks), beta
    assert torch.equal(ns["launch_dense"](q, k, v, scale), dense_attention(q, k, v))
