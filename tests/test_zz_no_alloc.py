"""The allocation-free entry point (sol_attention_noalloc), called through the
C-ABI, against the allocating path (sol_pool_kv + sol_attention_fwd through
_native.launch_sol, as two calls): bit-identical outputs and exact-block
counts on two calls in a row, the second smaller, so the shared device
workspace is reused."""

import ctypes
import math
import os
import subprocess
import sys

import pytest
import torch

from sol_attn_amd import _native
from sol_testlib import HAS_GPU, block_smooth

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="AMD ROCm GPU required")]


def _strides(x):
    s = x.stride()
    return (ctypes.c_int64 * 3)(s[0], s[1], s[2])


def _noalloc(q, k, v, beta, local, kv_sink, q_sink, out, counts):
    lib = _native.library()
    b, tq, h, d = q.shape
    rc = lib.sol_attention_noalloc(q.data_ptr(), _strides(q), k.data_ptr(), _strides(k), v.data_ptr(),
                                   _strides(v), b, tq, k.shape[1], h, d, d ** -0.5, beta, local, kv_sink,
                                   q_sink, out.data_ptr(), None if counts is None else counts.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.sol_last_error().decode()


# (batch, query tokens, key tokens, heads, head_dim, beta, local, kv sink, q sink);
# the second case is smaller than the first, the third exercises beta = -inf,
# the fourth fewer keys than one block (block tiles in the workspace), the
# fifth query sinks split by key range (split workspace in the scratch array),
# the sixth one launch that pools its keys itself (no workspace at all).
CASES = [(2, 4096, 4096, 16, 128, 1.0, 1, 128, 128),
         (1, 700, 1300, 3, 64, 0.5, 0, 64, 0),
         (1, 500, 900, 2, 128, -math.inf, 1, 0, 0),
         (1, 130, 40, 2, 64, 1.0, 1, 0, 0),
         (1, 4096, 4096, 4, 128, 1.0, 1, 64, 128),
         (1, 1024, 1024, 8, 64, 1.0, 1, 128, 128)]


def test_noalloc_matches_the_allocating_path_on_consecutive_calls(monkeypatch):
    # The reference path as two C-ABI calls (not sol_attention_all_in, which
    # shares the noalloc entry point's code).
    monkeypatch.setattr(_native, "ALL_IN", False)
    for i, (b, tq, tk, h, d, beta, local, kvs, qs) in enumerate(CASES):
        print(f"case {i}: B{b} Tq{tq} Tk{tk} H{h} D{d} beta {beta}", flush=True)
        q = block_smooth(b, tq, h, d, seed=10 + i, device="cuda")
        k = block_smooth(b, tk, h, d, seed=20 + i, device="cuda")
        v = block_smooth(b, tk, h, d, seed=30 + i, device="cuda")
        with torch.no_grad():
            ref, ref_counts = _native.launch_sol(q, k, v, d ** -0.5, beta, local, kvs, qs, True)
        out = torch.full_like(q, 7.0)
        counts = torch.full((b, -(-tq // 64), h), -5, device="cuda", dtype=torch.int32)
        _noalloc(q, k, v, beta, local, kvs, qs, out, counts)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"case {i}"
        assert torch.equal(counts, ref_counts), f"case {i}"


_FIRST_CALL = r"""
import ctypes
import torch
from sol_attn_amd import _native
from sol_testlib import block_smooth
b, tq, tk, h, d = 1, 4096, 4096, 4, 128
q = block_smooth(b, tq, h, d, seed=41, device="cuda")
k = block_smooth(b, tk, h, d, seed=42, device="cuda")
v = block_smooth(b, tk, h, d, seed=43, device="cuda")
torch.cuda.synchronize()
lib = _native.library()
st = lambda x: (ctypes.c_int64 * 3)(*x.stride()[:3])
out = torch.full_like(q, 7.0)
rc = lib.sol_attention_noalloc(q.data_ptr(), st(q), k.data_ptr(), st(k), v.data_ptr(), st(v), b, tq, tk, h, d,
                               d ** -0.5, 1.0, 1, 64, 128, out.data_ptr(), None,
                               torch.cuda.current_stream().cuda_stream)
assert rc == 0, lib.sol_last_error().decode()
torch.cuda.synchronize()
_native.ALL_IN = False
ref, _ = _native.launch_sol(q, k, v, d ** -0.5, 1.0, 1, 64, 128, False)
assert torch.equal(out, ref)
print("first-call noalloc ok", flush=True)
"""


def test_noalloc_as_the_first_call_of_a_process():
    # The entry point is the process's first SOL launch: the device array is
    # looked up and the kernels (split sink tiles included) loaded on it.
    here = os.path.dirname(os.path.abspath(__file__))
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([here, os.path.join(here, "..", "solattn-amd_amd"),
                                         env.get("PYTHONPATH", "")])
    print("fresh process: noalloc first", flush=True)
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL], env=env, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "first-call noalloc ok" in res.stdout
