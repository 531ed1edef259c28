"""Shared fixtures and tolerance helpers for the SOL tests."""

import numpy as np
import torch

HAS_GPU = torch.version.hip is not None and torch.cuda.is_available()


def tensors(nq=193, nk=317, d=64, b=1, h=2, device="cpu", strided=False, seed=42):
    """Seeded BF16 BTHD Q/K/V (shape of test_attention.py:13-17); strided views
    take every other head of a 2H allocation."""
    gen = torch.Generator(device=device).manual_seed(seed)
    xs = [torch.randn((b, n, h * (2 if strided else 1), d), generator=gen,
                      device=device, dtype=torch.bfloat16) for n in (nq, nk, nk)]
    return tuple(x[:, :, ::2] if strided else x for x in xs)


def block_smooth(b, t, h, d, seed, noise=0.1, device="cpu"):
    """Per 64-token block and head a centre ~N(0,1)^D plus noise * N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    nb = (t + 63) // 64
    centres = torch.randn((b, nb, h, d), generator=g)
    x = centres.repeat_interleave(64, 1)[:, :t] + noise * torch.randn((b, t, h, d), generator=g)
    return x.to(torch.bfloat16).to(device)


def to_np(x):
    return x.detach().float().cpu().numpy()


def assert_close(actual, expected):
    """Reference tolerance (test_attention.py:20-24) plus the max-abs 2e-2 /
    rel-L2 1e-2 bar of the port's parity contract."""
    a = torch.as_tensor(np.asarray(actual, dtype=np.float32)) if not torch.is_tensor(actual) else actual.float().cpu()
    e = torch.as_tensor(np.asarray(expected, dtype=np.float32)) if not torch.is_tensor(expected) else expected.float().cpu()
    assert torch.isfinite(a).all()
    torch.testing.assert_close(a, e, atol=0.012, rtol=0.025)
    rel = (a - e).norm() / e.norm().clamp_min(1e-8)
    assert rel < 0.008, f"relative L2 {rel:.5f}"
    assert (a - e).abs().max() <= 2e-2
