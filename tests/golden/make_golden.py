"""Write golden vectors from the reference's own CPU oracle.

Run in the build container only (the reference checkout is not present where
the tests run):

    python tests/golden/make_golden.py /root/reference

It imports ``sol_attn_amd.reference.sol_reference`` (``reference.py:18-66``)
and ``sol_attn_amd.indexed.IndexedPlan.create`` (``indexed.py:27-62``) from the
given checkout, evaluates them on seeded BF16 fixtures, and stores inputs
(BF16 bit patterns) and outputs in ``reference_vectors.npz`` beside this
script.  These pin the finite-beta routing and the plan builder on arbitrary
inputs, which closed forms do not cover.  Nothing from the reference is copied:
only its inputs and outputs.
"""

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def bits(x):
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def main(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "src"))
    from sol_attn_amd.reference import sol_reference
    from sol_attn_amd.indexed import IndexedPlan

    out = {}

    # Case A: the reference test fixture shape (193 x 317, H=2, D=64), seed 42.
    g = torch.Generator().manual_seed(42)
    qa, ka, va = [torch.randn((1, n, 2, 64), generator=g, dtype=torch.bfloat16)
                  for n in (193, 317, 317)]
    out["A_q"], out["A_k"], out["A_v"] = bits(qa), bits(ka), bits(va)
    cases_a = [
        ("b1", dict(beta=1.0)),
        ("b0", dict(beta=0.0)),
        ("bhalf_l0", dict(beta=0.5, local_blocks=0)),
        ("bneg_l2", dict(beta=-0.75, local_blocks=2)),
        ("b1_sinks", dict(beta=1.0, kv_sink_tokens=65, query_sink_tokens=1, local_blocks=0)),
        ("binf_sinks", dict(beta=math.inf, kv_sink_tokens=65, query_sink_tokens=1, local_blocks=0)),
        ("b2_scale", dict(beta=2.0, scale=0.05)),
    ]
    for name, kw in cases_a:
        o, c = sol_reference(qa, ka, va, **kw)
        out[f"A_{name}_out"] = o.numpy()
        out[f"A_{name}_counts"] = c.numpy()

    # Case B: batch 2, D=128, ragged tails on both sides, seed 5.
    g = torch.Generator().manual_seed(5)
    qb_, kb_, vb_ = [torch.randn((2, n, 1, 128), generator=g, dtype=torch.bfloat16)
                     for n in (100, 150, 150)]
    out["B_q"], out["B_k"], out["B_v"] = bits(qb_), bits(kb_), bits(vb_)
    for name, kw in [("b1", dict(beta=1.0)), ("b0", dict(beta=0.0))]:
        o, c = sol_reference(qb_, kb_, vb_, **kw)
        out[f"B_{name}_out"] = o.numpy()
        out[f"B_{name}_counts"] = c.numpy()

    # Case C: block-smooth input (centre + 0.1 noise), seed 11, with a random
    # plan protection mask and no local band (the indexed-path convention).
    g = torch.Generator().manual_seed(11)
    tq, tk = 160, 300
    xs = []
    for n in (tq, tk, tk):
        centres = torch.randn((1, (n + 63) // 64, 2, 64), generator=g)
        noise = torch.randn((1, n, 2, 64), generator=g)
        xs.append((centres.repeat_interleave(64, 1)[:, :n] + 0.1 * noise).to(torch.bfloat16))
    prot = torch.rand((1, 3, 5), generator=g) < 0.3
    out["C_q"], out["C_k"], out["C_v"] = (bits(x) for x in xs)
    out["C_prot"] = prot.numpy()
    o, c = sol_reference(*xs, beta=1.0, local_blocks=-1, protected_blocks=prot)
    out["C_b1_out"], out["C_b1_counts"] = o.numpy(), c.numpy()

    # Case D: IndexedPlan.create on seeded random windows.
    rng = np.random.default_rng(3)
    for i, (w, nq, nk, seq, local) in enumerate([(3, 150, 200, 1000, 64), (2, 70, 333, 700, 0),
                                                 (4, 64, 128, 512, 17)]):
        rows = np.stack([np.sort(rng.choice(seq, nq, replace=False)) for _ in range(w)])
        keys = np.stack([np.sort(rng.choice(seq, nk, replace=False)) for _ in range(w)])
        a = int(rng.integers(0, seq // 2))
        ranges = ((a, a + int(rng.integers(1, 40))), (seq - 5, seq))
        plan = IndexedPlan.create(torch.from_numpy(rows), torch.from_numpy(keys), seq,
                                  protected_ranges=ranges, local_tokens=local)
        out[f"D{i}_rows"], out[f"D{i}_keys"] = rows, keys
        out[f"D{i}_meta"] = np.array([seq, local, *ranges[0], *ranges[1]], np.int64)
        out[f"D{i}_prot"] = plan.protected_blocks.numpy()

    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
