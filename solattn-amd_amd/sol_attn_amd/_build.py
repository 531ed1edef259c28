"""Build libsol_attn_amd.so (hand-written HIP for gfx950) in-tree with hipcc.

    python -m sol_attn_amd._build        # from the package root directory

Every call recompiles all sources.  Objects go to ``csrc/_build/``; the shared
library lands next to this file, where ``_native`` loads it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.abspath(os.path.join(PKG, "..", "..", "include"))
LIB_NAME = "libsol_attn_amd.so"
SOURCES = ("pool.hip", "route.hip", "attention.hip", "pairing.hip", "plan.hip", "covariance.hip", "quant.hip", "capi.hip")
# pool.hip reproduces torch's rounding step for step: no multiply-add fusion.
EXTRA_FLAGS = {"pool.hip": ["-ffp-contract=off"]}
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the SOL HIP library needs ROCm's hipcc")


def compile_flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
        # Packed-FP32 VALU forms are kept out of the generated code on purpose.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE, "-I", CSRC,
    ]


def build(verbose: bool = False) -> str:
    cc = hipcc()
    out_dir = os.path.join(CSRC, "_build")
    os.makedirs(out_dir, exist_ok=True)
    procs = []
    objects = []
    for src in SOURCES:
        obj = os.path.join(out_dir, src.replace(".hip", ".o"))
        objects.append(obj)
        cmd = [cc, *compile_flags(), *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src),
               "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, proc in procs:
        log = proc.communicate()[0].decode(errors="replace")
        # hipcc's host pass does not know the packed-fp32 feature; that note is harmless.
        log = "\n".join(l for l in log.splitlines() if "packed-fp32-ops" not in l)
        if proc.returncode != 0:
            failed.append(f"{src}:\n{log}")
        elif verbose and log.strip():
            print(log)
    if failed:
        raise RuntimeError("HIP compilation failed:\n" + "\n".join(failed))
    lib = os.path.join(PKG, LIB_NAME)
    tmp = lib + ".tmp"
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError("HIP link failed:\n" + res.stdout.decode(errors="replace"))
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
