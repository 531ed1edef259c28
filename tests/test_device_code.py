"""Checks on the gfx950 device code of the attention kernels (CPU only: hipcc cross-compiles).

The key-block DMA (``dma16`` in ``csrc/attn_common.h``) writes M0 in inline
assembly and declares it clobbered, which hipcc does not honour for a
reserved register.  That is only sound while no other instruction of these
kernels touches M0, so the assembly is checked: every write of M0 is the
DMA's own ``s_mov_b32 m0, <SGPR>`` / ``s_nop 0`` / ``global_load_lds_dwordx4``
sequence, and nothing else names M0.
"""

import os
import re
import shutil
import subprocess

import pytest

from sol_attn_amd import _build

HIPCC = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else None)


@pytest.mark.skipif(HIPCC is None, reason="hipcc not installed")
def test_only_the_key_block_dma_uses_m0(tmp_path):
    src = os.path.join(_build.CSRC, "attention.hip")
    asm = tmp_path / "attention.s"
    cmd = [HIPCC, *_build.compile_flags(), "-Wno-inline-asm", "--cuda-device-only", "-S", src, "-o", str(asm)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    assert res.returncode == 0, res.stderr[-2000:]
    lines = [l.split(";")[0].strip() for l in asm.read_text().splitlines()]
    code = [l for l in lines if l and not l.startswith(".") and not l.endswith(":")]
    writes = 0
    for i, line in enumerate(code):
        if not re.search(r"\bm0\b", line):
            continue
        # The asm statement's scalar operand: any SGPR (vcc_lo/vcc_hi are SGPRs too).
        assert re.fullmatch(r"s_mov_b32 m0, (s\d+|vcc_lo|vcc_hi)", line), f"unexpected use of M0: {line!r}"
        assert code[i + 1] == "s_nop 0" and code[i + 2].startswith("global_load_lds_dwordx4"), \
            f"M0 write not followed by the DMA: {code[i:i + 3]!r}"
        writes += 1
    assert writes > 0  # the DMA helper is in the build at all
