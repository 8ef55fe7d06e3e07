"""Scratch budget of the hand-written kernels, read from the compiled code
objects (CPU only: hipcc cross-compiles for gfx950 here).

A kernel whose arrays the compiler can no longer keep in registers (a loop it
stops unrolling, a dynamically indexed accumulator, a spill) still computes
the right values, so the GPU parity tests pass, but it runs several times
slower: an epilogue branch once pushed the GEMM accumulators into scratch
and made every fp32 GEMM about 2.7x slower.  The code object shows it
directly as a nonzero private segment.
"""
import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from neuralscript_amd import build

SOURCES = ["gemm.hip", "attention.hip", "optim.hip", "rowops.hip", "moe.hip", "movement.hip"]
# Kernels allowed a private segment: none (every attention head size runs on
# the tiled MFMA kernels, padded where needed).
ALLOWED = ()

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not installed")


def _kernel_metadata(src, out_dir):
    """(kernel name, private segment bytes, VGPRs) of every kernel in src."""
    asm = os.path.join(out_dir, os.path.basename(src) + ".s")
    cmd = ["hipcc"] + build.HIPFLAGS + ["--cuda-device-only", "-S", src, "-o", asm]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    text = open(asm).read()
    rows = []
    for m in re.finditer(r"\.name:\s+(\S+)\n\s+\.private_segment_fixed_size:\s+(\d+)(.*?)\.vgpr_count:\s+(\d+)",
                         text, re.S):
        rows.append((m.group(1), int(m.group(2)), int(m.group(4))))
    return rows


def test_hot_kernels_use_no_scratch(tmp_path):
    srcs = [os.path.join(build.CSRC, s) for s in SOURCES]
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(lambda s: _kernel_metadata(s, str(tmp_path)), srcs))
    kernels = [k for rows in results for k in rows]
    assert len(kernels) >= 60, f"metadata not parsed: {len(kernels)} kernels"
    # the GEMM, MGS and flash-attention kernels must all be present
    for want in ("gemm_f32_kernel", "mgs_panel_kernel", "flash_bwd_dkdv_kernel", "flash_fwd_kernel"):
        assert any(want in name for name, _, _ in kernels), want
    bad = [(name, priv) for name, priv, _ in kernels if priv > 0 and not any(a in name for a in ALLOWED)]
    assert not bad, f"kernels with a private (scratch) segment: {bad}"
