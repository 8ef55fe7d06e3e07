"""Build libnship.so (hand-written gfx950 HIP kernels + runtime) in-tree, and
the per-network ABI drivers for the bundled networks.

    python -m neuralscript_amd.build          # compile everything
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

from . import emit

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libnship.so")
NETS = os.path.join(PKG, "nets")

ARCH = "gfx950"
# -packed-fp32-ops off: no packed fp32 VALU instructions are generated.
HIPFLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", os.path.join(REPO, "include"), "-I", CSRC,
            "-Wall", "-Wno-unused-command-line-argument"]


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = ["hipcc"] + HIPFLAGS + ["-c", src, "-o", obj]
    if src.endswith(".cpp"):  # plain host C++ (the IR parser)
        cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-I", os.path.join(REPO, "include"),
               "-I", CSRC, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build_lib(jobs=8):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = ["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_nets():
    """Per-network drivers for every bundled IR plan (neuralscript_amd/nets)."""
    out = []
    for ir in sorted(glob.glob(os.path.join(NETS, "*.mlir"))):
        name = os.path.splitext(os.path.basename(ir))[0]
        with open(ir) as f:
            text = f.read()
        out.append(emit.build_driver(name, text, NETS, PKG))
    return out


def main():
    build_lib()
    build_nets()
    print(LIB)


if __name__ == "__main__":
    sys.exit(main())
