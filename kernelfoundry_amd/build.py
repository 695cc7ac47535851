"""Build libkf_attn.so for gfx950.

Compilation is ahead of time and in-tree: the shared library lands in
``kernelfoundry_amd/lib/`` so it travels with the source tree to the GPU
host.  hipcc cross-compiles for gfx950 without a GPU present.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libkf_attn.so")
INCLUDE = os.path.join(REPO, "include")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-fp32 VALU ops are kept out of every code object (-packed-fp32-ops).
# -fno-honor-nans lets fmaxf skip NaN canonicalisation of MFMA results (the
# kernels never produce or test NaN); infinities keep their IEEE meaning,
# which the -inf score masking relies on.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fno-honor-nans",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def run(cmd, verbose=False):
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = (res.stdout or "") + (res.stderr or "")
    # hipcc's host pass does not know the packed-fp32 feature; that warning is noise.
    out = "\n".join(l for l in out.splitlines() if "not a recognized feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build_library(verbose=False, extra_flags=()):
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, *DEVICE_FLAGS, *extra_flags, "-shared", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}",
           os.path.join(CSRC, "attn_capi.hip"), "-o", tmp]
    run(cmd, verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_all(verbose=False):
    build_library(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built", LIB_PATH)
