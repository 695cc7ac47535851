"""Build the C++ HIP test/bench harness executables (test infrastructure).

They link libkf_attn.so (rpath'd in-tree) and the oracle's C restatement of
the reference's CPU attention (oracle/cpu_attn.c).  Outputs go to
tests/hip/bin/, which travels to the GPU host with the tree.
"""
from __future__ import annotations

import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

from kernelfoundry_amd import build as kbuild  # noqa: E402

BIN = os.path.join(HERE, "bin")


def build(verbose=False):
    os.makedirs(BIN, exist_ok=True)
    oracle_o = os.path.join(BIN, "cpu_attn.o")
    kbuild.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-c",
                os.path.join(REPO, "oracle", "cpu_attn.c"), "-o", oracle_o], verbose)
    outs = []
    for name in ("test_flash_attn", "bench_flash_attn"):
        src = os.path.join(HERE, name + ".cpp")
        if not os.path.exists(src):
            continue
        exe = os.path.join(BIN, name)
        cmd = [kbuild.HIPCC, *kbuild.DEVICE_FLAGS, f"-I{kbuild.INCLUDE}", "-x", "hip", src,
               "-x", "none", oracle_o, f"-L{kbuild.LIB_DIR}", "-lkf_attn",
               f"-Wl,-rpath,{kbuild.LIB_DIR}",
               "-Wl,-rpath,$ORIGIN/../../../kernelfoundry_amd/lib", "-o", exe + ".tmp"]
        kbuild.run(cmd, verbose)
        os.replace(exe + ".tmp", exe)
        outs.append(exe)
    return outs


if __name__ == "__main__":
    print("built", build(verbose="-v" in sys.argv))
