"""Build the C++ HIP test/bench harness executables and the measurement
probes (test infrastructure).

The executables link libkf_attn.so (rpath'd in-tree) and the oracle's C
restatement of the reference's CPU attention (oracle/cpu_attn.c);
libkf_probe.so (probe.hip, probe.h) holds the floors bench.py times beside the
decode.  Outputs go to tests/hip/bin/, which travels to the GPU host with the
tree.
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
PROBE_LIB = os.path.join(BIN, "libkf_probe.so")


def build_probe(verbose=False):
    """libkf_probe.so: a bare read of the decode's K / V bytes and an empty
    dispatch, timed by bench.py beside the decode step."""
    os.makedirs(BIN, exist_ok=True)
    cmd = [kbuild.HIPCC, *kbuild.DEVICE_FLAGS, "-shared", "-fPIC", f"-I{HERE}",
           os.path.join(HERE, "probe.hip"), "-o", PROBE_LIB + ".tmp"]
    kbuild.run(cmd, verbose)
    os.replace(PROBE_LIB + ".tmp", PROBE_LIB)
    return PROBE_LIB


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
    outs.append(build_probe(verbose))
    return outs


if __name__ == "__main__":
    print("built", build(verbose="-v" in sys.argv))
