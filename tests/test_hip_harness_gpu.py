"""Runs the C++ HIP harness tests/hip/test_flash_attn.cpp (and the C++ bench
tests/hip/bench_flash_attn.cpp) on the GPU.

The harness is the reference's tests/test_flash_attn.cu rewritten against
include/kf/flash_attn.hpp (the drop-in the integration notes describe): the
reference's 18 prefill cases through the synchronous launch_flash_attn,
decode and mixed-length cases through the asynchronous overload, the
kf::attn_fwd_ex / kf::attn_decode_paged extensions, and the asynchronous
launcher on two streams and on more streams than its workspace cache keeps.  __graft_entry__.build() compiles it to
tests/hip/bin/test_flash_attn.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "hip", "bin", "test_flash_attn")


@pytest.mark.gpu
def test_cpp_harness_passes():
    assert os.path.exists(EXE), (
        f"{EXE} is missing: build it with __graft_entry__.build() or "
        "`python tests/hip/build_harness.py`")
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=110)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    lines = r.stdout.splitlines()
    # 18 reference cases + 10 decode / mixed cases + extensions + two streams.
    assert sum("PASS" in l for l in lines) >= 30, r.stdout
    assert not any("FAIL" in l for l in lines), r.stdout
    assert "two streams" in r.stdout
    assert "through the workspace cache" in r.stdout


BENCH = os.path.join(HERE, "hip", "bin", "bench_flash_attn")


@pytest.mark.gpu
def test_cpp_bench_runs_every_reference_shape():
    """tests/hip/bench_flash_attn.cpp: the reference bench's 21 shapes
    (tests/bench_flash_attn.cu:150-185) through the asynchronous launcher,
    timed with HIP events; every shape reports a positive time."""
    assert os.path.exists(BENCH), f"{BENCH} is missing: build it with __graft_entry__.build()"
    r = subprocess.run([BENCH], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if " ms | " in l]
    assert len(lines) == 21, r.stdout
    for l in lines:
        ms = float(l.split("|")[1].split()[0])
        assert ms > 0, l
