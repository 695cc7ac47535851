"""tests/hip/CMakeLists.txt configures on a host without a GPU and registers
what the reference's tests/CMakeLists.txt registers: the end-to-end test under
ctest and one profiling target per ncu_* target (rocprofv3 here).  Only the
configure step runs (no compilation), so the check takes about a second."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("cmake") is None, reason="cmake not installed")
def test_cmake_harness_registers_test_and_profiling_targets(tmp_path):
    build = tmp_path / "build"
    subprocess.run(["cmake", "-S", os.path.join(HERE, "hip"), "-B", str(build)], check=True,
                   capture_output=True, text=True)
    targets = subprocess.run(["cmake", "--build", str(build), "--target", "help"], check=True,
                             capture_output=True, text=True).stdout
    for t in ("kf_attn", "test_flash_attn", "bench_flash_attn"):
        assert f"... {t}" in targets, targets
    if shutil.which("rocprofv3") or os.path.exists("/opt/rocm/bin/rocprofv3"):
        for t in ("rocprof_trace", "rocprof_mfma", "rocprof_bandwidth", "rocprof_stalls",
                  "rocprof_latency"):
            assert f"... {t}" in targets, targets
    tests = subprocess.run(["ctest", "--test-dir", str(build), "-N"], check=True,
                           capture_output=True, text=True).stdout
    assert "flash_attn" in tests and "Total Tests: 1" in tests, tests
