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
                  "rocprof_latency", "rocprof_roofline", "rocprof_full"):
            assert f"... {t}" in targets, targets
        # Like the reference's ncu targets (kernel name, the 5 warmup launches
        # skipped: tests/CMakeLists.txt:23-33), every counter pass runs one
        # shape under a kernel-name filter and the report skips the warmups.
        for t in ("rocprof_mfma", "rocprof_bandwidth", "rocprof_stalls", "rocprof_latency",
                  "rocprof_roofline"):
            mk = (build / "CMakeFiles" / f"{t}.dir" / "build.make").read_text()
            passes = [l for l in mk.splitlines() if "rocprofv3" in l and "--pmc" in l]
            assert passes, t
            for l in passes:
                assert "--kernel-include-regex kf_attn_prefill_wide_kernel" in l, l
                assert l.rstrip().endswith("bench_flash_attn --shape 1,4096,32,8,128"), l
        mk = (build / "CMakeFiles" / "rocprof_trace.dir" / "build.make").read_text()
        assert "rocprof_report.py trace" in mk and "shapes.md" in mk
        # rocprof_full runs its six passes itself, one after another (the
        # counters are device-wide: passes of a parallel build would mix).
        mk = (build / "CMakeFiles" / "rocprof_full.dir" / "build.make").read_text()
        assert "rocprof_report.py counters" in mk and "--skip 5 --count 50" in mk
        passes = [l for l in mk.splitlines() if "rocprofv3" in l and "--pmc" in l]
        assert [l.split(" -o ")[1].split()[0] for l in passes] == \
            ["mfma", "fetch", "write", "stalls", "latency", "roofline"]
        deps = (build / "CMakeFiles" / "Makefile2").read_text()
        full_deps = [l for l in deps.splitlines() if l.startswith("CMakeFiles/rocprof_full.dir/all:")]
        assert full_deps and not any("rocprof_mfma" in l or "rocprof_stalls" in l for l in full_deps)
    tests = subprocess.run(["ctest", "--test-dir", str(build), "-N"], check=True,
                           capture_output=True, text=True).stdout
    assert "flash_attn" in tests and "Total Tests: 1" in tests, tests
