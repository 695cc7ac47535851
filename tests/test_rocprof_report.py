"""tests/hip/rocprof_report.py on synthetic rocprofv3 CSV files (no GPU):
the kernel trace of the C++ bench is cut into its 21 shapes in run order, and
the counter report derives MFMA busy, calibrated HBM bytes and the roofline
point from the counter values it is given."""
import csv
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPORT = os.path.join(HERE, "hip", "rocprof_report.py")
BENCH = os.path.join(HERE, "hip", "bin", "bench_flash_attn")


def _write(path, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
        w.writeheader()
        w.writerows(rows)


@pytest.mark.skipif(not os.path.exists(BENCH), reason="C++ bench not built")
def test_trace_report_cuts_the_bench_into_its_shapes(tmp_path):
    listing = subprocess.run([BENCH, "--list"], capture_output=True, text=True, check=True).stdout
    shapes = [tuple(int(x) for x in l.split()) for l in listing.splitlines() if l.strip()]
    assert len(shapes) == 21
    rows, t, did = [], 1_000_000, 0
    for k, (B, kv, H_q, H_kv, D, q, n) in enumerate(shapes):
        for launch in range(55):
            for j in range(n):
                name = f"void kf::kf_kernel_{k}_{j}<{D}>(kf::AttnParams)"
                dur = 1000 * (k + 1) + j  # ns: shape k's kernels take k + 1 us (+ j ns)
                did += 1
                rows.append({"Dispatch_Id": did, "Kernel_Name": name, "Start_Timestamp": t,
                             "End_Timestamp": t + dur})
                t += dur + 500
    _write(str(tmp_path / "host" / "1_trace_kernel_trace.csv"), rows)
    out = subprocess.run([sys.executable, REPORT, "trace", str(tmp_path), BENCH],
                         capture_output=True, text=True, check=True).stdout
    table = [l for l in out.splitlines() if l.startswith("| tests/bench_flash_attn.cu:")]
    assert len(table) == 21
    for k, l in enumerate(table):
        cells = [c.strip() for c in l.strip("|").split("|")]
        n = shapes[k][6]
        assert f"kernel_{k}_0" in cells[6]
        assert float(cells[7]) == pytest.approx((1000 * (k + 1) * n + sum(range(n))) / 1000, abs=0.01)
    assert table[3].startswith("| tests/bench_flash_attn.cu:157 |")   # KV = 4096 decode
    assert table[13].startswith("| tests/bench_flash_attn.cu:171 |")  # S = 4096 prefill
    # A trace that does not hold the whole bench gets no table.
    _write(str(tmp_path / "host" / "1_trace_kernel_trace.csv"), rows[:-1])
    out = subprocess.run([sys.executable, REPORT, "trace", str(tmp_path), BENCH],
                         capture_output=True, text=True).stdout
    assert "does not match" in out


def test_counter_report_derives_the_figures(tmp_path):
    """Five warmup dispatches (wild values) are skipped; the medians of the
    timed ones give the derived figures."""
    name = "void kf::kf_attn_prefill_wide_kernel<128, false, 1, false>(kf::AttnParams)"

    def pmc(target, label, values, trace=False):
        rows, tr = [], []
        for d in range(1, 9):
            k = 7.0 if d <= 5 else (1.0 if d != 8 else 1.5)  # warmups off, one timed outlier
            for c, v in values.items():
                rows.append({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": c,
                             "Counter_Value": v * k})
            tr.append({"Dispatch_Id": d, "Kernel_Name": name, "Start_Timestamp": 10_000 * d,
                       "End_Timestamp": 10_000 * d + (2000 if d > 5 else 9000)})
        _write(str(tmp_path / target / "host" / f"1_{label}_counter_collection.csv"), rows)
        if trace:
            _write(str(tmp_path / target / "host" / f"1_{label}_kernel_trace.csv"), tr)

    pmc("rocprof_mfma", "mfma", {"SQ_VALU_MFMA_BUSY_CYCLES": 1024 * 1000 * 0.5,
                                 "GRBM_GUI_ACTIVE": 8 * 1000, "SQ_INSTS_MFMA": 16000,
                                 "SQ_VALU_MFMA_COEXEC_CYCLES": 1024 * 1000 * 0.5 * 0.25,
                                 "SQ_BUSY_CYCLES": 1, "SQ_INSTS_VALU": 1,
                                 "SQ_LDS_BANK_CONFLICT": 0})
    pmc("rocprof_bandwidth", "fetch", {"FETCH_SIZE": 1000.0})
    pmc("rocprof_bandwidth", "write", {"WRITE_SIZE": 3000.0})
    pmc("rocprof_roofline", "roofline", {"SQ_INSTS_VALU_MFMA_MOPS_F16": 2.0e9 / 512}, trace=True)
    out = subprocess.run([sys.executable, REPORT, "counters", str(tmp_path)],
                         capture_output=True, text=True, check=True).stdout
    assert "medians over dispatches 6-8" in out
    assert "| MFMA busy per SIMD | 50.0 %" in out
    assert "| VALU co-issued with MFMA | 25.0 %" in out
    assert "| HBM traffic | | 5120000 |" in out            # 1000 KiB x 2 + 3000 KiB x 1
    assert "| achieved | 1000.0 TFLOP/s" in out             # 2e9 FLOP in 2 us
    assert "2560.0 GB/s" in out                              # 5.12e6 B in 2 us
