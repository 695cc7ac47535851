#!/usr/bin/env python3
"""Summaries of the rocprof_* targets of tests/hip/CMakeLists.txt (test and
measurement infrastructure; reads rocprofv3 CSV output, runs nothing on the
GPU).

  rocprof_report.py trace <report dir> <bench_flash_attn>
      The kernel trace of the whole C++ bench (rocprof_trace), cut into the
      bench's shapes: ``bench_flash_attn --list`` gives the shapes in run order
      and the kernels per launch, and each shape is 5 warmup + 50 timed
      launches (tests/bench_flash_attn.cu:108-123).  Per shape: the median
      kernel time of a timed launch (the sum of its kernels), the back-to-back
      span per timed launch, and TFLOPS / GB/s from the span with the
      reference bench's formulas (:125-131).

  rocprof_report.py counters <reports root> [--cus N] [--xcds N] [--skip N] [--count N]
      The filtered counter passes (rocprof_mfma, rocprof_bandwidth,
      rocprof_stalls, rocprof_latency, rocprof_roofline) of one kernel of one
      shape: per counter the median over the kernel's dispatches after the
      first --skip (5: the bench's warmup launches; the reference's ncu
      targets skip the same five, tests/CMakeLists.txt:23-33) and at most
      --count of them (50: the timed launches), with the derived figures:
      MFMA busy per SIMD, VALU co-issue,
      HBM bytes (FETCH_SIZE x2 + WRITE_SIZE x1: the factors a 256 MiB device
      copy measures with the same counters on MI355X), wave-cycle shares,
      and the roofline point (FLOPs from SQ_INSTS_VALU_MFMA_MOPS_F16 x 512,
      duration from the same pass's kernel trace) against MI355X's
      published peaks.

Markdown on stdout.
"""
from __future__ import annotations

import csv
import glob
import os
import statistics
import subprocess
import sys
from collections import defaultdict

PEAK_FP16_TFLOPS = 2516.6  # 256 CU x 4096 FLOP/clk x 2.4 GHz, dense
PEAK_HBM_GBS = 8000.0
FETCH_SCALE, WRITE_SCALE = 2.0, 1.0
WARMUP, ITERS = 5, 50


def _rows(directory, pattern):
    out = []
    for f in sorted(glob.glob(os.path.join(directory, "**", pattern), recursive=True)):
        with open(f, newline="") as fh:
            out.extend(csv.DictReader(fh))
    return out


def _dur_us(r):
    return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0


def trace_report(report_dir, bench_exe):
    shapes = []
    listing = subprocess.run([bench_exe, "--list"], capture_output=True, text=True, check=True).stdout
    for line in listing.split("\n"):
        if line.strip():
            B, kv, H_q, H_kv, D, q, n = (int(x) for x in line.split())
            shapes.append((B, kv, H_q, H_kv, D, q, n))
    rows = [r for r in _rows(report_dir, "*kernel_trace.csv") if "kf_" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    need = sum((WARMUP + ITERS) * s[6] for s in shapes)
    print(f"# Kernel trace of the C++ bench, per shape\n")
    print(f"{len(rows)} kernel dispatches for {len(shapes)} shapes "
          f"(expected {need}: 5 warmup + 50 timed launches each).\n")
    if len(rows) != need:
        print("**dispatch count does not match the shape list; no per-shape table**")
        return 1
    print("| reference row | B | q_len | kv_len | H_q/H_kv | D | kernels | kernel us (median) "
          "| span us / launch | TFLOPS | GB/s |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    i = 0
    for idx, (B, kv, H_q, H_kv, D, q, n) in enumerate(shapes):
        launches = [rows[i + j * n: i + (j + 1) * n] for j in range(WARMUP + ITERS)]
        i += (WARMUP + ITERS) * n
        timed = launches[WARMUP:]
        ker = statistics.median(sum(_dur_us(r) for r in L) for L in timed)
        span = (int(timed[-1][-1]["End_Timestamp"]) - int(timed[0][0]["Start_Timestamp"])) / 1000.0 / ITERS
        names = " + ".join(r["Kernel_Name"].split("(")[0].replace("void ", "").replace("kf::", "")
                           for r in timed[0])
        flops = 4.0 * B * H_q * q * kv * D
        qn, kvn = B * H_q * q * D, B * H_kv * kv * D
        by = 2.0 * qn + 4.0 * kvn + 4.0 * qn
        ref_line = (154, 155, 156, 157, 158, 159, 162, 163, 164, 165, 168, 169, 170, 171, 174, 175,
                    176, 179, 180, 181, 182)
        ref = f"tests/bench_flash_attn.cu:{ref_line[idx]}" if len(shapes) == len(ref_line) else "-"
        print(f"| {ref} | {B} | {q} | {kv} | {H_q}/{H_kv} | {D} | `{names}` | {ker:.2f} | {span:.2f} "
              f"| {flops / (span * 1e6):.1f} | {by / (span * 1e3):.1f} |")
    print("\nkernel us: median over the 50 timed launches of the launch's kernel durations "
          "(begin to end of each dispatch, summed); span: first timed dispatch's begin to last "
          "timed dispatch's end, / 50, so it includes the kernel boundaries, as the bench's "
          "HIP-event time does.  Inputs are not rotated (the reference bench re-reads one set), "
          "so small decode shapes read the Infinity Cache.")
    return 0


def _selected(directory, skip, count):
    """The counter passes under `directory`: per pass (CSV file; one process
    each, dispatch ids restart at 1), the matching dispatches in id order,
    the first `skip` dropped and the next `count` kept.  Returns (kernel
    name, dispatch ids, {counter: median over those dispatches}, {dispatch id:
    kernel-trace row}) merged over the passes."""
    vals = defaultdict(list)
    names, ids, trace = set(), [], {}
    for f in sorted(glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)):
        per = defaultdict(lambda: defaultdict(float))
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                per[int(r["Dispatch_Id"])][r["Counter_Name"]] += float(r["Counter_Value"])
                names.add(r["Kernel_Name"])
        keep = sorted(per)[skip:skip + count]
        ids.extend(keep)
        for d in keep:
            for c, v in per[d].items():
                vals[c].append(v)
    for f in sorted(glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                trace[int(r["Dispatch_Id"])] = r
    med = {c: statistics.median(v) for c, v in vals.items()}
    return " / ".join(sorted(names)), ids, med, trace


def _head(target, name, ids):
    lo, hi = (min(ids), max(ids)) if ids else (0, 0)
    print(f"## {target}\n")
    print(f"`{name}`: medians over dispatches {lo}-{hi} of the kernel ({len(ids)} values per "
          "counter)\n")


def counters_report(root, cus, xcds, skip, count):
    simds = 4 * cus
    print("# Counter passes of the profiled kernel\n")
    print(f"Device: {cus} CUs ({simds} SIMDs) in {xcds} XCDs.  Each pass runs the C++ bench on one "
          f"shape with rocprofv3's --kernel-include-regex; the first {skip} dispatches of the "
          f"kernel (the bench's warmup launches) are skipped and the next {count} kept.\n")
    out = {}
    name, ids, v, _ = _selected(os.path.join(root, "rocprof_mfma"), skip, count)
    if v:
        cyc = v["GRBM_GUI_ACTIVE"] / xcds
        busy = v["SQ_VALU_MFMA_BUSY_CYCLES"] / (simds * cyc)
        out["mfma"] = busy
        _head("rocprof_mfma", name, ids)
        print("| counter | value |\n|---|---|")
        for k in sorted(v):
            print(f"| {k} | {v[k]:.0f} |")
        print(f"| MFMA busy per SIMD | {100 * busy:.1f} % (SQ_VALU_MFMA_BUSY_CYCLES / "
              f"({simds} SIMDs x GRBM_GUI_ACTIVE / {xcds})) |")
        print(f"| cycles per MFMA | {v['SQ_VALU_MFMA_BUSY_CYCLES'] / max(v['SQ_INSTS_MFMA'], 1):.1f} |")
        print(f"| VALU co-issued with MFMA | "
              f"{100 * v['SQ_VALU_MFMA_COEXEC_CYCLES'] / max(v['SQ_VALU_MFMA_BUSY_CYCLES'], 1):.1f} % "
              "of MFMA-busy cycles |")
        print(f"| active cycles per XCD | {cyc:.0f} |\n")
    name, ids, v, _ = _selected(os.path.join(root, "rocprof_bandwidth"), skip, count)
    if v:
        _head("rocprof_bandwidth (FETCH_SIZE and WRITE_SIZE, one pass each)", name, ids)
        print("| counter | KiB | bytes (calibrated) |\n|---|---|---|")
        tot = 0.0
        for k, sc in (("FETCH_SIZE", FETCH_SCALE), ("WRITE_SIZE", WRITE_SCALE)):
            if k in v:
                tot += v[k] * 1024 * sc
                print(f"| {k} | {v[k]:.0f} | {v[k] * 1024 * sc:.0f} (x{sc:.2f}) |")
        out["bytes"] = tot
        print(f"| HBM traffic | | {tot:.0f} |\n")
    name, ids, v, _ = _selected(os.path.join(root, "rocprof_stalls"), skip, count)
    if v:
        _head("rocprof_stalls", name, ids)
        wc = max(v.get("SQ_WAVE_CYCLES", 0.0), 1.0)
        print("| counter | value | share of SQ_WAVE_CYCLES |\n|---|---|---|")
        for k in sorted(v):
            print(f"| {k} | {v[k]:.0f} | {100 * v[k] / wc:.1f} % |")
        print()
    name, ids, v, _ = _selected(os.path.join(root, "rocprof_latency"), skip, count)
    if v:
        _head("rocprof_latency", name, ids)
        print("| counter | value (cycles) |\n|---|---|")
        for k in sorted(v):
            print(f"| {k} | {v[k]:.1f} |")
        print()
    name, ids, v, trace = _selected(os.path.join(root, "rocprof_roofline"), skip, count)
    if v:
        _head("rocprof_roofline", name, ids)
        flops = v.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) * 512
        print("| quantity | value |\n|---|---|")
        print(f"| SQ_INSTS_VALU_MFMA_MOPS_F16 | {v.get('SQ_INSTS_VALU_MFMA_MOPS_F16', 0):.0f} |")
        print(f"| MFMA FLOPs (x 512) | {flops:.4g} |")
        durs = [_dur_us(trace[d]) for d in ids if d in trace]
        if durs:
            us = statistics.median(durs)
            tf = flops / (us * 1e6)
            print(f"| duration (kernel trace of the same dispatches, median) | {us:.2f} us |")
            print(f"| achieved | {tf:.1f} TFLOP/s = {100 * tf / PEAK_FP16_TFLOPS:.1f} % of "
                  f"{PEAK_FP16_TFLOPS} (fp16 dense) |")
            if "bytes" in out:
                by = out["bytes"]
                print(f"| HBM bytes (rocprof_bandwidth) | {by:.0f} = {by / (us * 1e3):.1f} GB/s, "
                      f"{100 * by / (us * 1e3) / PEAK_HBM_GBS:.1f} % of {PEAK_HBM_GBS:.0f} |")
                ridge = PEAK_FP16_TFLOPS * 1e3 / PEAK_HBM_GBS
                print(f"| arithmetic intensity | {flops / by:.0f} FLOP/B (ridge {ridge:.0f}) -> "
                      f"{'MFMA' if flops / by > ridge else 'HBM'}-bound |")
        print()
    return 0


def main(argv):
    if len(argv) >= 3 and argv[0] == "trace":
        return trace_report(argv[1], argv[2])
    if len(argv) >= 2 and argv[0] == "counters":
        opt = {"--cus": 256, "--xcds": 8, "--skip": WARMUP, "--count": ITERS}
        rest = argv[2:]
        for i, a in enumerate(rest):
            if a in opt:
                opt[a] = int(rest[i + 1])
        return counters_report(argv[1], opt["--cus"], opt["--xcds"], opt["--skip"], opt["--count"])
    print(__doc__, file=sys.stderr)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
