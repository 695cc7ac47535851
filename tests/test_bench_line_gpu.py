"""bench.py end to end on the GPU: one short run prints the one JSON line the
bench contract asks for, with the headline metric of the configs[2] prefill,
its roofline point, every parity spot check passing, and configs[1]'s decode
block as the line's last key."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def line():
    print("bench.py --steps 3 --warmup 1 --no-cpu-baseline", flush=True)
    out = subprocess.run([sys.executable, "-u", os.path.join(REPO, "bench.py"), "--steps", "3",
                          "--warmup", "1", "--no-cpu-baseline"],
                         capture_output=True, text=True, timeout=300, cwd=REPO)
    assert out.returncode == 0, out.stderr[-2000:]
    lines = [l for l in out.stdout.splitlines() if l.strip()]
    assert len(lines) == 1, lines  # one JSON line and nothing else on stdout
    return json.loads(lines[0])


def test_contract_keys(line):
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
              "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
              "roofline"):
        assert k in line, k
    assert line["metric"] == "prefill TFLOPS @S=4096 GQA D=128; decode latency + HBM GB/s @KV=4096"
    assert line["n_gpus"] == 1 and line["steps"] == 3 and line["warmup"] == 1
    assert line["higher_is_better"] is True
    # vs_baseline: against the reference's published S=4096 figure (19.3 TFLOPS,
    # RTX 5070, the reference's README.md:49).
    assert line["vs_baseline"] == pytest.approx(line["value"] / 19.3, rel=1e-2)
    assert "workload" in line["config"]
    # value = TFLOPS of the configs[2] step: 2.749e11 FLOP per step.
    flops = 4.0 * 32 * 4096 * 4096 * 128
    assert line["value"] == pytest.approx(flops / (line["ms_per_step"] * 1e9), rel=2e-3)
    assert 100.0 < line["value"] < 2516.6


def test_roofline_point(line):
    r = line["roofline"]
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == 2516.6
    assert r["frac"] == pytest.approx(r["achieved"] / r["peak"], abs=1e-3)
    assert r["kernel"].startswith("kf_attn_prefill_wide_kernel<128, false, 1, false>")


def test_parity_spot_checks_pass(line):
    checks = [line["parity"], line["prefill_causal"]["parity"], line["decode_b32"]["parity"],
              line["decode_paged"]["parity"], line["decode_paged_c1"]["parity"]]
    checks += [r["parity"] for r in line["decode_sweep"]]
    checks += [r["parity"] for r in line["decode_kv4096_by_batch"]]
    checks += [s["parity"] for s in line["sweep"] if "parity" in s]
    assert len(checks) > 20
    for c in checks:
        assert c["ok"], c


def test_decode_block_is_last(line):
    assert list(line)[-1] == "decode"
    d = line["decode"]
    assert d["config"].startswith("configs[1]")
    assert d["roofline"]["bound"] == "hbm" and d["roofline"]["peak"] == 8000.0
    assert d["hbm_gbs"] == pytest.approx(d["roofline"]["bytes_per_launch"] / (d["latency_us"] * 1e3), rel=2e-3)
    assert d["parity_max_abs"] < 2e-3 and d["parity_rel_l2"] < 1e-2
    assert [b[0] for b in d["kv4096_by_batch"]] == [1, 2, 4, 8, 16, 32]
    # every reference bench row carries an MI355X figure
    assert len(line["reference_bench"]) == 21
    assert all(("us" in r) for r in line["reference_bench"])
