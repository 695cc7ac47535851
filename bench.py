#!/usr/bin/env python3
"""Benchmark of the MI355X flash-attention forward (one GPU).

Headline (``value``): GQA prefill, non-causal, B=1, H_q=32, H_kv=8, D=128,
Q_len = KV_len = 4096, fp16 in / fp32 out -- BASELINE.json configs[2], the
"prefill TFLOPS @S=4096" half of the metric.  A step is one forward pass over
that batch (one kernel launch); inputs are resident in HBM before timing.

Also reported in the same JSON line (the "decode latency + HBM GB/s @KV=4096"
half of the metric):
  * ``decode``    -- configs[1]: B=1, H_q=32, H_kv=8, D=128, Q_len=1,
                     KV=4096, the LAST key of the line (compact) so that the
                     end of the line carries it.  Its 16.8 MB working set fits
                     the 256 MB Infinity Cache, so each step reads the next of
                     ``--decode-sets`` distinct Q/K/V sets (> 512 MB total) and
                     the figure is an HBM figure, not a cache figure.
                     ``decode.floor``: a bare read of the same K/V bytes over
                     the same rotated sets (kf_probe_read) and an empty
                     back-to-back dispatch (one kernel boundary), timed the
                     same way; ``decode.graph_step_us``: the same steps
                     replayed from one captured HIP graph.
  * ``decode_b32`` -- configs[4]: B=32, KV=8192 (1.07 GB of unique K/V per
                     step), the clean HBM-streaming case, with the same bare
                     read of its 1.07 GB of K/V beside it (``floor``).
  * ``prefill_causal`` -- the configs[2] shape with the causal mask of
                     kf_attn_fwd_ex; FLOPs count only the visible pairs,
                     4*B*H_q*D*S(S+1)/2.
  * ``decode_paged`` -- the configs[4] decode over a paged cache
                     (kf_attn_decode_paged): 16-row pages scattered over a
                     pool twice the needed size (the reference's worst-case
                     fragmentation, bench_flash_attn2.py:153-215); bytes =
                     configs[4]'s plus the block table.  ``decode_paged_c1``:
                     the configs[1] decode over such a cache (rotated over
                     > 512 MB of pools).
  * ``decode_sweep`` -- the reference bench's decode shapes (B=1 KV=512..4096,
                     B=8 KV=512/1024, MQA KV=512/1024; tests/bench_flash_attn.cu:
                     154-159, 181-182), each rotated over > 512 MB of sets,
                     with the same read floor and an oracle spot check.
  * ``decode_kv4096_by_batch`` -- configs[1]'s decode at B = 2 .. 32 (rotated,
                     spot-checked): where the KV=4096 decode turns from
                     latency-bound to HBM-bound; ``decode.kv4096_by_batch``
                     repeats it compactly as [B, us, fraction of peak].
  * ``sweep``     -- prefill S = 512 / 1024 / 2048 (configs[0] / [2] sweep),
                     the MQA D=64 configs[3] and the configs[2] shape at
                     D=256 (the reference's largest head dimension), plain
                     and causal (visible-pair FLOPs), S = 512 / 1024 at
                     D=256 (small grids: two KV groups per workgroup), and
                     configs[2] with a per-sequence key count of 4000 (FLOPs
                     over those keys), causal prefill at 2 x 4096 and 1 x 8192
                     queries (grids that take the wide layout's causal kernel;
                     visible-pair FLOPs, spot-checked), and chunked prefill (q_len = 16 / 64 /
                     128 / 256 query rows against 4096-16384 keys, 32 / 8 heads,
                     D = 128, and 64 x 4096 at D = 256:
                     the split prefill's KV partitions + split merge, the
                     timed step covering both launches, spot-checked against
                     the oracle).  Each line names its kernels.
  * ``reference_bench`` -- every row of the reference bench
                     (tests/bench_flash_attn.cu:154-182) with its MI355X time,
                     TFLOPS or GB/s and, where README.md:46-58 publishes one,
                     the reference's RTX 5070 time; the rows not timed above
                     (short prefill, D = 64 at S = 1024, MQA D = 128 prefill)
                     are timed over rotated input sets (> 512 MB) and
                     spot-checked against the oracle.

FLOPs = 4*B*H_q*q_len*kv_len*D and bytes = fp16 Q + unique fp16 K,V + fp32 O
(tests/bench_flash_attn.cu:125-131).  ``roofline.achieved`` divides the
headline's FLOPs by the kernel's launch duration from the timed region (one
launch per step, back to back between two HIP events on the launch stream);
``roofline.launch_ms_event_pairs`` is the mean of an event pair around every
launch (a separate pass; the event records add about 1.5 us per launch).
``cpu_baseline`` times the repo's NumPy
restatement of the reference's CPU path (kernel_models/flash_attn.py:250-265)
on a bounded sample of the same workload on this host's cores;
``cpu_baseline_c1_tiled`` times the restated tiled online-softmax model
(kernel_models/flash_attn.py:184-246) on configs[0], the configuration
BASELINE.json says runs on CPU.  ``roofline.kernel`` is the plan's kernel
(kf_attn_kernel_names) and ``roofline.traffic`` the committed FETCH/WRITE
figure only when it was collected on the current kernel sources.

Timing protocol per workload: ``SETTLE_S`` seconds of untimed launches (the
clocks reach their loaded steady state), W untimed warmup steps, then K timed
back-to-back steps between two events on the launch stream, with a
synchronize on both sides: one such timed region for the headline, the
median of ``PASSES`` for every other workload.  Before each region's first
event a clock-bounded sleep kernel holds the stream while the host enqueues
the K steps (``queue_gate``), so a region times the GPU, not the host's
launch rate.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

METRIC = "prefill TFLOPS @S=4096 GQA D=128; decode latency + HBM GB/s @KV=4096"
PEAK_FP16_TFLOPS = 2516.6   # MI355X dense fp16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
REF_PREFILL_S4096_TFLOPS = 19.3   # reference, RTX 5070 (README.md:49)
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic_prefill_s4096.json")
PROBE_LIB = os.path.join(REPO, "tests", "hip", "bin", "libkf_probe.so")
# The sources the prefill kernel and its launch plan are built from; the
# committed FETCH/WRITE figures hold only for the sources they were collected on.
KERNEL_SOURCES = ("kernelfoundry_amd/csrc/attn_kernels.h", "kernelfoundry_amd/csrc/attn_capi.hip")


def source_sha256():
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(REPO, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def committed_traffic():
    """(HBM bytes per launch, note) from profiles/traffic_prefill_s4096.json,
    or (None, reason) when that file was collected on other kernel sources."""
    if not os.path.exists(TRAFFIC_FILE):
        return None, "no committed FETCH_SIZE / WRITE_SIZE collection"
    with open(TRAFFIC_FILE) as f:
        t = json.load(f)
    if t.get("source_sha256") != source_sha256():
        return None, ("stale: profiles/traffic_prefill_s4096.json was collected on other "
                      "kernel sources (source_sha256 differs); re-collect FETCH_SIZE / WRITE_SIZE")
    return t.get("traffic_bytes_per_launch"), "rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 (calibrated)"


def load_probe(kf):
    """libkf_probe.so (tests/hip/probe.h: measurement probes built beside the
    C++ bench harness, not part of the attention library), loaded after the
    attention library so that both bind to torch's HIP runtime."""
    kf.load_library()
    lib = ctypes.CDLL(PROBE_LIB)
    p, sz = ctypes.c_void_p, ctypes.c_size_t
    lib.kf_probe_read.argtypes = [p, p, sz, p, p]
    lib.kf_probe_read.restype = ctypes.c_int
    lib.kf_probe_empty.argtypes = [p]
    lib.kf_probe_empty.restype = ctypes.c_int
    return lib


def flops(B, H_q, q, kv, D):
    return 4.0 * B * H_q * q * kv * D


def causal_flops(B, H_q, S, D):
    """Algorithmic FLOPs of causal attention with q_len = kv_len = S: query i
    sees i + 1 keys, so sum_i (i + 1) = S (S + 1) / 2 score/PV pairs."""
    return 4.0 * B * H_q * D * S * (S + 1) / 2


def nbytes(B, H_q, H_kv, q, kv, D):
    qn, kvn = B * H_q * q * D, B * H_kv * kv * D
    return 2.0 * qn + 4.0 * kvn + 4.0 * qn


def _inputs(torch, B, H_q, H_kv, q, kv, D, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    Q = torch.randn((B, H_q, q, D), generator=g, device="cuda", dtype=torch.float32).half()
    K = torch.randn((B, H_kv, kv, D), generator=g, device="cuda", dtype=torch.float32).half()
    V = torch.randn((B, H_kv, kv, D), generator=g, device="cuda", dtype=torch.float32).half()
    return Q, K, V


class Runner:
    """Pre-resolved kf_attn_fwd call (no allocation inside the timed loop)."""

    def __init__(self, torch, kf, sets, D, flags=0, kv_lens=None):
        self.torch, self.kf = torch, kf
        self.flags = flags
        # Per-sequence key counts (device int32 [B]) for kf_attn_fwd_ex, or None.
        self.kv_lens = kv_lens
        Q, K, V = sets[0]
        B, H_q, q, _ = Q.shape
        _, H_kv, kv, _ = K.shape
        self.shape = (B, q, kv, H_q, H_kv, D)
        self.plan = kf.plan(B, q, kv, H_q, H_kv, D)
        self.ws_bytes = self.plan.workspace_bytes
        self.ws = torch.empty(max(self.ws_bytes, 256), dtype=torch.uint8, device="cuda")
        self.sets = sets
        self.outs = [torch.empty((B, H_q, q, D), dtype=torch.float32, device="cuda") for _ in sets]
        self.stream = torch.cuda.current_stream()
        self.lib = kf.load_library()
        self.i = 0

    def launch(self, stream=None):
        j = self.i % len(self.sets)
        self.i += 1
        Q, K, V = self.sets[j]
        B, q, kv, H_q, H_kv, D = self.shape
        cs = (stream or self.stream).cuda_stream
        if self.flags or self.kv_lens is not None:
            lens = None if self.kv_lens is None else self.kv_lens.data_ptr()
            st = self.lib.kf_attn_fwd_ex(Q.data_ptr(), K.data_ptr(), V.data_ptr(),
                                         self.outs[j].data_ptr(), None, None, B, q, kv, H_q, H_kv,
                                         D, lens, self.flags,
                                         self.ws.data_ptr() if self.ws_bytes else None,
                                         self.ws_bytes, cs)
        else:
            st = self.lib.kf_attn_fwd(Q.data_ptr(), K.data_ptr(), V.data_ptr(),
                                      self.outs[j].data_ptr(), None, None, B, q, kv, H_q, H_kv, D,
                                      self.ws.data_ptr() if self.ws_bytes else None,
                                      self.ws_bytes, cs)
        if st != 0:
            raise RuntimeError(f"kf_attn_fwd failed: {self.kf.status_string(st)}")
        return j


SETTLE_S = 0.1  # untimed launches per workload before its warmup steps
# Timed regions per workload other than the headline (median reported): one
# pass of a few microseconds moves with the box's momentary state.
PASSES = 3
# Inputs rotated through per workload that fits the 256 MB Infinity Cache, so
# that every step reads HBM.
ROTATE_BYTES = 600e6


def settle(torch, runner, seconds=SETTLE_S):
    """Untimed launches for about `seconds` of wall time.  The GPU's clocks
    ramp up under sustained load: measured on MI355X, the first 100 prefill
    steps after 10 warmup launches (27 ms) ran at 288 us per step, every later
    pass at 268 us.  This runs before the W warmup steps so that the K timed
    steps see the steady-state clock."""
    t = time.perf_counter()
    while time.perf_counter() - t < seconds:
        for _ in range(16):
            runner.launch()
        torch.cuda.synchronize()


# Length of the queue-ahead gate per timed step, in GPU clock cycles (about
# 19 us of host time per step at 2.1 GHz).
GATE_CYCLES_PER_STEP = 40_000


def queue_gate(torch, stream, steps):
    """A clock-bounded sleep kernel (torch.cuda._sleep: it spins until its own
    cycle counter has advanced by a fixed count, so it always ends) enqueued on
    the launch stream right before a timed region's first event.  While it
    runs, the host enqueues the region's steps ahead of the GPU, so the events
    time the GPU's back-to-back execution of the steps rather than the host's
    launch rate: a ctypes call plus the two hipLaunchKernel calls of a split
    decode step take about as long on the host as the configs[1] step takes
    on the GPU."""
    with torch.cuda.stream(stream):
        torch.cuda._sleep(int(GATE_CYCLES_PER_STEP * max(steps, 10)))


def time_steps(torch, runner, steps, warmup, passes=1):
    """Whole-step wall time over `steps` back-to-back launches (the median
    over `passes` such timed regions, each between two events on the launch
    stream with a synchronize on both sides and the queue-ahead gate before
    the first event), plus the average and median per-launch duration from an
    event pair around every launch."""
    settle(torch, runner)
    for _ in range(warmup):
        runner.launch()
    torch.cuda.synchronize()
    region = []
    for _ in range(passes):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        queue_gate(torch, runner.stream, steps)
        t0.record(runner.stream)
        for _ in range(steps):
            runner.launch()
        t1.record(runner.stream)
        torch.cuda.synchronize()
        region.append(t0.elapsed_time(t1) / steps)
    ms_step = statistics.median(region)
    # Per-launch durations (separate pass so the event records do not perturb
    # the back-to-back timing above).
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for a, b in evs:
        a.record(runner.stream)
        runner.launch()
        b.record(runner.stream)
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) for a, b in evs]
    return ms_step, statistics.mean(per), statistics.median(per)


def parity_spot_check(torch, runner, heads, causal=False):
    """Compare the last outputs on a few heads with the fp64 oracle."""
    from oracle import attn_oracle as orc
    import numpy as np

    j = (runner.i - 1) % len(runner.sets)
    Q, K, V = (t.cpu().numpy() for t in runner.sets[j])
    O = runner.outs[j].cpu().numpy()
    H_q, H_kv = Q.shape[1], K.shape[1]
    worst = (0.0, 0.0)
    for b, h in heads:
        hk = h // (H_q // H_kv)
        ref, _, _ = orc.sdpa(Q[b:b + 1, h:h + 1], K[b:b + 1, hk:hk + 1], V[b:b + 1, hk:hk + 1],
                             causal=causal)
        ok, mx, rel = orc.within_tolerance(O[b:b + 1, h:h + 1], ref)
        if not ok:
            raise AssertionError(f"bench parity failed on head ({b},{h}): max_abs={mx} rel={rel}")
        worst = (max(worst[0], mx), max(worst[1], rel))
    return {"heads": [list(x) for x in heads], "max_abs": worst[0], "rel_l2": worst[1],
            "atol": orc.ATOL, "rtol": orc.RTOL, "ok": True}


def run_paged_decode(torch, kf, steps, warmup, check, B=32, kv=8192, H_q=32, H_kv=8, D=128,
                     page_size=16, label="configs[4]"):
    """A decode over a fragmented paged cache: each set's pages are randomly
    placed in a pool twice the needed size; sets (pools, tables, queries) are
    rotated through until they exceed the Infinity Cache.  Returns a result
    dict."""
    max_pages = kv // page_size
    num_pages = 2 * B * max_pages
    set_bytes = 2 * num_pages * H_kv * page_size * D * 2
    n_sets = int(max(1, min(64, math.ceil(ROTATE_BYTES / set_bytes))))
    g = torch.Generator(device="cuda")
    g.manual_seed(4242)
    sets = []
    for _ in range(n_sets):
        Kp = torch.randn((num_pages, H_kv, page_size, D), generator=g, device="cuda").half()
        Vp = torch.randn((num_pages, H_kv, page_size, D), generator=g, device="cuda").half()
        Q = torch.randn((B, H_q, 1, D), generator=g, device="cuda").half()
        table = torch.randperm(num_pages, generator=g, device="cuda")[:B * max_pages] \
            .to(torch.int32).reshape(B, max_pages).contiguous()
        O = torch.empty((B, H_q, 1, D), dtype=torch.float32, device="cuda")
        sets.append((Q, Kp, Vp, table, O))
    lens = torch.full((B,), kv, dtype=torch.int32, device="cuda")
    need = kf.paged_workspace_bytes(B, 1, H_q, H_kv, D, page_size, max_pages)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
    lib = kf.load_library()
    stream = torch.cuda.current_stream()
    args = [(Q.data_ptr(), Kp.data_ptr(), Vp.data_ptr(), table.data_ptr(), lens.data_ptr(),
             O.data_ptr(), None, None, B, 1, H_q, H_kv, D, page_size, max_pages, num_pages, 0,
             ws.data_ptr(), need, stream.cuda_stream) for (Q, Kp, Vp, table, O) in sets]

    class _R:
        stream = None
        i = 0

        def launch(self):
            a = args[self.i % n_sets]
            self.i += 1
            st = lib.kf_attn_decode_paged(*a)
            if st != 0:
                raise RuntimeError(f"kf_attn_decode_paged failed: {kf.status_string(st)}")

    r = _R()
    r.stream = stream
    ms, kern_mean, _ = time_steps(torch, r, steps, warmup, PASSES)
    by = nbytes(B, H_q, H_kv, 1, kv, D) + B * max_pages * 4
    # The paged forms of the kernels the contiguous plan names.
    kern = kf.kernel_names(B, 1, kv, H_q, H_kv, D).replace(
        "decode_short_kernel", "decode_short_paged_kernel").replace(
        "kf_attn_decode_kernel<%d, false>" % D, "kf_attn_decode_kernel<%d, true>" % D)
    out = {"config": f"{label} over a paged cache: B={B} KV={kv} page_size={page_size}, "
                     f"pages randomly placed in a {num_pages}-page pool",
           "latency_us": round(ms * 1e3, 2), "hbm_gbs": round(by / (ms * 1e6), 1),
           "launch_us_mean": round(kern_mean * 1e3, 2), "bytes_per_launch": by,
           "sets_rotated": n_sets, "passes": PASSES, "kernels": kern,
           "roofline": {"bound": "hbm", "achieved": round(by / (ms * 1e6), 1),
                        "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(by / (ms * 1e6) / PEAK_HBM_GBS, 4)}}
    if check:
        from oracle import attn_oracle as orc
        import numpy as np
        Q, Kp, Vp, table, O = sets[(r.i - 1) % n_sets]
        tb = table.cpu().numpy()
        heads = [(0, 0), (B - 1, H_q - 1)]
        worst = (0.0, 0.0)
        for b, h in heads:
            hk = h // (H_q // H_kv)
            ids = torch.from_numpy(tb[b].astype(np.int64)).cuda()
            Kc = Kp[ids][:, hk].reshape(1, 1, kv, D).cpu().numpy()
            Vc = Vp[ids][:, hk].reshape(1, 1, kv, D).cpu().numpy()
            ref, _, _ = orc.sdpa(Q[b:b + 1, h:h + 1].cpu().numpy(), Kc, Vc)
            ok, mx, rel = orc.within_tolerance(O[b:b + 1, h:h + 1].cpu().numpy(), ref)
            if not ok:
                raise AssertionError(f"paged bench parity failed on ({b},{h}): {mx} {rel}")
            worst = (max(worst[0], mx), max(worst[1], rel))
        out["parity"] = {"heads": [list(x) for x in heads], "max_abs": worst[0],
                         "rel_l2": worst[1], "atol": orc.ATOL, "rtol": orc.RTOL, "ok": True}
    del sets, args
    torch.cuda.empty_cache()
    return out


class ProbeRunner:
    """Back-to-back launches of a probe (same interface as Runner)."""

    def __init__(self, torch, fn, n_sets=1):
        self.stream = torch.cuda.current_stream()
        self.fn, self.n, self.i = fn, n_sets, 0

    def launch(self, stream=None):
        j = self.i % self.n
        self.i += 1
        st = self.fn(j, (stream or self.stream).cuda_stream)
        if st != 0:
            raise RuntimeError(f"probe launch failed ({st})")


def decode_floors(torch, probe, sets, steps, warmup):
    """Floors of a small decode step, timed like the step itself: a bare read
    of the same K and V bytes (the same rotated sets) and an empty dispatch.
    Back to back on one stream, the empty dispatch is the cost of a kernel
    boundary."""
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    nbytes_kv = sets[0][1].numel() * 2

    def read(j, cs):
        return probe.kf_probe_read(sets[j][1].data_ptr(), sets[j][2].data_ptr(), nbytes_kv,
                                   sink.data_ptr(), cs)

    ms_read, _, _ = time_steps(torch, ProbeRunner(torch, read, len(sets)), steps, warmup, PASSES)
    ms_empty, _, _ = time_steps(torch, ProbeRunner(torch, lambda j, cs: probe.kf_probe_empty(cs)),
                                steps, warmup, PASSES)
    return ms_read * 1e3, ms_empty * 1e3, 2.0 * nbytes_kv


def time_graph(torch, runner, replays=20):
    """The decode steps of one pass over the rotated sets captured into one
    HIP graph (torch.cuda.CUDAGraph) and replayed back to back: per-step time,
    and whether every replay reproduced the eager outputs bit for bit.  The
    kernels record no memset, so the graph holds only their launches."""
    n = len(runner.sets)
    runner.i = 0
    for _ in range(n):
        runner.launch()
    torch.cuda.synchronize()
    eager = [o.clone() for o in runner.outs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        runner.i = 0
        for _ in range(n):
            runner.launch(torch.cuda.current_stream())
    torch.cuda.synchronize()
    ok = True
    for o in runner.outs:
        o.zero_()
    for _ in range(2):  # replays with eager work and syncs between them
        g.replay()
        torch.cuda.synchronize()
        ok = ok and all(torch.equal(a, b) for a, b in zip(runner.outs, eager))
        for o in runner.outs:
            o.zero_()
        torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(replays):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    ok = ok and all(torch.equal(a, b) for a, b in zip(runner.outs, eager))
    del g
    return t0.elapsed_time(t1) / (replays * n) * 1e3, ok


def cpu_baseline_tiled_c1(min_runs=3):
    """configs[0] as BASELINE.json states it, "on CPU via the NumPy reference
    model": the repo's restatement of the reference's tiled online-softmax
    model (oracle.tiled_online_softmax = kernel_models/flash_attn.py:184-246,
    Br=16, Bc_col=8, kv_block_rows=128, the k/co loops as row matmuls) on the
    whole C1 prefill (S=512, 32/8 heads, D=128), median of the timed runs."""
    import numpy as np

    from oracle import attn_oracle as orc

    S, D, H_q, H_kv = 512, 128, 32, 8
    q, k, v = orc.normal_fp16_inputs(1, H_q, H_kv, S, S, D, 0)
    q, k, v = q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)
    orc.tiled_online_softmax(q[:, :4], k[:, :1], v[:, :1])  # warm-up
    runs = []
    while len(runs) < min_runs:
        t = time.perf_counter()
        orc.tiled_online_softmax(q, k, v)
        runs.append(time.perf_counter() - t)
    sec = statistics.median(runs)
    cores, threads, blas, cpu_model = host_info()
    return {
        "value": round(flops(1, H_q, S, S, D) / sec / 1e12, 5), "unit": "TFLOPS",
        "cores": int(threads) if threads and threads.isdigit() else cores,
        "kind": "port",
        "sample": (f"configs[0] prefill S=512 GQA 32/8 D=128, all 32 heads, tiled online-softmax "
                   f"model (oracle.tiled_online_softmax = kernel_models/flash_attn.py:184-246), "
                   f"median of {len(runs)} runs = {sec:.2f} s; cpu '{cpu_model}', affinity "
                   f"{cores} cores, BLAS {blas}, BLAS threads {threads or 'default'}"),
    }


def host_info():
    import numpy as np

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    threads = os.environ.get("OPENBLAS_NUM_THREADS") or os.environ.get("OMP_NUM_THREADS")
    blas = "unknown"
    try:
        info = np.show_config(mode="dicts")["Build Dependencies"]["blas"]
        blas = f"{info.get('name', '?')} {info.get('version', '')}".strip()
    except Exception:  # older numpy: no dict form
        pass
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return cores, threads, blas, cpu_model


def cpu_baseline(seconds_target=12.0):
    """Time the NumPy restatement of the reference's CPU path (fp32 SDPA per
    head) on a bounded sample of the headline workload: up to all 32 query
    heads at S=4096, repeated until about ``seconds_target`` seconds of CPU
    work, scaled to TFLOPS (median run)."""
    import numpy as np

    from oracle import attn_oracle as orc

    S, D, H_q, H_kv = 4096, 128, 32, 8
    q, k, v = orc.normal_fp16_inputs(1, H_q, H_kv, S, S, D, 1)
    q, k, v = q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)
    orc.sdpa_fp32_reference_style(q[:, :1], k[:, :1], v[:, :1])   # warm-up, 1 head
    t = time.perf_counter()
    orc.sdpa_fp32_reference_style(q[:, :1], k[:, :1], v[:, :1])
    one = time.perf_counter() - t
    ratio = H_q // H_kv
    n_heads = int(max(1, min(H_q, seconds_target / 3.0 / max(one, 1e-3))))
    n_heads = max(ratio, n_heads // ratio * ratio)  # whole KV groups
    runs = []
    t_all = time.perf_counter()
    while len(runs) < 3 or (time.perf_counter() - t_all < seconds_target and len(runs) < 50):
        t = time.perf_counter()
        orc.sdpa_fp32_reference_style(q[:, :n_heads], k[:, :n_heads // ratio],
                                      v[:, :n_heads // ratio])
        runs.append(time.perf_counter() - t)
    sec = statistics.median(runs)
    tflops = flops(1, n_heads, S, S, D) / sec / 1e12
    cores, threads, blas, cpu_model = host_info()
    return {
        "value": round(tflops, 4), "unit": "TFLOPS",
        "cores": int(threads) if threads and threads.isdigit() else cores,
        "kind": "port",
        "sample": (f"prefill S=4096 GQA D=128, {n_heads} of 32 query heads, fp32 NumPy SDPA "
                   f"(oracle.sdpa_fp32_reference_style = kernel_models/flash_attn.py:250-265), "
                   f"median of {len(runs)} runs = {sec:.2f} s ({sum(runs):.1f} s sampled); "
                   f"cpu '{cpu_model}', "
                   f"affinity {cores} cores, BLAS {blas}, BLAS threads {threads or 'default'}"),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--decode-sets", type=int, default=40,
                    help="distinct Q/K/V sets rotated through for the KV=4096 decode")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["prefill", "prefill_causal", "decode", "decode_b32",
                                       "decode_paged", "copy"],
                    default=None,
                    help="run one workload only (for rocprof counter passes); prints no JSON")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the attention forward shards by KV head with no "
              "communication, so every GPU would run the same kernels on its share",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import kernelfoundry_amd as kf

    if not torch.cuda.is_available():
        print("bench.py needs the MI355X GPU", file=sys.stderr)
        sys.exit(1)
    kf.load_library()
    steps, warmup = args.steps, args.warmup

    if args.only == "copy":
        # Plain copy of known size, for calibrating FETCH_SIZE / WRITE_SIZE.
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy: {steps} x {src.numel()} bytes", flush=True)
        return

    results = {}

    def run_prefill(S, H_kv=8, D=128, steps_=steps, check=None, causal=False, key_count=None,
                    passes=PASSES, B=1):
        sets = [_inputs(torch, B, 32, H_kv, S, S, D, 1234 + S)]
        lens = None if key_count is None else torch.full((1,), key_count, dtype=torch.int32, device="cuda")
        r = Runner(torch, kf, sets, D, flags=kf.KF_ATTN_CAUSAL if causal else 0, kv_lens=lens)
        ms, kern_mean, kern_med = time_steps(torch, r, steps_, warmup, passes)
        if causal:
            f = causal_flops(B, 32, S, D)
        else:
            f = flops(B, 32, S, S if key_count is None else key_count, D)
        out = {"S": S, "H_kv": H_kv, "D": D, "ms": ms, "tflops": f / (ms * 1e9),
               "frac": round(f / (ms * 1e9) / PEAK_FP16_TFLOPS, 4),
               "kernel_ms_mean": kern_mean, "kernel_tflops": f / (kern_mean * 1e9),
               "grid_blocks": r.plan.grid_blocks, "passes": passes}
        if causal:
            out["causal"] = True
        if key_count is not None:
            out["key_count"] = key_count
        if B > 1:
            out["B"] = B
        out["kernels"] = kf.kernel_names(B, S, S, 32, H_kv, D, causal=causal, masked=key_count is not None)
        if check:
            out["parity"] = parity_spot_check(torch, r, check, causal=causal)
        return out

    if args.only in (None, "prefill"):
        print("bench: prefill S=4096 GQA D=128", file=sys.stderr, flush=True)
        # The headline: exactly `steps` timed steps in one timed region.
        results["prefill"] = run_prefill(4096, check=[(0, 0), (0, 31)] if args.only is None else None,
                                         passes=1)
        if args.only:
            return

    if args.only in (None, "prefill_causal"):
        print("bench: causal prefill S=4096 GQA D=128", file=sys.stderr, flush=True)
        sets = [_inputs(torch, 1, 32, 8, 4096, 4096, 128, 1234 + 4096)]
        rc = Runner(torch, kf, sets, 128, flags=kf.KF_ATTN_CAUSAL)
        ms, kern_mean, _ = time_steps(torch, rc, steps, warmup, PASSES)
        if args.only:
            return
        f = causal_flops(1, 32, 4096, 128)
        results["prefill_causal"] = {
            "config": "configs[2] shape, causal (kf_attn_fwd_ex, bottom-right aligned)",
            "ms": round(ms, 5), "tflops": round(f / (ms * 1e9), 2),
            "kernel_ms_mean": round(kern_mean, 5), "kernel_tflops": round(f / (kern_mean * 1e9), 2),
            "algorithmic_flops_per_launch": f,
            "frac": round(f / (ms * 1e9) / PEAK_FP16_TFLOPS, 4),
            "kernels": kf.kernel_names(1, 4096, 4096, 32, 8, 128, causal=True),
            "parity": parity_spot_check(torch, rc, [(0, 0), (0, 31)], causal=True),
        }
        del rc

    def run_decode(B, kv, n_sets, D=128, H_kv=8):
        sets = [_inputs(torch, B, 32, H_kv, 1, kv, D, 99 + i) for i in range(n_sets)]
        r = Runner(torch, kf, sets, D)
        ms, kern_mean, kern_med = time_steps(torch, r, steps, warmup, PASSES)
        by = nbytes(B, 32, H_kv, 1, kv, D)
        out = {"B": B, "kv_len": kv, "D": D, "H_kv": H_kv, "sets_rotated": n_sets,
               "latency_us": ms * 1e3, "gbs": by / (ms * 1e6),
               "launch_us_mean": kern_mean * 1e3, "launch_gbs": by / (kern_mean * 1e6),
               "bytes": by, "path": r.plan.path, "splits": r.plan.num_splits}
        return out, r

    if args.only in (None, "decode"):
        print("bench: decode B=1 KV=4096", file=sys.stderr, flush=True)
        results["decode"], rdec = run_decode(1, 4096, args.decode_sets)
        if args.only:
            return
        results["decode"]["parity"] = parity_spot_check(torch, rdec, [(0, 0), (0, 17)])
        probe = load_probe(kf)
        print("bench: decode floors and graph replay", file=sys.stderr, flush=True)
        read_us, empty_us, read_bytes = decode_floors(torch, probe, rdec.sets, steps, warmup)
        results["decode"]["floor"] = {
            "read_us": round(read_us, 3),
            "read_gbs": round(read_bytes / (read_us * 1e3), 1),
            "read_bytes": read_bytes,
            "boundary_us": round(empty_us, 3),
            "note": ("read_us: kf_probe_read of the same K and V bytes over the same rotated sets, "
                     "timed back to back like the decode step (one launch, one round trip per "
                     "lane, no compute); boundary_us: an empty dispatch back to back, the cost of "
                     "one kernel boundary on the stream; the split decode step is two launches"),
        }
        try:
            g_us, g_ok = time_graph(torch, rdec)
            results["decode"]["graph"] = {"step_us": round(g_us, 3), "replays_bitwise_equal": g_ok,
                                          "note": "one pass over the rotated sets captured in one "
                                                  "HIP graph, replayed back to back"}
        except Exception as e:  # capture unsupported: report, keep the eager figures
            results["decode"]["graph"] = {"step_us": None, "error": str(e)[:200]}
        del rdec
    if args.only in (None, "decode_b32"):
        print("bench: decode B=32 KV=8192", file=sys.stderr, flush=True)
        results["decode_b32"], rb = run_decode(32, 8192, 1)
        if args.only:
            return
        results["decode_b32"]["parity"] = parity_spot_check(torch, rb, [(0, 0), (31, 31)])
        # The bandwidth a kernel that only reads the same 1.07 GB of K and V
        # reaches on this GPU: the ceiling the decode's roofline fraction is
        # measured against in practice.
        read_us, _, read_bytes = decode_floors(torch, load_probe(kf), rb.sets, steps, warmup)
        results["decode_b32"]["floor"] = {
            "read_us": round(read_us, 2), "read_gbs": round(read_bytes / (read_us * 1e3), 1),
            "read_bytes": read_bytes,
            "decode_vs_read": round(read_us / results["decode_b32"]["latency_us"], 4),
            "note": "kf_probe_read of the same K and V bytes (16-byte non-temporal loads, no compute)"}
        del rb

    if args.only in (None, "decode_paged"):
        print("bench: paged decode B=32 KV=8192 page 16", file=sys.stderr, flush=True)
        results["decode_paged"] = run_paged_decode(torch, kf, steps, warmup, args.only is None)
        if args.only:
            return
        print("bench: paged decode B=1 KV=4096 page 16", file=sys.stderr, flush=True)
        results["decode_paged_c1"] = run_paged_decode(torch, kf, steps, warmup, True, B=1, kv=4096,
                                                      label="configs[1]")

    print("bench: decode sweep", file=sys.stderr, flush=True)
    probe = load_probe(kf)
    decode_sweep = []
    # The reference bench's decode shapes (tests/bench_flash_attn.cu:154-159,
    # 181-182), each rotated over > 512 MB of distinct Q/K/V sets so that a
    # step reads HBM, not the Infinity Cache copy of an earlier step.
    for (B, kv, H_kv) in ((1, 512, 8), (1, 1024, 8), (1, 2048, 8), (1, 4096, 8), (8, 512, 8),
                          (8, 1024, 8), (1, 512, 1), (1, 1024, 1)):
        by = nbytes(B, 32, H_kv, 1, kv, 128)
        n_sets = int(min(4000, math.ceil(ROTATE_BYTES / by)))
        d, r = run_decode(B, kv, n_sets, D=128, H_kv=H_kv)
        read_us, empty_us, _ = decode_floors(torch, probe, r.sets, steps, warmup)
        decode_sweep.append({
            "B": B, "H_q": 32, "H_kv": H_kv, "D": 128, "kv_len": kv, "sets_rotated": n_sets,
            "latency_us": round(d["latency_us"], 3), "hbm_gbs": round(d["gbs"], 1),
            "frac": round(d["gbs"] / PEAK_HBM_GBS, 4), "bytes": by,
            "floor_read_us": round(read_us, 3), "boundary_us": round(empty_us, 3),
            "passes": PASSES, "kernels": kf.kernel_names(B, 1, kv, 32, H_kv, 128),
            "parity": parity_spot_check(torch, r, [(0, 0), (B - 1, 31)])})
        del r
        torch.cuda.empty_cache()

    # configs[1]'s KV=4096 decode at larger batches (the north star's "KV=4096
    # decode" names no batch): B=1 is latency-bound, from a few sequences on
    # the step streams HBM.  Rotated like the rows above.
    print("bench: decode KV=4096 by batch", file=sys.stderr, flush=True)
    kv4096_batch = []
    for B in (2, 4, 8, 16, 32):
        by = nbytes(B, 32, 8, 1, 4096, 128)
        n_sets = int(min(4000, math.ceil(ROTATE_BYTES / by)))
        d, r = run_decode(B, 4096, n_sets)
        kv4096_batch.append({
            "B": B, "kv_len": 4096, "H_q": 32, "H_kv": 8, "D": 128, "sets_rotated": n_sets,
            "latency_us": round(d["latency_us"], 3), "hbm_gbs": round(d["gbs"], 1),
            "frac": round(d["gbs"] / PEAK_HBM_GBS, 4), "bytes": by, "passes": PASSES,
            "kernels": kf.kernel_names(B, 1, 4096, 32, 8, 128),
            "parity": parity_spot_check(torch, r, [(0, 0), (B - 1, 31)])})
        del r
        torch.cuda.empty_cache()

    print("bench: sweep", file=sys.stderr, flush=True)
    sweep = [run_prefill(S) for S in (512, 1024, 2048)]
    sweep.append(run_prefill(2048, H_kv=1, D=64))
    sweep.append(run_prefill(4096, H_kv=8, D=256))
    sweep.append(run_prefill(4096, H_kv=8, D=256, causal=True))
    sweep.extend(run_prefill(S, H_kv=8, D=256) for S in (512, 1024))
    # configs[2] with a per-sequence key count (kf_attn_fwd_ex kv_lens): the
    # sequence uses its first 4000 of the 4096 allocated key rows.
    sweep.append(run_prefill(4096, key_count=4000))
    # Causal prefill with two wide workgroups per CU or more (the wide
    # layout's causal kernel): 2 x 4096 and 1 x 8192 queries, 32 / 8 heads.
    sweep.append(run_prefill(4096, causal=True, B=2, check=[(0, 0), (1, 31)]))
    sweep.append(run_prefill(8192, causal=True, check=[(0, 31)]))
    # Chunked prefill (a short chunk of query rows against a long cache): the
    # split prefill's KV partitions + split merge.
    for q, kv, D in ((16, 8192, 128), (64, 4096, 128), (128, 8192, 128), (256, 16384, 128),
                     (64, 4096, 256)):
        cs = [_inputs(torch, 1, 32, 8, q, kv, D, 77 + q + kv)]
        rq = Runner(torch, kf, cs, D)
        ms, kern_mean, _ = time_steps(torch, rq, steps, warmup, PASSES)
        f = flops(1, 32, q, kv, D)
        sweep.append({"q_len": q, "kv_len": kv, "H_kv": 8, "D": D, "ms": ms,
                      "tflops": f / (ms * 1e9), "kernel_ms_mean": kern_mean,
                      "grid_blocks": rq.plan.grid_blocks, "num_splits": rq.plan.num_splits,
                      "passes": PASSES, "kernels": kf.kernel_names(1, q, kv, 32, 8, D),
                      "parity": parity_spot_check(torch, rq, [(0, 0), (0, 31)])})
        del rq
    # configs[3] decode: 0.54 MB per set, rotated over > 512 MB of distinct
    # sets like configs[1], so each step reads HBM, not the Infinity Cache.
    dq, _ = run_decode(1, 2048, 960, D=64, H_kv=1)
    sweep.append({"mqa_decode_d64": dq})
    torch.cuda.empty_cache()

    # The reference bench's prefill rows not timed above (short prefill
    # S = 64 / 128 / 256 and B = 8 x 64, tests/bench_flash_attn.cu:162-165;
    # D = 64 at S = 1024, :174; MQA D = 128 prefill at S = 512 / 1024,
    # :179-180), each rotated over > 512 MB of distinct input sets so that
    # every step reads its inputs from HBM, and spot-checked against the oracle.
    print("bench: reference bench rows", file=sys.stderr, flush=True)
    extra_prefill = {}
    for (B, S, H_kv, D) in ((1, 64, 8, 128), (1, 128, 8, 128), (1, 256, 8, 128), (8, 64, 8, 128),
                            (1, 1024, 8, 64), (1, 512, 1, 128), (1, 1024, 1, 128)):
        per_set = B * 32 * S * D * (2 + 4) + 2 * B * H_kv * S * D * 2
        n_sets = int(min(2000, max(1, math.ceil(ROTATE_BYTES / per_set))))
        sets = [_inputs(torch, B, 32, H_kv, S, S, D, 500 + 7 * i + S) for i in range(n_sets)]
        rr = Runner(torch, kf, sets, D)
        ms, kern_mean, _ = time_steps(torch, rr, steps, warmup, PASSES)
        f = flops(B, 32, S, S, D)
        extra_prefill[(B, S, H_kv, D)] = {
            "ms": ms, "tflops": f / (ms * 1e9), "sets_rotated": n_sets,
            "kernels": kf.kernel_names(B, S, S, 32, H_kv, D),
            "parity": parity_spot_check(torch, rr, [(0, 0), (B - 1, 31)])}
        del rr, sets
        torch.cuda.empty_cache()

    pre = results["prefill"]
    dec = results["decode"]
    b32 = results["decode_b32"]
    traffic, traffic_note = committed_traffic()

    # Every row of the reference bench (tests/bench_flash_attn.cu:154-182) with
    # its MI355X figure, beside the reference's published RTX 5070 time where
    # README.md:46-58 has one.
    by_sweep = {(1, s["S"], s["H_kv"], s["D"]): s for s in sweep
                if "S" in s and not s.get("causal") and "key_count" not in s}
    by_sweep[(1, 4096, 8, 128)] = pre
    ref_ms = {(1, 512, 8, 128): 0.305, (1, 1024, 8, 128): 1.028, (1, 2048, 8, 128): 3.866,
              (1, 4096, 8, 128): 14.279}
    ref_dec_ms = {512: 0.040, 1024: 0.078, 2048: 0.165, 4096: 0.303}
    rows = []
    dec_rows = {(d["B"], d["kv_len"], d["H_kv"]): d for d in decode_sweep}
    for line_no, (B, kv, H_kv) in zip((154, 155, 156, 157, 158, 159, 181, 182),
                                      ((1, 512, 8), (1, 1024, 8), (1, 2048, 8), (1, 4096, 8),
                                       (8, 512, 8), (8, 1024, 8), (1, 512, 1), (1, 1024, 1))):
        d = dec_rows[(B, kv, H_kv)]
        row = {"ref": line_no, "B": B, "q": 1, "kv": kv, "Hkv": H_kv, "D": 128,
               "us": d["latency_us"], "gbs": d["hbm_gbs"]}
        if B == 1 and H_kv == 8:
            row["ref_ms"] = ref_dec_ms[kv]
        rows.append(row)
    for line_no, key in ((162, (1, 64, 8, 128)), (163, (1, 128, 8, 128)), (164, (1, 256, 8, 128)),
                         (165, (8, 64, 8, 128)), (168, (1, 512, 8, 128)), (169, (1, 1024, 8, 128)),
                         (170, (1, 2048, 8, 128)), (171, (1, 4096, 8, 128)),
                         (174, (1, 1024, 8, 64)), (175, (1, 1024, 8, 128)), (176, (1, 1024, 8, 256)),
                         (179, (1, 512, 1, 128)), (180, (1, 1024, 1, 128))):
        s = extra_prefill.get(key) or by_sweep[key]
        B, S, H_kv, D = key
        row = {"ref": line_no, "B": B, "q": S, "kv": S, "Hkv": H_kv, "D": D,
               "us": round(s["ms"] * 1e3, 2), "tflops": round(s["tflops"], 1)}
        if key in ref_ms:
            row["ref_ms"] = ref_ms[key]
        rows.append(row)
    rows.sort(key=lambda r: r["ref"])

    line = {
        "metric": METRIC,
        "value": round(pre["tflops"], 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "clock_settle_s": SETTLE_S,
        "ms_per_step": round(pre["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(pre["tflops"] / REF_PREFILL_S4096_TFLOPS, 2),
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "GQA prefill non-causal, fp16 Q/K/V N(0,1), fp32 O",
                   "B": 1, "H_q": 32, "H_kv": 8, "D": 128, "q_len": 4096, "kv_len": 4096,
                   "baseline_config": "configs[2]"},
        "roofline": {
            "bound": "mfma",
            "kernel": kf.kernel_names(1, 4096, 4096, 32, 8, 128),
            "achieved": round(pre["tflops"], 2),
            "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(pre["tflops"] / PEAK_FP16_TFLOPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
            "kernel_sources_sha256": source_sha256(),
            "algorithmic_flops_per_launch": flops(1, 32, 4096, 4096, 128),
            "launch_ms": round(pre["ms"], 5),
            "launch_ms_event_pairs": round(pre["kernel_ms_mean"], 5),
            "note": ("achieved = algorithmic FLOPs / the kernel's launch duration from the timed "
                     "region (one launch per step, back to back between two HIP events on the "
                     "launch stream); launch_ms_event_pairs is the mean of an event pair around "
                     "every launch, which adds about 1.5 us of event overhead per launch"),
        },
        "prefill_causal": results["prefill_causal"],
        "decode_b32": {
            "config": "configs[4]: B=32 H_q=32 H_kv=8 D=128 q_len=1 kv_len=8192",
            "latency_us": round(b32["latency_us"], 2),
            "hbm_gbs": round(b32["gbs"], 1),
            "roofline": {"bound": "hbm", "achieved": round(b32["gbs"], 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(b32["gbs"] / PEAK_HBM_GBS, 4),
                         "bytes_per_launch": b32["bytes"]},
            "path": b32["path"], "splits": b32["splits"],
            "floor": b32["floor"],
            "parity": b32["parity"],
        },
        "decode_paged": results["decode_paged"],
        "decode_paged_c1": results["decode_paged_c1"],
        "decode_sweep": decode_sweep,
        "decode_kv4096_by_batch": kv4096_batch,
        "sweep": sweep,
        "parity": pre.get("parity"),
    }
    if not args.no_cpu_baseline:
        print("bench: cpu baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline()
        print("bench: cpu baseline, tiled model at configs[0]", file=sys.stderr, flush=True)
        line["cpu_baseline_c1_tiled"] = cpu_baseline_tiled_c1()
    line["reference_bench"] = rows
    # configs[1] last, compact, so that the end of the line (what a log tail
    # keeps) carries the decode half of the metric.
    line["decode"] = {
        "config": "configs[1]: B=1 H_q=32 H_kv=8 D=128 q_len=1 kv_len=4096",
        "latency_us": round(dec["latency_us"], 3),
        "hbm_gbs": round(dec["gbs"], 1),
        "roofline": {"bound": "hbm", "achieved": round(dec["gbs"], 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(dec["gbs"] / PEAK_HBM_GBS, 4),
                     "bytes_per_launch": dec["bytes"]},
        "floor": {"read_us": dec["floor"]["read_us"], "read_gbs": dec["floor"]["read_gbs"],
                  "boundary_us": dec["floor"]["boundary_us"]},
        "graph_step_us": dec["graph"].get("step_us"),
        "launch_us_mean": round(dec["launch_us_mean"], 3),
        "sets_rotated": dec["sets_rotated"], "passes": PASSES,
        "kernels": kf.kernel_names(1, 1, 4096, 32, 8, 128),
        "parity_max_abs": dec["parity"]["max_abs"], "parity_rel_l2": dec["parity"]["rel_l2"],
        # [B, us per step, fraction of HBM peak] of the same decode at larger batches
        "kv4096_by_batch": [[1, round(dec["latency_us"], 2), round(dec["gbs"] / PEAK_HBM_GBS, 3)]] + [
            [b["B"], round(b["latency_us"], 2), round(b["frac"], 3)] for b in kv4096_batch],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
