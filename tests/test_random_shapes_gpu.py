"""Seeded random-shape parity sweep of kf_attn_fwd_ex on the GPU.

Shapes, masks and output formats are drawn from a fixed seed so that, taken
together, they cross every dispatch the planner makes: the short-split decode
kernel (32- and 64-key splits) and the streaming decode kernel, each with and
without the split merge, and the prefill kernel in every workgroup layout
(8 waves x 256 rows, two KV groups of 8 or 4 waves, four KV groups of 8
waves, 4 and 2 waves; D = 256 with 4 waves) and the wide prefill kernel (8
waves x 64 rows at D = 64 / 128, 8 x 32 at D = 256, and at D = 256 its two
KV groups of 4 waves), the split prefill (KV partitions + the split merge,
at every head dimension), with causal masking, per-sequence key counts (empty
sequences included), ragged lengths and every head dimension.  Each case is
compared with oracle/attn_oracle.py's fp64 ``sdpa`` on the same fp16 inputs at
the north-star bar (max |got - ref| <= 2e-3, ||got - ref|| / ||ref|| <= 1e-2;
Mi to 1e-4, Li to 1e-3 relative; rows without keys exactly O = 0, Mi = -inf,
Li = 0).  Sizes keep the fp64 oracle to a few seconds per case.
"""
import numpy as np
import pytest

from oracle import attn_oracle as orc
from tests._parity import run_and_check

pytestmark = pytest.mark.gpu


def _cases(n=40, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([16, 64, 128, 128, 256]))
        H_kv = int(rng.choice([1, 2, 4, 8]))
        H_q = H_kv * int(rng.choice([1, 2, 4, 8]))
        B = int(rng.integers(1, 4))
        if i % 3 == 0:
            q_len = int(rng.integers(1, 9))                  # decode-sized
        else:
            q_len = int(rng.integers(9, 700))
        kv_len = int(rng.integers(1, 1500))
        causal = bool(rng.random() < 0.4)
        kv_lens = None
        if rng.random() < 0.4:
            kv_lens = [int(x) for x in rng.integers(0, kv_len + 1, size=B)]
        # keep the fp64 oracle cheap
        while B * H_q * q_len * kv_len * D > 6e9:
            kv_len = max(1, kv_len // 2)
            if kv_lens is not None:
                kv_lens = [min(x, kv_len) for x in kv_lens]
        out.append((B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens, int(rng.integers(1 << 30))))
    # Layouts random small shapes rarely reach: decode without split (at most
    # 32 keys), 8-wave workgroups (a grid of >= 256 workgroups x 256 rows),
    # the streaming decode kernel (more than 1024 short splits) with and
    # without the merge, 64-key short splits and a merge over 256 splits.
    out.append((3, 8, 8, 1, 30, 128, True, [30, 0, 17], 11))
    out.append((2, 64, 8, 1024, 200, 64, True, [200, 150], 12))
    out.append((16, 32, 8, 1, 1100, 128, False, None, 13))
    out.append((24, 8, 8, 1, 1500, 64, True, [int(x) for x in rng.integers(0, 1501, size=24)], 14))
    out.append((300, 8, 8, 1, 100, 16, False, None, 15))
    out.append((32, 8, 8, 1, 200, 16, True, [int(x) for x in rng.integers(0, 201, size=32)], 16))
    out.append((1, 4, 2, 1, 8192, 128, False, None, 17))
    out.append((1, 4, 2, 1, 300, 256, True, [257], 18))
    # Four KV groups (grid of < 256 workgroups x 128 rows, >= 512 keys): a
    # ragged last group, and key counts that leave groups without keys.
    out.append((1, 16, 4, 300, 900, 128, False, None, 19))
    out.append((2, 16, 2, 200, 1100, 64, True, [1100, 70], 20))
    # The wide prefill kernel (unmasked, 512-row workgroups in fewer rounds
    # than the 256-row kernel's): D = 128 and 64, ragged key counts.
    out.append((32, 32, 8, 90, 150, 128, False, None, 21))
    out.append((16, 16, 4, 300, 333, 64, False, None, 22))
    # D = 256: the wide kernel (256-row workgroups, causal) and its two-KV-group
    # form unmasked (random D = 256 shapes reach it masked).
    out.append((8, 32, 8, 150, 200, 256, True, None, 23))
    out.append((1, 8, 2, 200, 700, 256, False, None, 24))
    # The split prefill (few query rows per KV head against many keys: KV
    # partitions + the split merge), drawn from a second stream so the cases
    # above stay as they are: every head dimension, masks and key counts.
    rng2 = np.random.default_rng(seed + 1)
    for i in range(8):
        D = [16, 64, 128, 256][i % 4]
        H_kv = int(rng2.choice([1, 2, 4, 8]))
        H_q = H_kv * int(rng2.choice([4, 8]))
        B = int(rng2.integers(1, 3))
        q_len = int(rng2.integers(9, 65))
        kv_len = int(rng2.integers(2000, 9000))
        causal = bool(rng2.random() < 0.4)
        kv_lens = [int(x) for x in rng2.integers(0, kv_len + 1, size=B)] if rng2.random() < 0.4 else None
        out.append((B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens, int(rng2.integers(1 << 30))))
    return out


CASES = _cases()


def _layout(kf, B, H_q, H_kv, q_len, kv_len, D, causal=False, masked=False):
    """(path, kernel) for decode, kernel "short32" / "short64" (one wave per
    split of that many keys) or "stream"; ("prefill", waves, kv_groups) for
    prefill, read from the kernel name (kf_attn_prefill_kernel<D, mask,
    waves, kv_groups>), or ("prefill", "wide", kv_groups) for
    kf_attn_prefill_wide_kernel<D, mask, kv_groups, causal two-block layout>."""
    p = kf.plan(B, q_len, kv_len, H_q, H_kv, D)
    if p.path not in ("prefill", "prefill_split"):
        return (p.path, f"short{p.kv_per_split}" if p.splits_per_block == 4 else "stream")
    name = kf.kernel_names(B, q_len, kv_len, H_q, H_kv, D, causal=causal, masked=masked)
    if p.path == "prefill_split":
        name = name.split(" + ")[0]
        if name.startswith("kf_attn_prefill_parts_kernel"):
            return ("prefill_split", "parts")
        waves, groups = (int(x) for x in name.rstrip(">").split(",")[-2:])
        return ("prefill_split", waves, groups)
    if name.startswith("kf_attn_prefill_wide"):  # <D, mask, kv_groups, causal two-block layout>
        return ("prefill", "wide", int(name.rstrip(">").split(",")[2]))
    waves, groups = (int(x) for x in name.rstrip(">").split(",")[-2:])
    return ("prefill", waves, groups)


def test_sweep_covers_every_dispatch():
    """The drawn cases reach every kernel layout the planner chooses."""
    import kernelfoundry_amd as kf
    seen = {_layout(kf, *c[:7], c[7] is not None) for c in CASES}
    want = {("decode", "short32"), ("decode_split", "short32"), ("decode_split", "short64"),
            ("decode", "stream"), ("decode_split", "stream"),
            ("prefill", 8, 1), ("prefill", 8, 2), ("prefill", 8, 4), ("prefill", 4, 2), ("prefill", 4, 1),
            ("prefill", 2, 1), ("prefill", "wide", 1), ("prefill", "wide", 2),
            ("prefill_split", 8, 4), ("prefill_split", 2, 1), ("prefill_split", "parts")}
    assert want <= seen, sorted(seen)
    # The split merge at its widest: 256 partials per row (4 columns per wave).
    assert any(kf.plan(c[0], c[3], c[4], c[1], c[2], c[5]).num_splits == 256 for c in CASES)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_q{}_kv{}_D{}_c{}_{}".format(
    c[0], c[1], c[2], c[3], c[4], c[5], int(c[6]), "lens" if c[7] is not None else "full"))
def test_random_shape_parity(case):
    run_and_check(*case)
