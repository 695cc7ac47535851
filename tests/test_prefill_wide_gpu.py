"""GPU parity of the wide prefill kernel (kf_attn_prefill_wide_kernel<D, kMask, KS>: 8
waves x 64 query rows, 512 rows per workgroup, at D = 64 and 128; 8 waves x
32 rows at D = 256; KS = 2, D = 256 only: two KV groups of 4 waves on 128
rows, each on its half of every row's keys).

The planner runs it for unmasked calls when its grid finishes in less time
than the narrower kernel's (rounds of one workgroup per CU); every shape
here is chosen so that it does (asserted through kf.kernel_names), and so
that its edge cases are hit: padding query rows (rows per KV head % 512 !=
0, fewer than 512 rows), a ragged last tile (kv_len % 32 != 0), an odd tile
count (the last 64-row stage holds one tile), a partial last stage, a single
key, one to many stages, GQA ratios 1, 4 and 32, several row tiles per KV
head, and D = 256 with its LDS offsets derived by XOR.  O, Mi and Li are
compared with oracle/attn_oracle.py's fp64 ``sdpa`` on the same fp16 inputs
to the north-star bar (max |got - ref| <= 2e-3, ||got - ref|| / ||ref|| <=
1e-2; Mi to 1e-4, Li to 1e-3 relative).

The wide kernel computes every row with the same operation order as the
256-row kernel (the 128-row 4-wave kernel at D = 256), so its output must
equal, bit for bit, that kernel's on the same inputs (PAIRS, below), and
the masked wide kernel with every sequence's key count equal to kv_len must
give the unmasked one's bits.

Masked calls run kf_attn_prefill_wide_kernel<D, true, 1, false> when the planner
chooses the wide grid: at D = 256 causal and/or per-sequence key counts, at
D = 64 / 128 key counts; causal calls at D = 64 / 128 run
kf_attn_prefill_wide_kernel<D, true, 1, true> (each wave on 64 consecutive
rows) when the wide grid has two workgroups per CU or more and the rows see
2048 keys on average, else the 256-row kernel (CAUSAL_PAIRS, below).
MASKED_CASES cover causal with q_len = kv_len, kv_len > q_len and q_len >
kv_len (rows without keys), key counts with an empty sequence and a single
key, both together, and GQA ratio 16, against the oracle with rows without
keys exactly O = 0, Mi = -inf, Li = 0.  PAIRS check the wide kernels
against the 32-row kernel bit for bit through the planner's own choice
(B = 1 plans the 32-row kernel, B = 2 the wide one, at the same shape).

GROUP_CASES: the KV-group kernel (D = 256 grids that the 256-row tiles would
leave with idle CUs, from 256 keys on), unmasked and masked, against the
oracle: an odd tile count (the second group's last tile wholly past the
keys), a group with no key at all (key count 31, causal rows near the top),
empty sequences and rows, padding rows, MHA / GQA / MQA, and (max-size
test) keys at the 32-bit offset limit.  Its groups merge in another order
than any one-group kernel, so it is held to the oracle bar, not bit
equality; the masked kernel with key counts = kv_len still gives the
unmasked one's bits.
"""
import numpy as np
import pytest

from oracle import attn_oracle as orc
from tests._parity import run_and_check

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    return torch


CASES = [
    # B, H_q, H_kv, q_len, kv_len, D           what it hits
    (32, 32, 8, 100, 77, 128),     # 400 rows (< 512, padding), ragged tail, odd tiles, partial stage
    (32, 32, 8, 100, 1, 128),      # one key: one tile, 31 keys masked
    (16, 32, 8, 256, 160, 128),    # two row tiles per head, 2.5 stages
    (4, 64, 64, 1024, 96, 128),    # MHA (ratio 1), 1.5 stages
    (8, 32, 1, 512, 300, 128),     # MQA (ratio 32): 16384 rows, 32 row tiles, ragged
    (4, 32, 8, 2048, 1000, 128),   # 16 row tiles per head, 16 stages, ragged
    (32, 32, 8, 100, 77, 64),      # D = 64 (block-1 Q^T in registers)
    (8, 32, 1, 512, 513, 64),      # D = 64 MQA, one key into the last stage
    (16, 16, 8, 150, 333, 256),    # D = 256 (8 waves x 32 rows): 300 rows, ragged
    (8, 8, 8, 1024, 65, 256),      # D = 256 MHA, one key in the last tile
    (8, 32, 1, 256, 200, 256),     # D = 256 MQA, 32 row tiles per head
]


def _ids(c):
    return "B{}_Hq{}_Hkv{}_q{}_kv{}_D{}".format(*c)


def _inputs(B, H_q, H_kv, q_len, kv_len, D, seed):
    torch = _torch()
    q16, k16, v16 = orc.normal_fp16_inputs(B, H_q, H_kv, q_len, kv_len, D, seed)
    dev = (torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (q16, k16, v16))
    return (q16, k16, v16), tuple(dev)


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_wide_prefill_matches_oracle(case):
    import kernelfoundry_amd as kf
    torch = _torch()
    B, H_q, H_kv, q_len, kv_len, D = case
    names = kf.kernel_names(B, q_len, kv_len, H_q, H_kv, D)
    print("case", case, names, flush=True)
    assert names == f"kf_attn_prefill_wide_kernel<{D}, false, 1, false>", names
    (q16, k16, v16), (Q, K, V) = _inputs(B, H_q, H_kv, q_len, kv_len, D, 11 + kv_len)
    O, Mi, Li = kf.attn_fwd(Q, K, V, return_stats=True)
    torch.cuda.synchronize()
    O, Mi, Li = O.cpu().numpy(), Mi.cpu().numpy(), Li.cpu().numpy()
    Or, Mr, Lr = orc.sdpa(q16, k16, v16)
    assert np.isfinite(O).all(), "non-finite O"
    ok, max_abs, rel = orc.within_tolerance(O, Or)
    assert ok, f"max_abs={max_abs:.3g} rel={rel:.3g}"
    assert np.abs(Mi - Mr).max() <= 1e-4, "Mi"
    assert (np.abs(Li - Lr) / np.abs(Lr)).max() <= 1e-3, "Li"


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[4], CASES[6], CASES[8], CASES[10]],
                         ids=_ids)
def test_wide_masked_without_masking_equals_unmasked_bitwise(case):
    import kernelfoundry_amd as kf
    torch = _torch()
    B, H_q, H_kv, q_len, kv_len, D = case
    masked = kf.kernel_names(B, q_len, kv_len, H_q, H_kv, D, masked=True)
    print("case", case, masked, flush=True)
    assert masked == f"kf_attn_prefill_wide_kernel<{D}, true, 1, false>", masked
    _, (Q, K, V) = _inputs(B, H_q, H_kv, q_len, kv_len, D, 5)
    full = torch.full((B,), kv_len, dtype=torch.int32, device="cuda")
    Ow, Mw, Lw = kf.attn_fwd(Q, K, V, return_stats=True)
    On, Mn, Ln = kf.attn_fwd(Q, K, V, return_stats=True, kv_lens=full)
    torch.cuda.synchronize()
    assert torch.equal(Ow, On), f"O differs: max {(Ow - On).abs().max().item():.3g}"
    assert torch.equal(Mw, Mn) and torch.equal(Lw, Ln), "Mi / Li differ"


MASKED_CASES = [
    # B, H_q, H_kv, q_len, kv_len, causal, kv_lens, D         what it hits
    (4, 16, 4, 600, 600, True, None, 256),                     # causal, ragged row tiles
    (4, 16, 4, 600, 777, True, None, 256),                     # causal, kv_len > q_len
    (4, 16, 4, 700, 500, True, None, 256),                     # causal, 200 rows without keys
    (4, 16, 4, 600, 777, False, [777, 0, 31, 500], 256),       # key counts, an empty sequence
    (4, 16, 4, 640, 700, True, [700, 129, 0, 640], 256),       # causal + key counts
    (4, 32, 2, 300, 300, True, None, 256),                     # GQA ratio 16, causal
    (4, 32, 8, 600, 777, False, [777, 0, 31, 500], 128),       # two row blocks per wave: key counts
    (4, 32, 8, 600, 777, False, [1, 777, 64, 65], 64),         # D = 64 (pipelined loop), key counts
]


def _mids(c):
    return "B{}_Hq{}_Hkv{}_q{}_kv{}_c{}_{}_D{}".format(*c[:5], int(c[5]), "lens" if c[6] is not None else "full",
                                                     c[7])


@pytest.mark.parametrize("case", MASKED_CASES, ids=_mids)
def test_wide_masked_prefill_matches_oracle(case):
    import kernelfoundry_amd as kf
    B, H_q, H_kv, q_len, kv_len, causal, kv_lens, D = case
    name = kf.kernel_names(B, q_len, kv_len, H_q, H_kv, D, causal=causal, masked=kv_lens is not None)
    print("case", case, name, flush=True)
    assert name == f"kf_attn_prefill_wide_kernel<{D}, true, 1, false>", name
    run_and_check(B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens, 300 + q_len)


# At q_len = 2048 the planner runs the 256-row kernel (the 128-row one at
# D = 256, below 256 keys) for B = 1 and the wide kernel for B = 2: batch 0
# of the B = 2 call holds the B = 1 call's inputs, so its O, Mi and Li must
# be the same bits.
PAIRS = [
    # D, H_q, H_kv, kv_len, causal, batch-0 key count (None: unmasked)
    (128, 32, 8, 2048, False, None),
    (128, 32, 8, 2048, False, 1500),
    (64, 32, 8, 2048, False, None),
    (64, 32, 8, 2048, False, 777),
    (256, 16, 4, 200, False, None),
    (256, 16, 4, 255, False, 150),
    (256, 16, 4, 255, True, None),     # rows 1793.. see keys
]


@pytest.mark.parametrize("case", PAIRS, ids=lambda c: "D{}_Hq{}_Hkv{}_kv{}_c{}_{}".format(
    c[0], c[1], c[2], c[3], int(c[4]), "full" if c[5] is None else f"k{c[5]}"))
def test_wide_and_narrow_kernels_agree_bitwise(case):
    import kernelfoundry_amd as kf
    torch = _torch()
    D, H_q, H_kv, kv, causal, k0 = case
    S = 2048
    masked = k0 is not None
    n1 = kf.kernel_names(1, S, kv, H_q, H_kv, D, causal=causal, masked=masked)
    n2 = kf.kernel_names(2, S, kv, H_q, H_kv, D, causal=causal, masked=masked)
    print("case", case, n1, "|", n2, flush=True)
    assert n1.startswith("kf_attn_prefill_kernel<") and n2.startswith("kf_attn_prefill_wide_kernel<"), (n1, n2)
    assert n2.endswith(", 1, false>"), n2  # one KV group: the 32-row kernel's operation order
    _, (Q, K, V) = _inputs(2, H_q, H_kv, S, kv, D, 77)
    l1 = torch.tensor([k0], dtype=torch.int32, device="cuda") if masked else None
    l2 = torch.tensor([k0, kv - 5], dtype=torch.int32, device="cuda") if masked else None
    O1, M1, L1 = kf.attn_fwd(Q[:1].contiguous(), K[:1].contiguous(), V[:1].contiguous(), return_stats=True,
                             causal=causal, kv_lens=l1)
    O2, M2, L2 = kf.attn_fwd(Q, K, V, return_stats=True, causal=causal, kv_lens=l2)
    torch.cuda.synchronize()
    assert torch.equal(O1[0], O2[0]), f"O differs: max {(O1[0] - O2[0]).abs().max().item():.3g}"
    assert torch.equal(M1[0], M2[0]) and torch.equal(L1[0], L2[0]), "Mi / Li differ"


GROUP_CASES = [
    # B, H_q, H_kv, q_len, kv_len, causal, kv_lens           what it hits
    (1, 16, 4, 512, 512, False, None),                   # 16 tiles: 8 per group
    (1, 16, 4, 300, 333, False, None),                   # 11 tiles: group 1's last past the keys; padding rows
    (2, 8, 8, 256, 256, False, None),                    # MHA, 256 keys (the smallest KV-group case)
    (1, 32, 1, 520, 1000, False, None),                  # MQA, 16640 rows (130 row tiles: no KV partitions), ragged keys
    (2, 16, 4, 257, 257, False, None),                   # 9 tiles, group 1 from key 160
    (1, 16, 4, 600, 600, True, None),                    # causal, ragged row tiles
    (1, 16, 4, 600, 777, True, None),                    # causal, kv_len > q_len
    (1, 16, 4, 700, 500, True, None),                    # causal, 200 rows without keys
    (4, 16, 4, 300, 777, False, [777, 0, 31, 500]),      # key counts: empty; 31 keys (group 1 has none)
    (4, 16, 4, 300, 700, True, [700, 129, 0, 640]),      # causal + key counts
    (1, 32, 2, 300, 300, True, None),                    # GQA ratio 16, causal
]


def _gids(c):
    return "B{}_Hq{}_Hkv{}_q{}_kv{}_c{}_{}".format(*c[:5], int(c[5]), "lens" if c[6] is not None else "full")


@pytest.mark.parametrize("case", GROUP_CASES, ids=_gids)
def test_kv_group_wide_prefill_matches_oracle(case):
    import kernelfoundry_amd as kf
    B, H_q, H_kv, q_len, kv_len, causal, kv_lens = case
    mask = causal or kv_lens is not None
    name = kf.kernel_names(B, q_len, kv_len, H_q, H_kv, 256, causal=causal, masked=kv_lens is not None)
    print("case", case, name, flush=True)
    assert name == f"kf_attn_prefill_wide_kernel<256, {'true' if mask else 'false'}, 2, false>", name
    run_and_check(B, H_q, H_kv, q_len, kv_len, 256, causal, kv_lens, 900 + kv_len)


@pytest.mark.parametrize("case", [c for c in GROUP_CASES if not c[5] and c[6] is None], ids=_gids)
def test_kv_group_masked_without_masking_equals_unmasked_bitwise(case):
    import kernelfoundry_amd as kf
    torch = _torch()
    B, H_q, H_kv, q_len, kv_len = case[:5]
    masked = kf.kernel_names(B, q_len, kv_len, H_q, H_kv, 256, masked=True)
    print("case", case, masked, flush=True)
    assert masked == "kf_attn_prefill_wide_kernel<256, true, 2, false>", masked
    _, (Q, K, V) = _inputs(B, H_q, H_kv, q_len, kv_len, 256, 6)
    full = torch.full((B,), kv_len, dtype=torch.int32, device="cuda")
    Ow, Mw, Lw = kf.attn_fwd(Q, K, V, return_stats=True)
    On, Mn, Ln = kf.attn_fwd(Q, K, V, return_stats=True, kv_lens=full)
    torch.cuda.synchronize()
    assert torch.equal(Ow, On), f"O differs: max {(Ow - On).abs().max().item():.3g}"
    assert torch.equal(Mw, Mn) and torch.equal(Lw, Ln), "Mi / Li differ"


# Causal calls at D = 64 / 128: at q_len = 4096 (8192 at 16 / 8 heads) the
# planner runs the 256-row kernel for B = 1 (one wide workgroup per CU) and
# the wide layout's causal kernel for B = 2.  Each row sees the same tiles in
# the same order in both (the wide kernel computes, for a wave's first 32
# rows, tiles wholly masked for them, which add exactly nothing), so batch 0
# of the B = 2 call must equal the B = 1 call bit for bit, O, Mi and Li,
# also with key counts (rows without keys: O = 0, Mi = -inf, Li = 0) and with
# row tiles that straddle heads (q_len = 5184 = 10.125 x 512).
CAUSAL_PAIRS = [
    # D, H_q, H_kv, q_len, kv_len, batch-0 key count (None: all keys)
    (128, 32, 8, 4096, 4096, None),
    (64, 32, 8, 4096, 4096, None),
    (128, 32, 8, 4096, 6144, None),     # kv_len > q_len
    (128, 32, 8, 4096, 4096, 1000),     # 3096 rows of batch 0 see no key
    (64, 32, 8, 4096, 4608, 3333),
    (128, 32, 8, 5184, 5184, None),     # row tiles across heads, padding rows
    (128, 16, 8, 8192, 8192, None),     # GQA ratio 2
]


@pytest.mark.parametrize("case", CAUSAL_PAIRS, ids=lambda c: "D{}_Hq{}_Hkv{}_q{}_kv{}_{}".format(
    *c[:5], "full" if c[5] is None else f"k{c[5]}"))
def test_wide_causal_kernel_equals_256_row_kernel_bitwise(case):
    import kernelfoundry_amd as kf
    torch = _torch()
    D, H_q, H_kv, S, kv, k0 = case
    masked = k0 is not None
    n1 = kf.kernel_names(1, S, kv, H_q, H_kv, D, causal=True, masked=masked)
    n2 = kf.kernel_names(2, S, kv, H_q, H_kv, D, causal=True, masked=masked)
    print("case", case, n1, "|", n2, flush=True)
    assert n1 == f"kf_attn_prefill_kernel<{D}, true, 8, 1>", n1
    assert n2 == f"kf_attn_prefill_wide_kernel<{D}, true, 1, true>", n2
    _, (Q, K, V) = _inputs(2, H_q, H_kv, S, kv, D, 91)
    l1 = torch.tensor([k0], dtype=torch.int32, device="cuda") if masked else None
    l2 = torch.tensor([k0, kv - 7], dtype=torch.int32, device="cuda") if masked else None
    O1, M1, L1 = kf.attn_fwd(Q[:1].contiguous(), K[:1].contiguous(), V[:1].contiguous(), return_stats=True,
                             causal=True, kv_lens=l1)
    O2, M2, L2 = kf.attn_fwd(Q, K, V, return_stats=True, causal=True, kv_lens=l2)
    torch.cuda.synchronize()
    assert torch.equal(O1[0], O2[0]), f"O differs: max {(O1[0] - O2[0]).abs().max().item():.3g}"
    assert torch.equal(M1[0], M2[0]) and torch.equal(L1[0], L2[0]), "Mi / Li differ"
    if masked:
        empty = S - k0  # rows before this one see no key of batch 0
        assert torch.count_nonzero(O2[0, :, :empty]).item() == 0
        assert torch.isinf(M2[0, :, :empty]).all() and torch.count_nonzero(L2[0, :, :empty]).item() == 0


@pytest.mark.parametrize("D", [64, 128])
def test_wide_causal_kernel_matches_oracle(D):
    """Batch 1 of a B = 2 causal call (the wide causal kernel), heads 0 and
    the last, against the fp64 oracle on the same fp16 inputs."""
    import kernelfoundry_amd as kf
    torch = _torch()
    S, kv, H_q, H_kv = 4096, 4608, 32, 8
    name = kf.kernel_names(2, S, kv, H_q, H_kv, D, causal=True)
    print("case D", D, name, flush=True)
    assert name == f"kf_attn_prefill_wide_kernel<{D}, true, 1, true>", name
    (q16, k16, v16), (Q, K, V) = _inputs(2, H_q, H_kv, S, kv, D, 123 + D)
    O, Mi, Li = kf.attn_fwd(Q, K, V, return_stats=True, causal=True)
    torch.cuda.synchronize()
    O, Mi, Li = O.cpu().numpy(), Mi.cpu().numpy(), Li.cpu().numpy()
    for h in (0, H_q - 1):
        hk = h // (H_q // H_kv)
        Or, Mr, Lr = orc.sdpa(q16[1:2, h:h + 1], k16[1:2, hk:hk + 1], v16[1:2, hk:hk + 1], causal=True)
        ok, max_abs, rel = orc.within_tolerance(O[1:2, h:h + 1], Or)
        assert ok, f"head {h}: max_abs={max_abs:.3g} rel={rel:.3g}"
        assert np.abs(Mi[1, h] - Mr[0, 0]).max() <= 1e-4, "Mi"
        assert (np.abs(Li[1, h] - Lr[0, 0]) / np.abs(Lr[0, 0])).max() <= 1e-3, "Li"


def _causal_random_cases(n=12, seed=20261202):
    """Seeded shapes that the planner sends to the causal two-block kernel
    for the whole batch and to the 32-row kernel (one KV group) for each
    sequence alone: GQA ratios 1-8, 1-8 KV heads, D = 64 / 128, q_len a
    multiple of 64 from 1024 to 8192, keys from q_len / 2 + 2048 on, key
    counts in some."""
    import kernelfoundry_amd as kf
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        D = int(rng.choice([64, 128]))
        H_kv = int(rng.choice([1, 2, 4, 8]))
        H_q = H_kv * int(rng.choice([1, 2, 4, 8]))
        B = int(rng.integers(2, 9))
        q = 64 * int(rng.integers(16, 129))
        kv = int(rng.integers(q // 2 + 2048, q + 3000))
        lens = bool(rng.random() < 0.4)
        if kf.kernel_names(B, q, kv, H_q, H_kv, D, causal=True, masked=lens) != \
                f"kf_attn_prefill_wide_kernel<{D}, true, 1, true>":
            continue
        if kf.kernel_names(1, q, kv, H_q, H_kv, D, causal=True, masked=lens) != \
                f"kf_attn_prefill_kernel<{D}, true, 8, 1>":
            continue
        if B * H_q * q * D * 2 > 1e9:
            continue
        kl = [int(x) for x in rng.integers(0, kv + 1, size=B)] if lens else None
        out.append((B, H_q, H_kv, q, kv, D, kl, int(rng.integers(1 << 30))))
    return out


@pytest.mark.parametrize("case", _causal_random_cases(), ids=lambda c: "B{}_Hq{}_Hkv{}_q{}_kv{}_D{}_{}".format(
    *c[:6], "lens" if c[6] is not None else "full"))
def test_wide_causal_random_shapes_equal_256_row_kernel_bitwise(case):
    import kernelfoundry_amd as kf
    torch = _torch()
    B, H_q, H_kv, q, kv, D, kl, seed = case
    print("case", case[:7], flush=True)
    g = torch.Generator(device="cuda").manual_seed(seed)
    Q = torch.randn(B, H_q, q, D, generator=g, device="cuda").half()
    K = torch.randn(B, H_kv, kv, D, generator=g, device="cuda").half()
    V = torch.randn(B, H_kv, kv, D, generator=g, device="cuda").half()
    lens = None if kl is None else torch.tensor(kl, dtype=torch.int32, device="cuda")
    O, M, L = kf.attn_fwd(Q, K, V, return_stats=True, causal=True, kv_lens=lens)
    for b in range(B):
        O1, M1, L1 = kf.attn_fwd(Q[b:b + 1].contiguous(), K[b:b + 1].contiguous(), V[b:b + 1].contiguous(),
                                 return_stats=True, causal=True,
                                 kv_lens=None if lens is None else lens[b:b + 1].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(O[b], O1[0]), f"batch {b}: O differs by {(O[b] - O1[0]).abs().max().item():.3g}"
        assert torch.equal(M[b], M1[0]) and torch.equal(L[b], L1[0]), f"batch {b}: Mi / Li differ"
