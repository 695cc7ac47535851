"""GPU parity of the prefill kernel in 8-wave (256-row) workgroups at D = 128.

The planner uses 8-wave workgroups when that grid fills the chip; the other
prefill tests mostly run small grids (2- and 4-wave workgroups).  Every shape
here is chosen so that the 8-wave kernel runs (asserted through kf.plan: 512
threads per workgroup), and so that its edge cases are hit: a partial last
LDS stage (kv_len % 64 != 0), a ragged last tile (kv_len % 32 != 0), padding
query rows (rows per KV head % 256 != 0), one to a few tiles (stages the
prologue issues, buffers never filled), more tiles than one unrolled loop
body, causal masking with per-sequence key counts and an empty sequence.  O, Mi and Li are
compared with oracle/attn_oracle.py's fp64 ``sdpa`` on the same fp16 inputs
to the north-star bar (max |got - ref| <= 2e-3, ||got - ref|| / ||ref|| <=
1e-2; Mi to 1e-4, Li to 1e-3 relative); rows without keys must be exactly
O = 0, Mi = -inf, Li = 0.
"""
import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    return torch


def _announce(**kw):
    print("case", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _run(q16, k16, v16, causal=False, kv_lens=None):
    import kernelfoundry_amd as kf
    torch = _torch()
    Q, K, V = (torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (q16, k16, v16))
    lens = None if kv_lens is None else torch.tensor(kv_lens, dtype=torch.int32, device="cuda")
    O, Mi, Li = kf.attn_fwd(Q, K, V, return_stats=True, causal=causal, kv_lens=lens)
    torch.cuda.synchronize()
    return O.cpu().numpy(), Mi.cpu().numpy(), Li.cpu().numpy()


def _check(got, ref, label):
    O, Mi, Li = got
    Or, Mr, Lr = ref
    assert np.isfinite(O).all(), f"{label}: non-finite O"
    ok, max_abs, rel = orc.within_tolerance(O, Or)
    assert ok, f"{label}: max_abs={max_abs:.3g} rel={rel:.3g}"
    empty = np.isneginf(Mr)
    assert np.array_equal(np.isneginf(Mi), empty), f"{label}: Mi = -inf on the wrong rows"
    assert (O[empty] == 0).all() and (Li[empty] == 0).all(), f"{label}: empty rows not zero"
    full = ~empty
    assert np.abs(Mi[full] - Mr[full]).max() <= 1e-4, f"{label}: Mi"
    rel_l = np.abs(Li[full] - Lr[full]).max() / np.abs(Lr[full]).max()
    assert rel_l <= 1e-3, f"{label}: Li rel err {rel_l:.3g}"


CASES = [
    # B, H_q, H_kv, q_len, kv_len, causal, kv_lens        what it hits
    (2, 32, 8, 1000, 1000, False, None),                  # partial stage, ragged tile, padding rows
    (1, 32, 8, 2048, 1, False, None),                     # one tile, one key
    (1, 32, 8, 2048, 40, False, None),                    # two tiles in one partial stage
    (1, 32, 8, 2048, 96, False, None),                    # two stages, three tiles
    (1, 32, 8, 2048, 200, False, None),                   # four stages
    (1, 32, 8, 2048, 520, False, None),                   # 17 tiles: past one unrolled body
    (2, 32, 8, 1024, 1100, True, [1100, 700]),            # causal + key counts, bottom-right
    (2, 32, 8, 1024, 600, False, [600, 0]),               # an empty sequence
    (2, 32, 8, 1024, 1024, True, [1024, 37]),             # causal, few keys: most rows masked
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_q{}_kv{}_c{}_{}".format(
    c[0], c[3], c[4], int(c[5]), "lens" if c[6] else "full"))
def test_prefill_8wave_parity(case):
    import kernelfoundry_amd as kf
    B, H_q, H_kv, q_len, kv_len, causal, kv_lens = case
    D = 128
    pl = kf.plan(B, q_len, kv_len, H_q, H_kv, D)
    assert pl.path == "prefill" and pl.block_threads == 512, pl  # 8-wave workgroups
    _announce(test="prefill_8wave", B=B, q_len=q_len, kv_len=kv_len, causal=causal, kv_lens=kv_lens,
              grid=pl.grid_blocks)
    q16, k16, v16 = orc.normal_fp16_inputs(B, H_q, H_kv, q_len, kv_len, D, 31000 + kv_len)
    ref = orc.sdpa(q16, k16, v16, causal=causal, kv_lens=kv_lens)
    got = _run(q16, k16, v16, causal, kv_lens)
    _check(got, ref, f"case {case}")


def test_prefill_8wave_masked_matches_unmasked_bitwise():
    """Per-sequence key counts equal to kv_len run the masked instantiation,
    whose arithmetic on unmasked rows is the unmasked one: bitwise equal."""
    import kernelfoundry_amd as kf
    torch = _torch()
    B, H_q, H_kv, S, D = 2, 32, 8, 1000, 128
    assert kf.plan(B, S, S, H_q, H_kv, D).block_threads == 512
    _announce(test="prefill_8wave_masked_vs_unmasked", B=B, S=S)
    q16, k16, v16 = orc.normal_fp16_inputs(B, H_q, H_kv, S, S, D, 82)
    Q, K, V = (torch.from_numpy(x).cuda() for x in (q16, k16, v16))
    O0 = kf.attn_fwd(Q, K, V)
    O1 = kf.attn_fwd(Q, K, V, kv_lens=torch.full((B,), S, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    assert torch.equal(O0, O1)


# ---------------------------------------------------------------------------
# KV groups: grids too small for 8-wave workgroups split each row's keys
# between two groups of waves (8 waves x 128 rows, or 4 x 64) or four (8 waves
# x 64 rows, at least 512 keys), merged in LDS.
# ---------------------------------------------------------------------------
KV_GROUP_CASES = [
    # B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens, threads, rows   what it hits
    (1, 32, 8, 1024, 1024, 128, False, None, 512, 128),        # sweep S=1024: 8 waves x 2 groups
    (1, 32, 8, 512, 512, 128, False, None, 512, 64),           # C1 shape: 8 waves x 4 groups
    (1, 32, 8, 512, 520, 128, False, None, 512, 64),           # 4 groups, ragged last group
    (1, 32, 8, 512, 600, 128, True, None, 512, 64),            # 4 groups, causal, q_len < kv_len
    (1, 32, 8, 512, 512, 128, False, [100], 512, 64),          # 4 groups of one tile each
    (1, 32, 8, 512, 512, 128, True, [20], 512, 64),            # groups 1..3 see no key
    (1, 32, 8, 512, 130, 128, False, None, 256, 64),           # 4 waves x 2 groups: 3 and 2 tiles
    (1, 32, 8, 512, 128, 128, False, None, 256, 64),           # exactly 4 tiles
    (2, 32, 8, 256, 300, 128, True, [300, 129], 256, 64),      # causal + key counts
    (2, 32, 8, 256, 256, 128, True, [256, 40], 256, 64),       # second group sees no key
    (1, 32, 1, 1024, 1024, 64, False, None, 512, 128),         # MQA D=64, 8 waves x 2 groups
    (1, 32, 1, 512, 512, 64, False, None, 512, 64),            # MQA D=64, 8 waves x 4 groups
    (1, 32, 1, 512, 700, 64, True, None, 512, 64),             # MQA D=64 causal, 4 groups
]


@pytest.mark.parametrize("case", KV_GROUP_CASES, ids=lambda c: "B{}_Hkv{}_q{}_kv{}_D{}_c{}_{}".format(
    c[0], c[2], c[3], c[4], c[5], int(c[6]), "lens" if c[7] else "full"))
def test_kv_groups_parity(case):
    import kernelfoundry_amd as kf
    B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens, threads, rows = case
    pl = kf.plan(B, q_len, kv_len, H_q, H_kv, D)
    R = H_q // H_kv * q_len
    assert pl.path == "prefill" and pl.block_threads == threads, pl
    assert pl.grid_blocks == B * H_kv * -(-R // rows), pl       # KV groups per workgroup
    _announce(test="kv_groups", B=B, H_kv=H_kv, q_len=q_len, kv_len=kv_len, D=D, causal=causal,
              kv_lens=kv_lens, grid=pl.grid_blocks)
    q16, k16, v16 = orc.normal_fp16_inputs(B, H_q, H_kv, q_len, kv_len, D, 47000 + kv_len + D)
    ref = orc.sdpa(q16, k16, v16, causal=causal, kv_lens=kv_lens)
    got = _run(q16, k16, v16, causal, kv_lens)
    _check(got, ref, f"case {case}")
