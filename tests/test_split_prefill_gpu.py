"""GPU parity of the split prefill (kf_attn_fwd_ex on the prefill_split path).

A prefill whose grid leaves half the CUs idle or more -- few query rows per
KV head against many keys, as in chunked prefill or speculative
verification -- splits each row tile's keys into KV partitions:
kf_attn_prefill_kernel writes one fp32 partial (O unnormalised, row max,
row sum) per partition and kf_attn_split_merge_kernel combines them, as on
the split decode path.  Each case asserts that the planner takes that path,
runs the HIP kernels through the C ABI on seeded fp16 inputs and compares
them with the fp64 oracle (oracle/attn_oracle.py ``sdpa``) to the
north-star bar (tests/_parity.py: max |got - ref| <= 2e-3,
||got - ref|| / ||ref|| <= 1e-2, Mi to 1e-4, Li to 1e-3 relative, rows
without keys exactly O = 0, Mi = -inf, Li = 0).

Covered: every head dimension (16 and 256 -- the 4-wave kernel with the
partition code compiled in -- one KV group per workgroup, the epilogue
writes the partial; 64 / 128: four KV groups, the group merge writes it),
a last partition shorter than one tile, causal masking (bottom-right aligned, partitions that some rows of a wave do not
reach), per-sequence key counts (sequences without keys, partitions past a
sequence's keys), GQA and MQA, B > 1, up to 32 partitions per row tile.
"""
import numpy as np
import pytest

from tests._parity import run_and_check

pytestmark = pytest.mark.gpu

CASES = [
    # B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens
    (1, 32, 8, 16, 8192, 128, False, None),          # 32 partitions of 256 keys
    (1, 32, 8, 64, 4000, 128, False, None),          # last partition 416 keys: partial tile
    (1, 32, 8, 64, 1024, 64, False, None),           # D = 64, 4 partitions
    (2, 16, 4, 48, 3000, 128, True, None),           # causal, q_len not a multiple of 32
    (2, 32, 8, 64, 5000, 128, False, [4321, 77]),    # key counts: partitions past 77 keys
    (2, 32, 8, 64, 3000, 64, True, [3000, 0]),       # causal + an empty sequence
    (1, 32, 1, 8, 8192, 128, False, None),           # MQA, 32 partitions
    (1, 32, 8, 32, 3333, 16, True, None),            # D = 16 (one KV group), causal
    (2, 32, 8, 40, 4096, 16, False, [4096, 100]),    # D = 16, key counts
    (3, 8, 2, 100, 2500, 64, True, [2500, 1800, 5]), # causal + key counts
    (1, 4, 1, 200, 6000, 128, False, None),          # 16 partitions, rows spanning heads
    (1, 32, 8, 16, 8192, 256, False, None),          # D = 256 (4-wave kernel), 32 partitions
    (2, 16, 4, 100, 3000, 256, True, None),          # D = 256, causal, partial last tile
    (2, 32, 8, 64, 4000, 256, False, [3999, 1]),     # D = 256, key counts, a one-key sequence
    (1, 16, 4, 32, 2048, 256, True, [0]),            # D = 256, 64-key partitions, no keys at all
]


@pytest.mark.parametrize("case", CASES,
                         ids=lambda c: "B{}_Hq{}_Hkv{}_q{}_kv{}_D{}".format(*c[:6]) +
                         ("_causal" if c[6] else "") + ("_lens" if c[7] else ""))
def test_split_prefill_matches_oracle(case):
    import kernelfoundry_amd as kf
    B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens = case
    p = kf.plan(B, q_len, kv_len, H_q, H_kv, D)
    assert p.path == "prefill_split" and p.num_splits > 1, p
    assert kf.kernel_names(B, q_len, kv_len, H_q, H_kv, D, causal=causal).endswith(
        "kf_attn_split_merge_kernel<%d, %d, %d>" % (D, *_merge_shape(kf, B, q_len, kv_len, H_q, H_kv, D)))
    run_and_check(B, H_q, H_kv, q_len, kv_len, D, causal, kv_lens, seed=900 + D + q_len)


def _merge_shape(kf, B, q_len, kv_len, H_q, H_kv, D):
    name = kf.kernel_names(B, q_len, kv_len, H_q, H_kv, D)
    tail = name.split("kf_attn_split_merge_kernel<")[1].rstrip(">")
    _, per, cw = (int(x) for x in tail.split(","))
    return per, cw


def test_split_prefill_masked_kernel_agrees_with_unmasked():
    """Key counts equal to kv_len run the masked instantiation over the same
    partitions as the unmasked call, with the same arithmetic on every
    visible key: bit-identical O, Mi and Li (the partial's rebase factor is
    one explicit fused multiply-add in both)."""
    import torch

    import kernelfoundry_amd as kf
    from oracle import attn_oracle as orc
    B, H_q, H_kv, q_len, kv_len, D = 2, 32, 8, 64, 3000, 128
    assert kf.plan(B, q_len, kv_len, H_q, H_kv, D).path == "prefill_split"
    print("case split masked vs unmasked", (B, H_q, H_kv, q_len, kv_len, D), flush=True)
    q16, k16, v16 = orc.normal_fp16_inputs(B, H_q, H_kv, q_len, kv_len, D, 31)
    Q, K, V = (torch.from_numpy(x).cuda() for x in (q16, k16, v16))
    O0, M0, L0 = kf.attn_fwd(Q, K, V, return_stats=True)
    lens = torch.full((B,), kv_len, dtype=torch.int32, device="cuda")
    O1, M1, L1 = kf.attn_fwd(Q, K, V, return_stats=True, kv_lens=lens)
    torch.cuda.synchronize()
    assert torch.equal(M0, M1) and torch.equal(O0, O1) and torch.equal(L0, L1)


def test_split_prefill_result_does_not_depend_on_the_workspace():
    """Every partial the merge reads is written by this call: a workspace
    filled with NaN and one filled with zeros give the same O bit for bit."""
    import torch

    import kernelfoundry_amd as kf
    from oracle import attn_oracle as orc
    B, H_q, H_kv, q_len, kv_len, D = 2, 32, 8, 40, 4096, 16
    assert kf.plan(B, q_len, kv_len, H_q, H_kv, D).path == "prefill_split"
    print("case split workspace contents", (B, H_q, H_kv, q_len, kv_len, D), flush=True)
    q16, k16, v16 = orc.normal_fp16_inputs(B, H_q, H_kv, q_len, kv_len, D, 32)
    Q, K, V = (torch.from_numpy(x).cuda() for x in (q16, k16, v16))
    lens = torch.tensor([4096, 100], dtype=torch.int32, device="cuda")
    need = kf.workspace_bytes(B, q_len, kv_len, H_q, H_kv, D)
    outs = []
    for fill in (float("nan"), 0.0):
        ws = torch.full((need // 4,), fill, dtype=torch.float32, device="cuda")
        outs.append(kf.attn_fwd(Q, K, V, kv_lens=lens, causal=True, workspace=ws))
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1])
    assert np.array_equal(outs[0].cpu().numpy(), outs[1].cpu().numpy())
