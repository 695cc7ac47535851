"""Property test of the dispatch planner (kf_attn_plan, host code only) over
random shapes: every prefill plan's row tiles cover the query rows of a
head, every decode and split-prefill plan covers all keys of a head exactly
once with whole 32-key stages, stays within the split merge's one-pass capacity, gives the
streaming decode kernel at least one stage per wave in each split, and sizes
the split workspace for every partial."""
import pytest
from hypothesis import given, settings, strategies as st

import kernelfoundry_amd as kf

RATIOS = [1, 2, 4, 8, 16, 32]


@settings(max_examples=400, deadline=None)
@given(B=st.integers(1, 64), H_kv=st.sampled_from([1, 2, 4, 8]), ratio=st.sampled_from(RATIOS),
       q=st.integers(1, 300), kv=st.integers(1, 300000), D=st.sampled_from([16, 64, 128, 256]),
       cus=st.sampled_from([32, 80, 256, 304]))
def test_plan_invariants(B, H_kv, ratio, q, kv, D, cus):
    H_q = H_kv * ratio
    try:
        p = kf.plan(B, q, kv, H_q, H_kv, D, num_cus=cus)
    except kf.KfError as e:
        # Only shapes beyond 32-bit in-head indexing are refused.
        assert e.status == kf.KF_ERR_SIZE
        assert (ratio * q) * D > 2 ** 31 - 1 or kv * D > 2 ** 31 - 1 or B * H_q * q > 2 ** 31 - 1
        return
    R = ratio * q
    n_groups = B * H_kv
    assert p.rows_per_group == R
    if p.path == "prefill":
        assert R > 32
        waves = p.block_threads // 64
        assert waves in ((4, 8) if D == 256 else (2, 4, 8))
        # A workgroup holds 32 query rows per wave, or 32 per wave of one of
        # its two or four KV groups (each taking that share of the keys), or
        # (the wide kernel, 8 waves at D = 64 / 128) 64 per wave; row tiles
        # cover R.
        assert p.grid_blocks % n_groups == 0
        tiles = p.grid_blocks // n_groups
        wide = (-(-R // 512),) if (waves == 8 and D in (64, 128)) else ()
        assert tiles in (-(-R // (32 * waves)), -(-R // (16 * waves)), -(-R // (8 * waves))) + wide
        assert p.workspace_bytes == 0 and p.num_splits == 1
        return
    if p.path == "prefill_split":
        # The same workgroup layouts (D <= 128) with the keys split into
        # partitions of whole tiles, only where the unsplit grid leaves half
        # the CUs idle or more and the split grid fits one round; every key
        # in exactly one partition; each KV group's serial chain at least 6
        # tiles shorter; the partials sized.
        assert R > 32
        waves = p.block_threads // 64
        assert waves in ((4,) if D == 256 else (2, 4, 8))
        assert p.grid_blocks % (n_groups * p.num_splits) == 0
        tiles = p.grid_blocks // (n_groups * p.num_splits)
        assert tiles in (-(-R // (32 * waves)), -(-R // (16 * waves)), -(-R // (8 * waves)))
        assert 2 * n_groups * tiles <= cus and p.grid_blocks <= cus
        assert 1 < p.num_splits <= 256 and p.kv_per_split % 32 == 0
        # KV groups per workgroup (ks) consistent with the row tiles; the
        # partition holds whole tiles of every group.
        units = [32 * ks for ks in (1, 2, 4)
                 if tiles == -(-R // (32 * waves // ks)) and p.kv_per_split % (32 * ks) == 0]
        if D == 256:
            # Against the wide kernel's chain (two KV groups or one), a
            # 4-wave tile counting 1.4 wide tiles.
            assert any(-(-kv // w) - 1.4 * (p.kv_per_split // 32) >= 6 for w in (32, 64))
        else:
            assert any(-(-kv // u) - p.kv_per_split // u >= 6 for u in units)
        assert (p.num_splits - 1) * p.kv_per_split < kv <= p.num_splits * p.kv_per_split
        assert p.workspace_bytes >= n_groups * p.num_splits * R * (D + 2) * 4
        return
    assert R <= 32
    assert p.kv_per_split % 32 == 0
    assert (p.num_splits - 1) * p.kv_per_split < kv <= p.num_splits * p.kv_per_split
    assert p.num_splits <= 256
    if p.splits_per_block == 4:                       # short-split kernel
        assert p.kv_per_split in (32, 64)
        assert p.grid_blocks * 4 >= n_groups * p.num_splits > (p.grid_blocks - 1) * 4
    else:                                             # streaming kernel
        waves = 8 if D <= 128 else 4
        assert p.block_threads == 64 * waves
        assert p.grid_blocks == n_groups * p.num_splits
        assert p.num_splits == 1 or p.kv_per_split >= 32 * waves
    if p.num_splits == 1:
        assert p.path == "decode" and p.workspace_bytes == 0
    else:
        assert p.path == "decode_split"
        assert p.workspace_bytes >= n_groups * p.num_splits * R * (D + 2) * 4
