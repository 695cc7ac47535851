"""The C ABI of libkf_attn.so, exercised without a GPU.

Checks that the library loads, exports every function include/kf/attn.h
declares, carries gfx950 code, plans the documented dispatch, and rejects
every invalid argument with its status code before any HIP call (the fake
device pointers below are never dereferenced).
"""
import ctypes
import os
import re
import subprocess

import pytest

import kernelfoundry_amd as kf

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

FAKE = 0x10000          # 16-byte aligned, never dereferenced
FAKE_WS = 0x20000       # 256-byte aligned


@pytest.fixture(scope="module")
def lib():
    return kf.load_library()


def test_library_exports_every_declared_symbol(lib):
    names = kf.exported_symbols()
    assert set(names) >= {"kf_attn_fwd", "kf_attn_plan", "kf_attn_workspace_bytes",
                          "kf_launch_flash_attn", "kf_status_string", "kf_last_hip_error",
                          "kf_version"}
    for n in names:
        assert hasattr(lib, n), f"{n} declared in kf/attn.h but not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", kf.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\s[TW]\s+(kf_\w+)$", out, re.M))
    assert exported == set(names), f"undeclared exports: {exported - set(names)}"


def test_library_carries_gfx950_code():
    with open(kf.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"gfx950" in blob
    for kern in (b"kf_attn_prefill_kernel", b"kf_attn_decode_kernel"):
        assert kern in blob


def test_no_kernel_uses_scratch(tmp_path):
    """Every kernel of the gfx950 code object keeps its state in registers and
    LDS: no private (scratch) segment, no spilled VGPRs (but the AGPR spills
    of one instantiation, below).  Read from the
    library's own code object metadata (llvm-objcopy + clang-offload-bundler
    + llvm-readelf from the ROCm toolchain)."""
    tools = "/opt/rocm/llvm/bin"
    objcopy, bundler, readelf = (os.path.join(tools, t) for t in
                                 ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf"))
    if not all(os.path.exists(t) for t in (objcopy, bundler, readelf)):
        pytest.skip("ROCm LLVM tools not found")
    fat, co = tmp_path / "fatbin", tmp_path / "gfx950.co"
    subprocess.run([objcopy, "--dump-section", f".hip_fatbin={fat}", kf.LIB_PATH], check=True)
    subprocess.run([bundler, "--unbundle", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--input={fat}", f"--output={co}"], check=True)
    notes = subprocess.run([readelf, "--notes", str(co)], capture_output=True, text=True,
                           check=True).stdout
    kernels = {}
    for block in re.split(r"\n\s+- \.agpr_count:", notes)[1:]:
        name = re.search(r"\.name:\s+(\S+)", block).group(1)
        scratch = int(re.search(r"\.private_segment_fixed_size:\s+(\d+)", block).group(1))
        spills = int(re.search(r"\.vgpr_spill_count:\s+(\d+)", block).group(1))
        kernels[name] = (scratch, spills)
    assert any("kf_attn_prefill_kernel" in n for n in kernels)
    assert any("kf_attn_decode_kernel" in n for n in kernels)
    # One exception: the D = 256 split prefill (kf_attn_prefill_parts_kernel,
    # the 4-wave kernel with its KV-partition code) moves two values from
    # VGPRs to AGPRs -- spills without a scratch segment, so no memory
    # traffic (the unsplit 4-wave kernel has none).
    split256 = re.compile(r"kf_attn_prefill_parts_kernelILi256E")
    bad = {n: v for n, v in kernels.items()
           if v != (0, 0) and not (split256.search(n) and v[0] == 0 and v[1] <= 4)}
    assert not bad, f"kernels with scratch / spills: {bad}"
    assert any(split256.search(n) for n in kernels)


def test_version(lib):
    assert b"gfx950" in lib.kf_version()


def _fwd(B=1, q=4, kv=64, H_q=8, H_kv=2, D=128, Q=FAKE, K=FAKE, V=FAKE, O=FAKE, ws=None,
         ws_bytes=0):
    return kf.attn_fwd_ptr(Q, K, V, O, 0, 0, B, q, kv, H_q, H_kv, D, ws or 0, ws_bytes, 0)


@pytest.mark.parametrize("D", [0, -1, 8, 32, 96, 100, 512])
def test_bad_head_dim(D):
    assert _fwd(D=D) == kf.KF_ERR_HEAD_DIM
    assert kf.workspace_bytes(1, 1, 64, 8, 2, D) == 0


@pytest.mark.parametrize("H_q,H_kv", [(8, 3), (5, 2), (1, 2)])
def test_bad_gqa_ratio(H_q, H_kv):
    assert _fwd(H_q=H_q, H_kv=H_kv) == kf.KF_ERR_GQA


@pytest.mark.parametrize("field", ["B", "q", "kv", "H_q", "H_kv"])
@pytest.mark.parametrize("value", [0, -3])
def test_bad_sizes(field, value):
    assert _fwd(**{field: value}) == kf.KF_ERR_SIZE


def test_size_overflow_of_32bit_in_head_indexing():
    assert _fwd(kv=(1 << 31) // 128 + 1, H_q=8, H_kv=8) == kf.KF_ERR_SIZE
    assert _fwd(q=(1 << 31) // (128 * 4) + 1, H_q=8, H_kv=2) == kf.KF_ERR_SIZE


@pytest.mark.parametrize("which", ["Q", "K", "V", "O"])
def test_null_pointers(which):
    assert _fwd(**{which: 0}) == kf.KF_ERR_NULL


@pytest.mark.parametrize("which", ["Q", "K", "V", "O"])
def test_misaligned_pointers(which):
    assert _fwd(**{which: FAKE + 2}) == kf.KF_ERR_ALIGN


def test_workspace_required_for_split_decode():
    pl = kf.plan(1, 1, 4096, 32, 8, 128)
    assert pl.path == "decode_split" and pl.workspace_bytes > 0
    args = dict(B=1, q=1, kv=4096, H_q=32, H_kv=8, D=128)
    assert _fwd(**args) == kf.KF_ERR_WORKSPACE
    assert _fwd(ws=FAKE_WS, ws_bytes=pl.workspace_bytes - 1, **args) == kf.KF_ERR_WORKSPACE
    assert _fwd(ws=FAKE_WS + 16, ws_bytes=pl.workspace_bytes, **args) == kf.KF_ERR_ALIGN


def _fwd_ex(kv_lens=0, flags=0, **kw):
    a = dict(B=1, q=4, kv=64, H_q=8, H_kv=2, D=128)
    a.update(kw)
    return kf.attn_fwd_ex_ptr(FAKE, FAKE, FAKE, FAKE, 0, 0, a["B"], a["q"], a["kv"], a["H_q"],
                              a["H_kv"], a["D"], kv_lens, flags)


def test_fwd_ex_validation():
    assert _fwd_ex(flags=16) == kf.KF_ERR_FLAGS
    assert _fwd_ex(flags=-1) == kf.KF_ERR_FLAGS
    assert _fwd_ex(flags=kf.KF_ATTN_OUT_F16 | kf.KF_ATTN_OUT_BF16) == kf.KF_ERR_FLAGS
    assert _fwd_ex(kv_lens=FAKE + 2) == kf.KF_ERR_ALIGN        # int array: 4-byte aligned
    assert _fwd_ex(D=96, flags=kf.KF_ATTN_CAUSAL) == kf.KF_ERR_HEAD_DIM
    assert _fwd_ex(H_kv=3, flags=kf.KF_ATTN_CAUSAL) == kf.KF_ERR_GQA
    assert _fwd_ex(q=0, kv_lens=FAKE) == kf.KF_ERR_SIZE
    assert kf.attn_fwd_ex_ptr(0, FAKE, FAKE, FAKE, 0, 0, 1, 4, 64, 8, 2, 128, 0,
                              kf.KF_ATTN_CAUSAL) == kf.KF_ERR_NULL
    # Split decode still needs its workspace with masking.
    assert _fwd_ex(q=1, kv=4096, H_q=32, H_kv=8, flags=kf.KF_ATTN_CAUSAL) == kf.KF_ERR_WORKSPACE


def test_reference_launcher_rejects_like_the_reference():
    # tests/test_flash_attn.cu:96-100: unsupported D -> cudaErrorInvalidValue.
    assert kf.launch_flash_attn(FAKE, FAKE, FAKE, FAKE, 1, 64, 8, 2, 96) == kf.HIP_ERROR_INVALID_VALUE
    assert kf.launch_flash_attn(FAKE, FAKE, FAKE, FAKE, 1, 64, 8, 3, 128) == kf.HIP_ERROR_INVALID_VALUE
    assert kf.launch_flash_attn(0, FAKE, FAKE, FAKE, 1, 64, 8, 2, 128) == kf.HIP_ERROR_INVALID_VALUE


def test_status_strings_distinct(lib):
    texts = [kf.status_string(s) for s in range(9)]
    assert len(set(texts)) == 9
    assert kf.status_string(99) == "unknown status"


def test_plan_null_out(lib):
    assert lib.kf_attn_plan(1, 1, 1, 1, 1, 128, None) == kf.KF_ERR_NULL


# ---------------------------------------------------------------------------
# Dispatch plans for the BASELINE.json configs and the split geometry.
# ---------------------------------------------------------------------------
def test_plans_for_baseline_configs():
    p = kf.plan(1, 4096, 4096, 32, 8, 128)           # C3 prefill: wide kernel,
    assert p.path == "prefill" and p.rows_per_group == 4 * 4096
    assert p.block_threads == 512                    # 8 waves x 64 query rows
    assert p.grid_blocks == 8 * (4 * 4096 // 512) == 256
    assert kf.kernel_names(1, 4096, 4096, 32, 8, 128) == "kf_attn_prefill_wide_kernel<128, false, 1, false>"
    # masked: the 256-row kernel (8 waves x 32 rows), 512 workgroups
    assert kf.kernel_names(1, 4096, 4096, 32, 8, 128, causal=True) == "kf_attn_prefill_kernel<128, true, 8, 1>"
    p = kf.plan(1, 2048, 2048, 32, 8, 128)           # S = 2048: 128 wide workgroups would idle CUs
    assert p.grid_blocks == 256
    assert kf.kernel_names(1, 2048, 2048, 32, 8, 128) == "kf_attn_prefill_kernel<128, false, 8, 1>"
    p = kf.plan(1, 512, 512, 32, 8, 128)             # C1: 64 8-wave blocks would idle CUs
    assert p.path == "prefill" and p.block_threads == 512  # 2 row waves x 4 KV groups
    assert p.grid_blocks == 8 * (4 * 512 // 64) == 256
    assert kf.kernel_names(1, 512, 512, 32, 8, 128) == "kf_attn_prefill_kernel<128, false, 8, 4>"
    assert p.workspace_bytes == 0
    assert p.splits_per_block == 0
    p = kf.plan(1, 1, 4096, 32, 8, 128)              # C2 decode: 1024 one-wave splits
    assert p.path == "decode_split" and p.rows_per_group == 4
    assert p.splits_per_block == 4 and p.kv_per_split == 32 and p.num_splits == 128
    assert p.grid_blocks == 8 * 128 // 4 and p.block_threads == 256
    p = kf.plan(1, 2048, 2048, 32, 1, 64)            # C4a MQA prefill
    assert p.path == "prefill" and p.rows_per_group == 32 * 2048
    p = kf.plan(1, 1, 2048, 32, 1, 64)               # C4b MQA decode
    assert p.path == "decode_split" and p.rows_per_group == 32
    assert p.splits_per_block == 4 and p.num_splits == 64 and p.grid_blocks == 16
    p = kf.plan(32, 1, 8192, 32, 8, 128)             # C5 batched decode: streaming kernel,
    assert p.path == "decode" and p.grid_blocks == 256  # one 8-wave workgroup per KV head
    assert p.splits_per_block == 1 and p.num_splits == 1 and p.block_threads == 512
    assert p.workspace_bytes == 0                        # and no split merge


@pytest.mark.parametrize("B,q,kv,H_q,H_kv,D", [
    (1, 1, 1, 4, 1, 128), (1, 1, 31, 8, 8, 64), (1, 1, 129, 8, 8, 64), (2, 3, 1000, 8, 2, 16),
    (1, 1, 100000, 32, 8, 128), (64, 1, 300, 32, 8, 256), (1, 8, 4000, 4, 1, 128),
])
def test_decode_split_geometry_covers_kv(B, q, kv, H_q, H_kv, D):
    p = kf.plan(B, q, kv, H_q, H_kv, D)
    assert p.rows_per_group == (H_q // H_kv) * q <= 32
    assert p.kv_per_split % 32 == 0
    assert (p.num_splits - 1) * p.kv_per_split < kv <= p.num_splits * p.kv_per_split
    splits = B * H_kv * p.num_splits
    if p.splits_per_block == 4:
        # Short-split kernel: one wave per split of 32 or 64 keys (64 only for
        # D <= 128), 4 per workgroup, at most 4 waves per CU.
        assert p.kv_per_split in ((32, 64) if D <= 128 else (32,))
        assert p.grid_blocks == -(-splits // 4) and p.block_threads == 256 and splits <= 4 * 256
    else:
        # Streaming kernel: 8 waves (4 at D = 256), at least one 32-key stage
        # per wave in every split.
        waves = 8 if D <= 128 else 4
        assert p.splits_per_block == 1 and p.grid_blocks == splits
        assert p.block_threads == 64 * waves
        assert p.kv_per_split >= 32 * waves or p.num_splits == 1
    if p.num_splits == 1:
        assert p.path == "decode" and p.workspace_bytes == 0
    else:
        parts = B * H_q * q * p.num_splits
        assert p.workspace_bytes >= parts * (D + 2) * 4
        # The split merge reads every partial in one pass.
        assert p.num_splits <= 256


@pytest.mark.parametrize("B,H_kv,kv,D,splits,per_block", [
    (1, 8, 131072, 128, 32, 1), (1, 1, 262144, 128, 249, 1), (1, 1, 65536, 64, 228, 1),
    (1, 1, 1 << 20, 16, 251, 1), (1, 4, 40000, 256, 125, 1), (1, 8, 8192, 128, 128, 4),
    (1, 8, 4096, 128, 128, 4), (1, 8, 16384, 128, 32, 1), (2, 8, 16384, 128, 16, 1),
    (2, 8, 8192, 128, 16, 1), (8, 8, 1024, 128, 16, 4),
    (12, 8, 4096, 128, 8, 1), (32, 8, 8192, 128, 1, 1),
])
def test_decode_split_counts(B, H_kv, kv, D, splits, per_block):
    """Streaming decode (one 8-wave workgroup per CU at D <= 128): the fewest
    splits whose busiest CU streams within 2 % of an even share of the heads
    (96 heads: 8 splits = 3 full rounds of 256 workgroups), at most the 256
    partials the split merge reads in one pass, the key counts then rounded
    to whole 32-key stages; D = 256 (4 waves) aims at two workgroups per CU.
    Short-split decode: 64-key splits while they give 4 waves per CU, else
    32-key ones, up to 4 waves per CU and 256 splits."""
    p = kf.plan(B, 1, kv, 32, H_kv, D)
    assert p.path == ("decode_split" if splits > 1 else "decode") and p.num_splits == splits
    assert p.splits_per_block == per_block
    assert p.num_splits * p.kv_per_split >= kv


@pytest.mark.parametrize("S,H_kv,D,waves,groups", [
    (4096, 8, 128, 8, 1), (2048, 8, 128, 8, 1), (1024, 8, 128, 8, 2), (512, 8, 128, 8, 4),
    (256, 8, 128, 4, 2), (100, 8, 128, 2, 1), (2048, 1, 64, 8, 1), (512, 1, 64, 8, 4), (1024, 1, 64, 8, 2),
    (130, 2, 256, 4, 1), (4096, 8, 256, 4, 1), (512, 8, 256, 4, 1), (2048, 4, 256, 4, 1),
])
def test_prefill_waves_per_workgroup(S, H_kv, D, waves, groups):
    """Waves and KV groups per workgroup (32 query rows per wave of a KV
    group): 8 waves x 256 rows (4 x 128 at D = 256) when that grid gives every
    CU a workgroup.  Otherwise D = 64 / 128 split each row's keys between KV
    groups of waves if there are at least 128 keys: two (8 waves x 128 rows),
    then four (8 waves x 64 rows) if every group keeps 128 keys, else two of
    4 waves x 64 rows; the remaining cases halve the waves (down to 2, or 4 at
    D = 256)."""
    p = kf.plan(1, S, S, 32, H_kv, D)
    wide = kf.kernel_names(1, S, S, 32, H_kv, D).startswith("kf_attn_prefill_wide_kernel")
    # A grid that leaves CUs idle also splits the keys into partitions
    # (test_split_prefill_plans); the workgroup layout is the same.
    assert p.path in ("prefill", "prefill_split") and p.block_threads == (512 if wide else 64 * waves)
    # Masked calls run this kernel at D = 64 / 128; unmasked ones, and masked
    # ones at D = 256, may run a wide kernel instead (test_wide_prefill_selection).
    masked_name = kf.kernel_names(1, S, S, 32, H_kv, D, causal=True)
    rows = 32 * waves // groups
    R = 32 // H_kv * S
    # D = 256: 256-row tiles when they take fewer rounds (at 0.7 of the time
    # per row), else, from 256 keys on, two KV groups on the 128-row tiles.
    ks = 0
    if D == 256:
        n128, n256 = H_kv * -(-R // 128), H_kv * -(-R // 256)
        ks = 1 if -(-n256 // 256) * 256 * 0.7 < -(-n128 // 256) * 128 else 2 if S >= 256 else 0
        assert wide == (ks > 0)
    if wide and D == 256:
        assert masked_name == f"kf_attn_prefill_wide_kernel<256, true, {ks}, false>"
    else:
        assert masked_name.split(" + ")[0] == f"kf_attn_prefill_kernel<{D}, true, {waves}, {groups}>"
    if wide:
        assert p.grid_blocks == H_kv * -(-R // (512 if D != 256 else 256 if ks == 1 else 128))
    else:
        assert kf.kernel_names(1, S, S, 32, H_kv, D).split(" + ")[0] == \
            f"kf_attn_prefill_kernel<{D}, false, {waves}, {groups}>"
        assert p.grid_blocks == H_kv * -(-R // rows) * p.num_splits
    full = H_kv * -(-R // (256 if D <= 128 else 128)) >= 256
    if full:
        assert rows == (256 if D <= 128 else 128) and groups == 1
    elif D <= 128 and S >= 128:
        assert groups in (2, 4) and waves >= 4
        assert rows == 64 or H_kv * -(-R // 128) >= 256
        assert groups < 4 or S >= 4 * 128
    else:
        assert groups == 1


@pytest.mark.parametrize("B,S,H_q,H_kv,D,cus", [
    (1, 4096, 32, 8, 128, 256), (1, 2048, 32, 8, 128, 256), (1, 8192, 32, 8, 128, 256),
    (1, 4096, 32, 8, 64, 256), (1, 2048, 32, 1, 64, 256), (32, 100, 32, 8, 128, 256),
    (32, 130, 32, 8, 128, 256), (4, 1024, 64, 64, 128, 256), (1, 4096, 32, 8, 128, 80),
    (1, 4096, 32, 8, 128, 32), (1, 4096, 32, 8, 256, 256), (1, 4096, 32, 8, 16, 256),
    (3, 3000, 32, 8, 128, 304),
])
def test_wide_prefill_selection(B, S, H_q, H_kv, D, cus):
    """Unmasked prefill at D = 64 / 128 runs the wide kernel (8 waves x 64
    rows = 512 rows per workgroup) when the 256-row kernel would run 8-wave
    workgroups without KV groups and the wide grid's rounds of one workgroup
    per CU take less time, a wide row costing 0.94 of a 256-row-kernel row:
    rounds(wide) * 512 * 0.94 < rounds(256-row) * 256.  D = 256: 8 waves x
    32 rows against the 4-wave kernel's 128 rows, a row costing 0.7."""
    p = kf.plan(B, S, S, H_q, H_kv, D, num_cus=cus)
    R = H_q // H_kv * S
    n_groups = B * H_kv
    nrows, wrows, cost = (128, 256, 0.7) if D == 256 else (256, 512, 0.94)
    narrow = n_groups * -(-R // nrows)
    wide = n_groups * -(-R // wrows)
    rounds = lambda w: -(-w // cus)
    expect = (D in (64, 128, 256) and narrow >= cus and
              rounds(wide) * wrows * cost < rounds(narrow) * nrows)
    if expect:
        assert p.grid_blocks == wide and p.block_threads == 512
    elif D in (64, 128, 256) and narrow >= cus:
        assert p.grid_blocks == narrow


@pytest.mark.parametrize("cus", [32, 80, 256])
def test_plans_scale_with_the_device_cu_count(cus):
    """kf_attn_plan_for_cus sizes the dispatch for `cus` compute units: the
    prefill splits rows between KV groups, and the decode uses short
    one-wave splits, only while the plain grid would leave CUs idle; a
    decode that fills the device streams with the fewest splits whose
    busiest CU is within 2 % of an even share."""
    # C1 prefill (S=512): 8 heads x 8 row tiles of 256 rows = 64 workgroups.
    p = kf.plan(1, 512, 512, 32, 8, 128, num_cus=cus)
    rounds = lambda w: -(-w // cus)
    if 64 >= cus and rounds(32) * 512 * 0.94 < rounds(64) * 256:
        assert p.block_threads == 512 and p.grid_blocks == 32          # wide kernel, 512 rows
    elif 64 >= cus:
        assert p.block_threads == 512 and p.grid_blocks == 64          # 8 waves, one KV group
    elif 8 * (4 * 512 // 128) >= cus:
        assert p.block_threads == 512 and p.grid_blocks == 128         # 2 KV groups, 128 rows
    else:
        assert p.block_threads == 512 and p.grid_blocks == 256         # 4 KV groups, 64 rows
    # C3 prefill: 256 wide workgroups, or 512 of the 256-row kernel where
    # those take less time (80 CUs: 7 rounds of 256 rows against 4 of 512).
    wide_c3 = rounds(256) * 512 * 0.94 < rounds(512) * 256
    assert kf.plan(1, 4096, 4096, 32, 8, 128, num_cus=cus).grid_blocks == (256 if wide_c3 else 512)
    # C2 decode: short splits while the one-wave splits fit 4 per CU.
    p = kf.plan(1, 1, 4096, 32, 8, 128, num_cus=cus)
    w64, w32 = 8 * 64, 8 * 128                   # waves of 64- and 32-key splits
    if w64 == 4 * cus:                           # 64-key splits give exactly 4 waves per CU
        assert p.splits_per_block == 4 and p.kv_per_split == 64
    elif w32 <= 4 * cus:
        assert p.splits_per_block == 4 and p.kv_per_split == 32
    elif w64 <= 4 * cus:
        assert p.splits_per_block == 4 and p.kv_per_split == 64
    else:
        assert p.splits_per_block == 1
    if cus == 32:
        # 1024 one-wave splits would be 32 waves per CU: the streaming
        # kernel, one workgroup per CU (8 heads x 4 splits).
        assert p.splits_per_block == 1 and p.grid_blocks == 32 and p.num_splits == 4
    # C5 decode: 256 heads; busiest CU within 2 % of an even share.
    p = kf.plan(32, 1, 8192, 32, 8, 128, num_cus=cus)
    rounds = -(-256 * p.num_splits // cus) / p.num_splits
    assert rounds <= 256 / cus * 1.02 or p.num_splits == 1 and 256 % cus == 0
    assert p.grid_blocks == 256 * p.num_splits


def test_plan_without_a_visible_device_is_the_mi355x_plan():
    """On a host without a GPU kf_attn_plan plans for a whole MI355X."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: kf_attn_plan uses its CU count")
    for shape in [(1, 4096, 4096, 32, 8, 128), (1, 512, 512, 32, 8, 128), (1, 1, 4096, 32, 8, 128),
                  (32, 1, 8192, 32, 8, 128), (4, 1, 70000, 32, 8, 256)]:
        assert kf.plan(*shape) == kf.plan(*shape, num_cus=256)


def test_plan_for_cus_rejects_bad_counts(lib):
    out = kf._PlanStruct()
    assert lib.kf_attn_plan_for_cus(1, 1, 1, 1, 1, 128, 0, ctypes.byref(out)) == kf.KF_ERR_SIZE
    assert lib.kf_attn_plan_for_cus(1, 1, 1, 1, 1, 128, -4, ctypes.byref(out)) == kf.KF_ERR_SIZE
    assert lib.kf_attn_plan_for_cus(1, 1, 1, 1, 1, 128, 80, None) == kf.KF_ERR_NULL


def _assert_causal_wide_rule():
    """Causal calls at D = 64 / 128 take the wide layout's causal kernel when
    the wide grid has two workgroups per CU or more (256 CUs here: no device),
    q_len is a multiple of 64 and the rows see kv_len - q_len / 2 >= 2048
    keys on average; else the 256-row kernel."""
    wide = "kf_attn_prefill_wide_kernel<{}, true, 1, true>"
    narrow = "kf_attn_prefill_kernel<{}, true, 8, 1>"
    for (B, q, kv, H_q, H_kv, D), want in [
            ((2, 4096, 4096, 32, 8, 128), wide),      # 512 wide workgroups, 2048 keys per row
            ((1, 8192, 8192, 32, 8, 128), wide),
            ((2, 4096, 4096, 32, 8, 64), wide),
            ((2, 4096, 6144, 32, 8, 128), wide),
            ((1, 4096, 4096, 32, 8, 128), narrow),    # one wide workgroup per CU
            ((4, 2048, 2048, 32, 8, 128), narrow),    # 1024 keys per row on average
            ((2, 4096, 3000, 32, 8, 128), narrow),    # 952
            ((2, 4032, 4096, 32, 8, 128), wide),      # q_len = 63 x 64: row tiles across heads
            ((2, 4064, 4096, 32, 8, 128), narrow)]:   # q_len % 64 = 32
        assert kf.kernel_names(B, q, kv, H_q, H_kv, D, causal=True) == want.format(D), (B, q, kv, D)
        # unmasked and key-count calls of these shapes never take the causal kernel
        assert not kf.kernel_names(B, q, kv, H_q, H_kv, D).endswith("true>")
        assert not kf.kernel_names(B, q, kv, H_q, H_kv, D, masked=True).endswith(", true>")


def test_kernel_names_follow_the_plan(lib):
    """kf_attn_kernel_names names the kernels in launch order, as the
    profiler lists them."""
    assert kf.kernel_names(1, 4096, 4096, 32, 8, 128) == "kf_attn_prefill_wide_kernel<128, false, 1, false>"
    assert kf.kernel_names(1, 4096, 4096, 32, 8, 128, masked=True) == "kf_attn_prefill_wide_kernel<128, true, 1, false>"
    assert kf.kernel_names(1, 4096, 4096, 32, 8, 128, causal=True) == "kf_attn_prefill_kernel<128, true, 8, 1>"
    assert kf.kernel_names(1, 2048, 2048, 32, 8, 128) == "kf_attn_prefill_kernel<128, false, 8, 1>"
    assert kf.kernel_names(1, 4096, 4096, 32, 8, 128, causal=True) == \
        "kf_attn_prefill_kernel<128, true, 8, 1>"
    assert kf.kernel_names(1, 512, 512, 32, 8, 128) == "kf_attn_prefill_kernel<128, false, 8, 4>"
    assert kf.kernel_names(1, 256, 256, 32, 8, 128) == "kf_attn_prefill_kernel<128, false, 4, 2>"
    assert kf.kernel_names(1, 4096, 4096, 32, 8, 256) == "kf_attn_prefill_wide_kernel<256, false, 1, false>"
    assert kf.kernel_names(1, 4096, 4096, 32, 8, 256, causal=True) == "kf_attn_prefill_wide_kernel<256, true, 1, false>"
    assert kf.kernel_names(1, 4096, 4096, 32, 8, 256, masked=True) == "kf_attn_prefill_wide_kernel<256, true, 1, false>"
    assert kf.kernel_names(1, 2048, 2048, 16, 4, 256) == "kf_attn_prefill_wide_kernel<256, false, 2, false>"
    assert kf.kernel_names(1, 2048, 2048, 16, 4, 256, causal=True) == "kf_attn_prefill_wide_kernel<256, true, 2, false>"
    assert kf.kernel_names(1, 2048, 255, 16, 4, 256) == "kf_attn_prefill_kernel<256, false, 4, 1>"
    assert kf.kernel_names(1, 2048, 255, 16, 4, 256, causal=True) == "kf_attn_prefill_kernel<256, true, 4, 1>"
    assert kf.kernel_names(1, 1, 4096, 32, 8, 128) == \
        "kf_attn_decode_short_kernel<128, 1> + kf_attn_split_merge_kernel<128, 8, 4>"
    assert kf.kernel_names(32, 1, 8192, 32, 8, 128) == "kf_attn_decode_kernel<128, false>"
    buf = ctypes.create_string_buffer(8)
    _assert_causal_wide_rule()
    assert lib.kf_attn_kernel_names(1, 1, 4096, 32, 8, 128, 0, None, buf, 8) == kf.KF_ERR_SIZE
    assert lib.kf_attn_kernel_names(1, 1, 4096, 32, 8, 128, 0, None, None, 8) == kf.KF_ERR_NULL
    assert lib.kf_attn_kernel_names(1, 1, 4096, 32, 8, 100, 0, None, buf, 8) == kf.KF_ERR_HEAD_DIM


def test_noalloc_validation(lib):
    """kf_attn_fwd_noalloc validates like kf_attn_fwd_ex and refuses a shape
    whose split-KV partials exceed its static scratch before any launch."""
    assert lib.kf_attn_noalloc_scratch_bytes() == 16 << 20
    big = (1, 1, 8192, 256, 8, 128)                    # B, q, kv, H_q, H_kv, D: 16.25 MiB
    assert kf.workspace_bytes(*big) > lib.kf_attn_noalloc_scratch_bytes()
    B, q, kv, H_q, H_kv, D = big
    args = (FAKE, FAKE, FAKE, FAKE, None, None)
    assert lib.kf_attn_fwd_noalloc(*args, B, q, kv, H_q, H_kv, D, None, 0, None) == \
        kf.KF_ERR_SCRATCH
    assert lib.kf_attn_fwd_noalloc(*args, 1, 1, 4096, 32, 8, 100, None, 0, None) == \
        kf.KF_ERR_HEAD_DIM
    assert lib.kf_attn_fwd_noalloc(*args, 0, 1, 4096, 32, 8, 128, None, 0, None) == kf.KF_ERR_SIZE
    assert lib.kf_attn_fwd_noalloc(*args, 1, 1, 4096, 30, 8, 128, None, 0, None) == kf.KF_ERR_GQA
    # A prefill without KV partitions needs no scratch: pointer validation
    # answers first.
    assert kf.plan(1, 300, 100, 8, 2, 128).path == "prefill"
    assert lib.kf_attn_fwd_noalloc(None, FAKE, FAKE, FAKE, None, None, 1, 300, 100, 8, 2, 128,
                                   None, 0, None) == kf.KF_ERR_NULL
    assert lib.kf_attn_fwd_noalloc(FAKE, FAKE, FAKE, FAKE, None, None, 1, 300, 100, 8, 2, 128,
                                   None, 64, None) == kf.KF_ERR_FLAGS
    assert "static maximum" in kf.status_string(kf.KF_ERR_SCRATCH)
    # On a shape beyond the scratch, argument errors still come first, as
    # kf_attn_fwd_ex reports them: flags, NULL, misalignment, then SCRATCH.
    assert lib.kf_attn_fwd_noalloc(*args, B, q, kv, H_q, H_kv, D, None, 64, None) == kf.KF_ERR_FLAGS
    assert lib.kf_attn_fwd_noalloc(None, FAKE, FAKE, FAKE, None, None, B, q, kv, H_q, H_kv, D,
                                   None, 0, None) == kf.KF_ERR_NULL
    assert lib.kf_attn_fwd_noalloc(FAKE, FAKE + 2, FAKE, FAKE, None, None, B, q, kv, H_q, H_kv, D,
                                   None, 0, None) == kf.KF_ERR_ALIGN
    assert lib.kf_attn_fwd_noalloc(*args, B, q, kv, H_q, H_kv, D, ctypes.c_void_p(FAKE + 2), 0,
                                   None) == kf.KF_ERR_ALIGN


def test_split_prefill_runs_without_a_workspace(lib):
    """A split prefill needs no workspace: given none (or too little) it is
    re-planned with fewer KV partitions or unsplit, so the call gets past the
    workspace check (on this GPU-less host it then fails at its first HIP
    call), while a split decode still requires its workspace."""
    shape = dict(B=1, q=16, kv=8192, H_q=32, H_kv=8, D=128)
    assert kf.plan(1, 16, 8192, 32, 8, 128).path == "prefill_split"
    need = kf.workspace_bytes(1, 16, 8192, 32, 8, 128)
    assert need > 0
    assert _fwd(**shape) == kf.KF_ERR_HIP
    assert _fwd(ws=FAKE_WS, ws_bytes=need // 3, **shape) == kf.KF_ERR_HIP
    assert _fwd(ws=FAKE_WS + 16, ws_bytes=need // 3, **shape) == kf.KF_ERR_ALIGN
    assert _fwd(B=1, q=1, kv=4096, H_q=32, H_kv=8) == kf.KF_ERR_WORKSPACE


def test_probe_library_exports_its_header():
    """libkf_probe.so (bench.py's measurement probes, built beside the C++
    bench harness) exports exactly what tests/hip/probe.h declares, and the
    product's library directory and public headers hold no probe."""
    lib_path = os.path.join(REPO, "tests", "hip", "bin", "libkf_probe.so")
    header = os.path.join(REPO, "tests", "hip", "probe.h")
    assert not os.path.exists(os.path.join(os.path.dirname(kf.LIB_PATH), "libkf_probe.so"))
    assert not os.path.exists(os.path.join(REPO, "include", "kf", "probe.h"))
    names = kf.exported_symbols(header)
    assert set(names) == {"kf_probe_read", "kf_probe_empty"}
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True,
                         text=True, check=True).stdout
    assert set(re.findall(r"\s[TW]\s+(kf_\w+)$", out, re.M)) == set(names)
    kf.load_library()
    probe = ctypes.CDLL(lib_path)
    probe.kf_probe_read.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_size_t] + [ctypes.c_void_p] * 2
    assert probe.kf_probe_read(None, FAKE, 1024, FAKE, None) == 1       # null buffer
    assert probe.kf_probe_read(FAKE, FAKE, 1000, FAKE, None) == 1       # not a multiple of 16
    assert probe.kf_probe_read(FAKE + 8, FAKE, 1024, FAKE, None) == 1   # misaligned


def test_prefill_threshold():
    assert kf.plan(1, 8, 100, 4, 1, 128).path != "prefill"   # 32 rows per KV head
    assert kf.plan(1, 9, 100, 4, 1, 128).path == "prefill"   # 36 rows


# ---------------------------------------------------------------------------
# Headers compile; the product never imports the oracle.
# ---------------------------------------------------------------------------
def test_c_header_compiles_as_c(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "kf/attn.h"\nint main(void){kf_attn_plan_t p; return kf_attn_plan(1,1,1,1,1,128,&p);}\n')
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only",
                    f"-I{os.path.join(REPO, 'include')}", str(src)], check=True)


def test_product_does_not_use_oracle():
    pkg = os.path.join(REPO, "kernelfoundry_amd")
    for root, _, files in os.walk(pkg):
        for fn in files:
            if fn.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(root, fn)).read()
                assert "import oracle" not in text and "from oracle" not in text, fn
                assert "cpu_attn" not in text and "kf_oracle" not in text, fn


def _paged(B=2, q=1, H_q=32, H_kv=8, D=128, ps=16, max_pages=64, num_pages=200, table=FAKE,
           lens=FAKE, flags=0, ws=FAKE_WS, ws_bytes=1 << 30):
    return kf.attn_decode_paged_ptr(FAKE, FAKE, FAKE, table, lens, FAKE, 0, 0, B, q, H_q, H_kv, D,
                                    ps, max_pages, num_pages, flags, ws, ws_bytes)


def test_paged_decode_validation():
    for ps in (0, 8, 15, 24, 48, 3 << 10, 1 << 21):
        assert _paged(ps=ps) == kf.KF_ERR_SIZE, ps
    assert _paged(max_pages=0) == kf.KF_ERR_SIZE
    assert _paged(num_pages=0) == kf.KF_ERR_SIZE
    assert _paged(ps=1 << 20, max_pages=4096) == kf.KF_ERR_SIZE       # capacity beyond int
    assert _paged(q=9, H_q=32, H_kv=8) == kf.KF_ERR_SIZE              # 36 rows per KV head
    assert _paged(D=96) == kf.KF_ERR_HEAD_DIM
    assert _paged(H_kv=3) == kf.KF_ERR_GQA
    assert _paged(table=0) == kf.KF_ERR_NULL
    assert _paged(lens=0) == kf.KF_ERR_NULL
    assert _paged(table=FAKE + 2) == kf.KF_ERR_ALIGN
    assert _paged(flags=16) == kf.KF_ERR_FLAGS
    assert _paged(flags=kf.KF_ATTN_OUT_F16 | kf.KF_ATTN_OUT_BF16) == kf.KF_ERR_FLAGS
    need = kf.paged_workspace_bytes(2, 1, 32, 8, 128, 16, 64)
    # Paged decode is planned as the contiguous decode over the capacity
    # (64 pages x 16 rows = 1024 keys): here the short-split kernel's 32
    # one-wave splits of 32 keys, each a partial of 2 x 32 rows of D + 2
    # floats.
    assert need == 32 * 64 * (128 + 2) * 4
    assert kf.workspace_bytes(2, 1, 64 * 16, 32, 8, 128) == need
    assert _paged(ws_bytes=need - 1) == kf.KF_ERR_WORKSPACE
    assert kf.paged_workspace_bytes(2, 9, 32, 8, 128, 16, 64) == 0    # not a decode shape
    assert kf.paged_workspace_bytes(2, 1, 32, 8, 128, 24, 64) == 0    # bad page size


def test_library_loaded_before_torch_keeps_one_hip_runtime():
    """kf.plan() before `import torch` must not leave two HIP / HSA runtimes
    in the process (the library's system libamdhip64.so.7 and the copy
    torch's wheel loads by its unversioned name): load_library() imports torch
    first.  Checked in a fresh interpreter through /proc/self/maps."""
    import subprocess
    import sys
    pytest.importorskip("torch")
    code = (
        "import re, kernelfoundry_amd as kf\n"
        "kf.plan(1, 1, 4096, 32, 8, 128)\n"
        "import torch\n"
        "m = open('/proc/self/maps').read()\n"
        "print(len(set(re.findall(r'\\S*libamdhip64\\S*', m))),"
        " len(set(re.findall(r'\\S*libhsa-runtime64\\S*', m))))\n")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=root,
                       timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.split() == ["1", "1"], r.stdout
