// attn_capi.hip -- C ABI of libkf_attn.so: validation, dispatch plan, launches.
//
// Entry points are declared in include/kf/attn.h.  Every argument check runs
// before the first HIP call, so invalid calls are rejected on any host (the
// CPU-only tests rely on that) and never reach a kernel.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "attn_kernels.h"
#include "kf/attn.h"

namespace {

// The dispatch plan is sized for the device's compute units and XCDs,
// read once per device (hipDeviceGetAttribute).  Without a visible device
// (plan queries on a host without a GPU) it plans for a whole MI355X.
constexpr int kDefaultCUs = 256;        // MI355X in SPX mode
constexpr int kDefaultXcds = 8;
constexpr int kMaxDevices = 64;
constexpr int kDecodeMaxRows = 32;      // query rows per KV head on the decode path
// Streaming decode: a split holds at least one 32-key stage per wave.
inline int decode_min_split_rows(int D) { return kf::decode_waves(D) * kf::kDecodeStage; }

// Splits per KV head for the streaming decode kernel, before the caps.
// D <= 128 (8-wave workgroups, one per CU by LDS): the fewest splits whose
// busiest CU streams at most 2 % more than an even share, where a CU streams
// ceil(n_groups * s / CUs) workgroups of 1 / s of a head each (96 heads: 8
// splits = 3 full rounds, not 3 splits = 1 round plus a 32-workgroup tail).
// D = 256 (4 waves; its LDS holds one workgroup per CU): grids of two
// workgroups per CU, i.e. two rounds, which measured 3 % faster than one.
long long decode_stream_splits(long long n_groups, long long max_splits, int D, int cus) {
    if (D >= 256) return (2LL * cus + n_groups - 1) / n_groups;
    const double even = (double)n_groups / cus;
    long long best = 1;
    double best_t = 1e300;
    for (long long s = 1; s <= max_splits; ++s) {
        const double t = (double)((n_groups * s + cus - 1) / cus) / (double)s;
        if (t <= even * 1.02) return s;
        if (t < best_t * 0.98) {
            best = s;
            best_t = t;
        }
    }
    return best;
}
// Short-split decode (one wave per split of 32 or 64 keys): used while the
// job is at most kShortMaxWavesPerCU such waves per CU; beyond it the
// streaming decode kernel takes over.  64-key splits are preferred while they
// still give kShortMinWavesPerCU waves per CU.  Measured (MI355X, rotated
// inputs, one process): with 8 waves per CU allowed, the 2048-wave jobs (e.g.
// 2 x 8192, 8 x 2048 or 16 x 1024 keys at 32 / 8 heads) ran 1.23-1.26x
// slower than on the streaming kernel and 1536-wave jobs 1.04-1.13x; jobs of
// <= 1024 waves (configs[1], 8 x 1024 keys) are faster on the short kernel.
constexpr long long kShortMaxWavesPerCU = 4;
constexpr long long kShortMinWavesPerCU = 4;
constexpr int kMinGroupKeys = 128;      // keys before a prefill row's keys are split between KV groups
// Keys each KV group of a prefill workgroup keeps in a KV partition (split
// prefill, below).
constexpr int kMinSplitGroupKeys = 64;
// Serial 32-key tiles per KV group a split prefill must save (measured at
// 32 / 8 heads, D = 64 / 128: 4 saved tiles lose 3-22 %, 6 win 18-34 %).
constexpr long long kMinSplitSavedTiles = 6;
// Time of a 32-key tile of the 4-wave D = 256 prefill kernel (128 rows per
// workgroup) relative to one of the wide kernel's KV groups (689 vs 487 us
// for the whole S = 4096, 32 / 8 heads prefill).
constexpr double kSplit256TileCost = 1.4;
// kf_attn_fwd_noalloc's static scratch (split-KV partials), per device.
constexpr size_t kStaticScratchBytes = size_t(16) << 20;
// Time per query row of the wide prefill kernel relative to the 256-row
// kernel (measured at S = 4096, 32 / 8 heads: 254 vs 267-271 us).
constexpr double kWideRowCost = 0.94;
// The same for the 8-wave D = 256 kernel (256 rows per workgroup) against the
// 4-wave one (128 rows): 487 vs 689 us at S = 4096, 32 / 8 heads.
constexpr double kWide256RowCost = 0.7;
// D = 256 grids that the 256-row wide kernel does not take run as the wide
// kernel with two KV groups (8 waves on the 4-wave kernel's 128-row tiles)
// from this many keys per row on: 78.8 vs 94.0 us at S = 2048, 16 / 4 heads,
// 25.5 vs 30.7 at S = 512, 32 / 8.  Where the 256-row kernel is taken it
// stays ahead (S = 1536-5120, 32 / 8 heads: the KV groups 1-6 % slower).
constexpr int kWide256GroupKeys = 2 * kMinGroupKeys;
// Causal calls at D = 64 / 128 take the wide kernel from this many keys per
// query row on average (kv_len - q_len / 2, two wide workgroups per CU or
// more): against the 256-row kernel, A/B in one process, 2 x 4096 and 1 x 8192
// queries at 32 / 8 heads 1.08-1.09x (D = 64 1.02-1.06x), 2 x 4096 queries
// against 6144 keys 1.09x, but 4 x 2048 queries 0.88x.
constexpr int kWideCausalMinKeys = 2048;
constexpr size_t kWsAlign = 256;

thread_local int g_last_hip_error = 0;

struct DeviceShape {
    int cus;
    int xcds;
};

// CU and XCD counts of the device current on the calling thread, cached per
// device; the MI355X defaults when no device is visible.
DeviceShape current_device_shape() {
    static std::atomic<int> cache[kMaxDevices][2];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return {kDefaultCUs, kDefaultXcds};
    }
    int cus = cache[dev][0].load(std::memory_order_relaxed);
    int xcds = cache[dev][1].load(std::memory_order_relaxed);
    if (cus <= 0 || xcds <= 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = kDefaultCUs;
        if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess ||
            xcds <= 0)
            xcds = kDefaultXcds;
        (void)hipGetLastError();
        cache[dev][0].store(cus, std::memory_order_relaxed);
        cache[dev][1].store(xcds, std::memory_order_relaxed);
    }
    return {cus, xcds};
}

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

bool supported_head_dim(int D) { return D == 16 || D == 64 || D == 128 || D == 256; }

struct Plan {
    int path;
    int R;
    int n_groups;
    int rows_total;
    int n_splits;
    int kv_per_split;
    int row_tiles;
    int grid;
    int threads;
    int waves;          // prefill: waves per workgroup
    int kv_groups;      // prefill: KV groups per workgroup (1, 2 or 4)
    int wide_row_tiles; // prefill: row tiles of the wide kernel per KV head (512 rows
                        // at D = 64 / 128, 256 or, with KV groups, 128 at D = 256),
                        // 0 = the 32-row-per-wave kernel
    int wide_grid;      // workgroups of the wide kernel
    int wide_kv_groups; // KV groups of the wide kernel (2: D = 256, 128 rows per workgroup)
    bool wide_causal;   // D = 64 / 128: causal calls take the wide kernel too
    int short_stages;   // decode: 32-key stages per split of the short-split kernel, 0 = streaming kernel
    int merge_cw;       // split merge: float4 columns per wave
    int merge_per;      // split merge: splits per lane
    size_t ws_bytes;
    size_t ws_o_off, ws_m_off, ws_l_off;
    int xcds;           // XCDs of the target device (workgroup id remap)
};

// paged: K/V come from a page pool (kf_attn_decode_paged); the planner
// makes the same choice as for a contiguous cache (both decode kernels have
// a paged form).  cus: compute units of the target device.
// Workspace bytes of split partials (O, M, L) for `parts` (partition, row)
// pairs.
size_t split_ws_bytes(size_t parts, int D) {
    return align_up(parts * D * sizeof(float), kWsAlign) + 2 * align_up(parts * sizeof(float), kWsAlign);
}

bool prefill_path(int path) { return path == KF_PATH_PREFILL || path == KF_PATH_PREFILL_SPLIT; }

// ws_cap: most workspace a split prefill plan may ask for (it then takes
// fewer KV partitions, or none); split decode plans ignore it, and
// kf_attn_fwd_noalloc refuses those that exceed its scratch.
int make_plan(int B, int q_len, int kv_len, int H_q, int H_kv, int D, const DeviceShape& dev,
              Plan* pl, bool paged = false, size_t ws_cap = SIZE_MAX) {
    const int cus = dev.cus;
    if (B <= 0 || q_len <= 0 || kv_len <= 0 || H_q <= 0 || H_kv <= 0 || cus <= 0) return KF_ERR_SIZE;
    if (!supported_head_dim(D)) return KF_ERR_HEAD_DIM;
    if (H_q % H_kv != 0) return KF_ERR_GQA;
    const long long ratio = H_q / H_kv;
    const long long R = ratio * q_len;
    const long long n_groups = (long long)B * H_kv;
    const long long rows_total = n_groups * R;
    // In-head offsets are 32-bit (row * D, kv * D); group bases are 64-bit.
    if (R * D > INT_MAX || (long long)kv_len * D > INT_MAX || rows_total > INT_MAX)
        return KF_ERR_SIZE;

    Plan p{};
    p.xcds = dev.xcds;
    p.R = (int)R;
    p.n_groups = (int)n_groups;
    p.rows_total = (int)rows_total;
    if (R <= kDecodeMaxRows) {
        // Short splits (one wave each) while the whole job is a few waves
        // per CU: 64 keys per split (D <= 128) while that keeps 4 waves per
        // CU, else 32, else 64.  Paged caches too (pages of >= 16 rows: a
        // split spans at most 4 pages).
        int nst = 0;
        {
            const auto waves = [&](int st) { return n_groups * ((kv_len + 32LL * st - 1) / (32LL * st)); };
            const auto fits = [&](int st) {
                return st <= (D >= 256 ? 1 : 2) && waves(st) <= kShortMaxWavesPerCU * cus &&
                       (kv_len + 32LL * st - 1) / (32LL * st) <= kf::kMergeMaxSplits;
            };
            if (fits(2) && waves(2) >= kShortMinWavesPerCU * cus) nst = 2;
            else if (fits(1)) nst = 1;
            else if (fits(2)) nst = 2;
        }
        long long splits, per;
        if (nst > 0) {
            per = 32LL * nst;
            splits = (kv_len + per - 1) / per;
            p.grid = (int)((n_groups * splits + kf::kShortWaves - 1) / kf::kShortWaves);
            p.threads = 64 * kf::kShortWaves;
        } else {
            long long max_splits = kv_len / decode_min_split_rows(D);
            if (max_splits < 1) max_splits = 1;
            if (max_splits > kf::kMergeMaxSplits) max_splits = kf::kMergeMaxSplits;
            splits = decode_stream_splits(n_groups, max_splits, D, cus);
            if (splits > max_splits) splits = max_splits;
            if (splits > kf::kMergeMaxSplits) splits = kf::kMergeMaxSplits;
            if (splits < 1) splits = 1;
            per = (kv_len + splits - 1) / splits;
            per = (per + kf::kDecodeStage - 1) / kf::kDecodeStage * kf::kDecodeStage;
            splits = (kv_len + per - 1) / per;
            if (n_groups * splits > INT_MAX) return KF_ERR_SIZE;
            p.grid = (int)(n_groups * splits);
            p.threads = 64 * kf::decode_waves(D);
        }
        p.short_stages = nst;
        p.n_splits = (int)splits;
        p.kv_per_split = (int)per;
        p.merge_cw = kf::merge_cols(D, p.n_splits);
        p.merge_per = kf::merge_per_lane(p.merge_cw, p.n_splits);
        if (splits > 1 && rows_total * ((D / 4) / p.merge_cw) > INT_MAX) return KF_ERR_SIZE;
        p.path = splits > 1 ? KF_PATH_DECODE_SPLIT : KF_PATH_DECODE;
    } else {
        // Waves per workgroup: the most the head dimension allows.  When that
        // grid would leave CUs without a workgroup, D = 64 / 128 split each
        // row's keys between KV groups of waves: two (8 waves x 128 rows),
        // then four (8 waves x 64 rows) while every group keeps at least
        // kMinGroupKeys keys, else two groups of 4 waves x 64 rows (two such
        // workgroups share a CU); all keep two waves per SIMD.  Other head
        // dimensions halve the waves (down to 2).  D = 256 stays at 4 waves
        // (its accumulators need a SIMD per wave).
        int nw = kf::prefill_max_waves(D), ks = 1;
        const auto wgs = [&](long long rows) { return n_groups * ((R + rows - 1) / rows); };
        if ((D == 64 || D == 128) && wgs(32 * nw) < cus && kv_len >= kMinGroupKeys) {
            ks = 2;
            if (wgs(128) < cus) {
                if (kv_len >= 4LL * kMinGroupKeys)
                    ks = 4;
                else
                    nw = 4;
            }
        } else {
            const int nw_min = D >= 256 ? 4 : 2;
            while (nw > nw_min && wgs(32 * nw) < cus) nw /= 2;
        }
        const int rows = 32 * nw / ks;
        const long long row_tiles = (R + rows - 1) / rows;
        if (n_groups * row_tiles > INT_MAX) return KF_ERR_SIZE;
        p.n_splits = 1;
        p.kv_per_split = kv_len;
        p.row_tiles = (int)row_tiles;
        p.grid = (int)(n_groups * row_tiles);
        p.threads = 64 * nw;
        p.waves = nw;
        p.kv_groups = ks;
        p.path = KF_PATH_PREFILL;
        // Unmasked calls at D = 64 / 128 with 8-wave workgroups: the wide
        // kernel (64 rows per wave, 512 per workgroup) when its rounds of
        // workgroups take less time than the 256-row kernel's; one workgroup
        // runs per CU in either kernel, and a wide row costs kWideRowCost of
        // a 256-row-kernel row (also for calls with key counts, and causal
        // ones when wide_causal, below).  D = 256, masked calls included: the
        // wide kernels' 8 waves x 32 rows against 4 waves x 32 rows, by the
        // same rule (kWide256RowCost), else, from kWide256GroupKeys keys on,
        // the wide kernel with two KV groups on the 4-wave kernel's tiles.
        const bool wide_ok = ((D == 64 || D == 128) && nw == 8 && ks == 1) || (D == 256 && nw == 4);
        if (wide_ok) {
            const int wrows = D >= 256 ? kf::WideCfg<256>::kRows : kf::WideCfg<128>::kRows;
            const double wcost = D >= 256 ? kWide256RowCost : kWideRowCost;
            const long long wrt = (R + wrows - 1) / wrows;
            const long long wg = n_groups * wrt;
            const long long rounds_n = (p.grid + cus - 1) / cus, rounds_w = (wg + cus - 1) / cus;
            if (wg <= INT_MAX && (double)rounds_w * wrows * wcost < (double)rounds_n * rows) {
                p.wide_row_tiles = (int)wrt;
                p.wide_grid = (int)wg;
                p.wide_kv_groups = 1;
                // Causal row tiles differ in length up to the whole key range:
                // dealt longest first, they fill every CU evenly once there
                // are two workgroups per CU or more (the average load per CU
                // then exceeds the longest tile); with fewer, the longest
                // tiles set the launch and the 256-row kernel's twice as many
                // tiles balance better.  A wave's 64 rows must lie in one
                // head (q_len a multiple of 64), and the rows must see
                // kWideCausalMinKeys keys on average: the waves of a 512-row
                // tile end up to 14 tiles apart, and a SIMD whose partner has
                // finished runs its last tiles alone.
                const long long avg_keys = (long long)kv_len - q_len / 2;
                p.wide_causal = wg >= 2LL * cus && q_len % 64 == 0 && avg_keys >= kWideCausalMinKeys;
            } else if (D == 256 && kv_len >= kWide256GroupKeys) {
                p.wide_row_tiles = p.row_tiles;  // 128 rows per workgroup
                p.wide_grid = p.grid;
                p.wide_kv_groups = 2;
            }
        }
        // Few query rows per KV head against many keys (chunked prefill,
        // speculative verification): a grid that leaves half the CUs or more
        // without a workgroup also splits the keys across workgroups into KV
        // partitions -- kf_attn_prefill_kernel writes split partials that
        // the split-merge kernel combines, as on the split decode path -- as
        // many as fit one round of workgroups while every KV group keeps
        // kMinSplitGroupKeys keys of each partition (and the partials fit
        // ws_cap), and only where that shortens each KV group's serial chain
        // by kMinSplitSavedTiles 32-key tiles or more: the merge launch and
        // the partials' round trip cost about that much.  At D = 256 the
        // split runs the 4-wave kernel, whose 32-key tile costs
        // kSplit256TileCost of a wide-kernel tile, against the wide kernel's
        // chain (halved by its two KV groups where it has them).
        if ((p.wide_row_tiles == 0 || D == 256) && 2LL * p.grid <= cus) {
            long long ns = cus / p.grid;
            const long long by_keys = kv_len / ((long long)ks * kMinSplitGroupKeys);
            if (ns > by_keys) ns = by_keys;
            if (ns > kf::kMergeMaxSplits) ns = kf::kMergeMaxSplits;
            while (ns > 1 && split_ws_bytes((size_t)ns * (size_t)rows_total, D) > ws_cap) --ns;
            if (ns > 1) {
                // Partition length: whole tiles for every KV group.
                const long long unit = 32LL * ks;
                long long per = (kv_len + ns - 1) / ns;
                per = (per + unit - 1) / unit * unit;
                ns = (kv_len + per - 1) / per;
                long long saved;
                if (D == 256) {
                    const long long wunit = 32LL * (p.wide_row_tiles > 0 ? p.wide_kv_groups : 1);
                    const double chain = (double)((kv_len + wunit - 1) / wunit);
                    saved = (long long)(chain - kSplit256TileCost * (double)(per / 32));
                } else {
                    const long long tiles = ((long long)kv_len + unit - 1) / unit;  // per KV group, unsplit
                    saved = tiles - per / unit;
                }
                const int cw = kf::merge_cols(D, (int)ns);
                if (ns > 1 && saved >= kMinSplitSavedTiles && (long long)p.grid * ns <= INT_MAX && rows_total * ((D / 4) / cw) <= INT_MAX) {
                    p.n_splits = (int)ns;
                    p.kv_per_split = (int)per;
                    p.grid = (int)((long long)p.grid * ns);
                    p.merge_cw = cw;
                    p.merge_per = kf::merge_per_lane(cw, p.n_splits);
                    p.path = KF_PATH_PREFILL_SPLIT;
                    p.wide_row_tiles = 0;  // D = 256: the 4-wave kernel
                    p.wide_grid = 0;
                }
            }
        }
    }
    if (p.path == KF_PATH_DECODE_SPLIT || p.path == KF_PATH_PREFILL_SPLIT) {
        const size_t parts = (size_t)p.n_splits * (size_t)rows_total;
        p.ws_o_off = 0;
        p.ws_m_off = align_up(parts * D * sizeof(float), kWsAlign);
        p.ws_l_off = p.ws_m_off + align_up(parts * sizeof(float), kWsAlign);
        p.ws_bytes = p.ws_l_off + align_up(parts * sizeof(float), kWsAlign);
    }
    *pl = p;
    return KF_OK;
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

int hip_fail(hipError_t e) {
    g_last_hip_error = (int)e;
    return KF_ERR_HIP;
}

template <int D, int NW, int KS = 1>
void launch_prefill(const Plan& pl, const kf::AttnParams& prm, bool mask, hipStream_t stream) {
    if constexpr (D >= 256 && NW == 4 && KS == 1) {
        // The KV-partition code is a kernel of its own at D = 256.
        if (pl.path == KF_PATH_PREFILL_SPLIT) {
            if (mask)
                kf::kf_attn_prefill_parts_kernel<D, true><<<dim3(pl.grid), dim3(pl.threads), 0, stream>>>(prm);
            else
                kf::kf_attn_prefill_parts_kernel<D, false><<<dim3(pl.grid), dim3(pl.threads), 0, stream>>>(prm);
            return;
        }
    }
    if (mask)
        kf::kf_attn_prefill_kernel<D, true, NW, KS><<<dim3(pl.grid), dim3(pl.threads), 0, stream>>>(prm);
    else
        kf::kf_attn_prefill_kernel<D, false, NW, KS><<<dim3(pl.grid), dim3(pl.threads), 0, stream>>>(prm);
}

// The prefill kernel of the plan (either prefill path).
template <int D>
hipError_t launch_prefill_kernel(const Plan& pl, const kf::AttnParams& prm, hipStream_t stream) {
    const bool mask = prm.causal || prm.kv_lens;
    if constexpr (D >= 256) {
        if (pl.wide_row_tiles > 0) {
            kf::AttnParams pw = prm;
            pw.row_tiles = pl.wide_row_tiles;
            const dim3 grid(pl.wide_grid), block(kf::WideCfg<D>::kThreads);
            if (pl.wide_kv_groups == 2) {
                if (mask)
                    kf::kf_attn_prefill_wide_kernel<D, true, 2><<<grid, block, 0, stream>>>(pw);
                else
                    kf::kf_attn_prefill_wide_kernel<D, false, 2><<<grid, block, 0, stream>>>(pw);
            } else if (mask) {
                kf::kf_attn_prefill_wide_kernel<D, true, 1><<<grid, block, 0, stream>>>(pw);
            } else {
                kf::kf_attn_prefill_wide_kernel<D, false, 1><<<grid, block, 0, stream>>>(pw);
            }
            return hipGetLastError();
        }
        launch_prefill<D, 4>(pl, prm, mask, stream);
    } else {
        if constexpr (D == 64 || D == 128) {
            if (pl.kv_groups == 4) {
                launch_prefill<D, 8, 4>(pl, prm, mask, stream);
                return hipGetLastError();
            }
            if (pl.kv_groups == 2) {
                if (pl.waves == 8)
                    launch_prefill<D, 8, 2>(pl, prm, mask, stream);
                else
                    launch_prefill<D, 4, 2>(pl, prm, mask, stream);
                return hipGetLastError();
            }
        }
        if constexpr (D == 64 || D == 128) {
            // Causal calls take the wide layout's causal kernel when its grid
            // balances (wide_causal), else the 256-row kernel.
            if (pl.wide_row_tiles > 0 && (!prm.causal || pl.wide_causal)) {
                kf::AttnParams pw = prm;
                pw.row_tiles = pl.wide_row_tiles;
                if (prm.causal)
                    kf::kf_attn_prefill_wide_kernel<D, true, 1, true><<<dim3(pl.wide_grid),
                                                                dim3(kf::WideCfg<D>::kThreads), 0, stream>>>(pw);
                else if (mask)
                    kf::kf_attn_prefill_wide_kernel<D, true, 1><<<dim3(pl.wide_grid),
                                                                  dim3(kf::WideCfg<D>::kThreads), 0, stream>>>(pw);
                else
                    kf::kf_attn_prefill_wide_kernel<D, false, 1><<<dim3(pl.wide_grid),
                                                                   dim3(kf::WideCfg<D>::kThreads), 0, stream>>>(pw);
                return hipGetLastError();
            }
        }
        if (pl.waves == 8) {
            launch_prefill<D, 8>(pl, prm, mask, stream);
        } else if (pl.waves == 4) {
            launch_prefill<D, 4>(pl, prm, mask, stream);
        } else {
            launch_prefill<D, 2>(pl, prm, mask, stream);
        }
    }
    return hipGetLastError();
}

// The split-merge kernel over the plan's partials (split decode and split
// prefill).
template <int D>
hipError_t launch_merge(const Plan& pl, const kf::AttnParams& prm, hipStream_t stream) {
    const dim3 mgrid(pl.rows_total * ((D / 4) / pl.merge_cw)), mblock(kf::kMergeThreads);
    // The (column block, splits per lane) pairs merge_cols / merge_per_lane
    // produce: the widest block with up to kMergeTarget (kMergePer when the
    // widest is 4) splits per lane, narrower blocks with kMergeTarget, and
    // CW = 4 with kMergePer.
    constexpr int kCWMax = D / 4 < 64 ? D / 4 : 64;
    constexpr int kT = kf::kMergeTarget, kP = kf::kMergePer;
    const int cw = pl.merge_cw, per = pl.merge_per;
    if (cw == kCWMax) {
        switch (per) {
            case 1: kf::kf_attn_split_merge_kernel<D, 1, kCWMax><<<mgrid, mblock, 0, stream>>>(prm); break;
            case 2: kf::kf_attn_split_merge_kernel<D, 2, kCWMax><<<mgrid, mblock, 0, stream>>>(prm); break;
            case 4: kf::kf_attn_split_merge_kernel<D, 4, kCWMax><<<mgrid, mblock, 0, stream>>>(prm); break;
            case kT: kf::kf_attn_split_merge_kernel<D, kT, kCWMax><<<mgrid, mblock, 0, stream>>>(prm); break;
            case kP:
                if constexpr (kCWMax == 4) {  // D = 16: the widest block is the narrowest
                    kf::kf_attn_split_merge_kernel<D, kP, 4><<<mgrid, mblock, 0, stream>>>(prm);
                    break;
                } else {
                    return hipErrorInvalidValue;  // not planned
                }
            default: return hipErrorInvalidValue;
        }
    } else if (cw == 4 && per == kP) {
        kf::kf_attn_split_merge_kernel<D, kP, 4><<<mgrid, mblock, 0, stream>>>(prm);
    } else if (per == kT) {
        switch (cw) {
            case 4: kf::kf_attn_split_merge_kernel<D, kT, 4><<<mgrid, mblock, 0, stream>>>(prm); break;
            case 8:
                if constexpr (kCWMax > 8) {
                    kf::kf_attn_split_merge_kernel<D, kT, 8><<<mgrid, mblock, 0, stream>>>(prm);
                    break;
                } else {
                    return hipErrorInvalidValue;
                }
            case 16:
                if constexpr (kCWMax > 16) {
                    kf::kf_attn_split_merge_kernel<D, kT, 16><<<mgrid, mblock, 0, stream>>>(prm);
                    break;
                } else {
                    return hipErrorInvalidValue;
                }
            case 32:
                if constexpr (kCWMax > 32) {
                    kf::kf_attn_split_merge_kernel<D, kT, 32><<<mgrid, mblock, 0, stream>>>(prm);
                    break;
                } else {
                    return hipErrorInvalidValue;
                }
            default: return hipErrorInvalidValue;
        }
    } else {
        return hipErrorInvalidValue;  // not a pair the planner makes
    }
    return hipGetLastError();
}

template <int D>
hipError_t launch_all(const Plan& pl, const kf::AttnParams& prm, hipStream_t stream) {
    if (prefill_path(pl.path)) {
        const hipError_t e = launch_prefill_kernel<D>(pl, prm, stream);
        if (e != hipSuccess || pl.path != KF_PATH_PREFILL_SPLIT) return e;
        return launch_merge<D>(pl, prm, stream);
    }
    const dim3 grid(pl.grid), block(pl.threads);
    if (prm.block_table) {
        if (pl.short_stages == 0) {
            kf::kf_attn_decode_kernel<D, true><<<grid, block, 0, stream>>>(prm);
        } else if (pl.short_stages == 1) {
            kf::kf_attn_decode_short_paged_kernel<D, 1><<<grid, block, 0, stream>>>(prm);
        } else {
            if constexpr (kf::kShortMaxStages<D> >= 2)
                kf::kf_attn_decode_short_paged_kernel<D, 2><<<grid, block, 0, stream>>>(prm);
            else
                return hipErrorInvalidValue;  // the planner never asks for it
        }
    } else if (pl.short_stages == 0) {
        kf::kf_attn_decode_kernel<D, false><<<grid, block, 0, stream>>>(prm);
    } else if (pl.short_stages == 1) {
        kf::kf_attn_decode_short_kernel<D, 1><<<grid, block, 0, stream>>>(prm);
    } else {
        if constexpr (kf::kShortMaxStages<D> >= 2)
            kf::kf_attn_decode_short_kernel<D, 2><<<grid, block, 0, stream>>>(prm);
        else
            return hipErrorInvalidValue;  // the planner never asks for it
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || pl.path != KF_PATH_DECODE_SPLIT) return e;
    return launch_merge<D>(pl, prm, stream);
}

// Flag, pointer and alignment checks shared by every forward entry point,
// in this order (after the shape checks of make_plan, before anything about
// the workspace or scratch): unknown or conflicting flags, NULL tensors,
// misaligned tensors, misaligned key-count / block-table arrays.
int check_args(int flags, const void* Q, const void* K, const void* V, const void* O,
               const int* kv_lens, const int* block_table) {
    constexpr int kKnown = KF_ATTN_CAUSAL | KF_ATTN_OUT_F16 | KF_ATTN_OUT_BF16 | KF_ATTN_LSE;
    if ((flags & ~kKnown) != 0) return KF_ERR_FLAGS;
    if ((flags & KF_ATTN_OUT_F16) && (flags & KF_ATTN_OUT_BF16)) return KF_ERR_FLAGS;
    if (!Q || !K || !V || !O) return KF_ERR_NULL;
    if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O)) return KF_ERR_ALIGN;
    if ((reinterpret_cast<uintptr_t>(kv_lens) & 3u) != 0) return KF_ERR_ALIGN;
    if ((reinterpret_cast<uintptr_t>(block_table) & 3u) != 0) return KF_ERR_ALIGN;
    return KF_OK;
}

// Shared tail of kf_attn_fwd_ex and kf_attn_decode_paged: argument and
// workspace checks, the common kernel parameters, the launches.  `prm`
// arrives with the masking / paging fields already set.
int run(const Plan& pl, kf::AttnParams prm, const void* Q, const void* K, const void* V, void* O,
        float* row_max, float* row_sumexp, int q_len, int kv_len, int H_kv, int D, int flags,
        void* workspace, size_t workspace_bytes, void* stream) {
    const int st = check_args(flags, Q, K, V, O, prm.kv_lens, prm.block_table);
    if (st != KF_OK) return st;
    if (pl.ws_bytes > 0) {
        if (!workspace || workspace_bytes < pl.ws_bytes) return KF_ERR_WORKSPACE;
        if ((reinterpret_cast<uintptr_t>(workspace) & (kWsAlign - 1)) != 0) return KF_ERR_ALIGN;
    }

    prm.Q = static_cast<const uint16_t*>(Q);
    prm.K = static_cast<const uint16_t*>(K);
    prm.V = static_cast<const uint16_t*>(V);
    prm.O = static_cast<float*>(O);
    prm.out_dtype = (flags & KF_ATTN_OUT_F16) ? kf::kOutF16 : (flags & KF_ATTN_OUT_BF16) ? kf::kOutBF16 : kf::kOutF32;
    prm.lse = (flags & KF_ATTN_LSE) ? 1 : 0;
    prm.Mi = row_max;
    prm.Li = row_sumexp;
    if (pl.ws_bytes > 0) {
        char* ws = static_cast<char*>(workspace);
        prm.Opart = reinterpret_cast<float*>(ws + pl.ws_o_off);
        prm.Mpart = reinterpret_cast<float*>(ws + pl.ws_m_off);
        prm.Lpart = reinterpret_cast<float*>(ws + pl.ws_l_off);
    }
    prm.rows_per_group = pl.R;
    prm.kv_len = kv_len;
    prm.row_tiles = pl.row_tiles;
    prm.n_splits = pl.n_splits;
    prm.kv_per_split = pl.kv_per_split;
    prm.rows_total = pl.rows_total;
    const double scale = 1.0 / __builtin_sqrt((double)D);
    prm.scale = 1.0f / __builtin_sqrtf((float)D);  // the reference's fp32 scale
    prm.scale_log2 = (float)(scale * 1.4426950408889634);
    prm.causal = (flags & KF_ATTN_CAUSAL) ? 1 : 0;
    prm.q_len = q_len;
    prm.heads_kv = H_kv;
    prm.xcds = pl.xcds;

    hipStream_t s = static_cast<hipStream_t>(stream);
    // Launch errors are read back with hipGetLastError(); clear whatever an
    // earlier, unrelated HIP call on this thread left there first, so that
    // only this call's own launches decide its status.
    (void)hipGetLastError();
    hipError_t e;
    switch (D) {
        case 16: e = launch_all<16>(pl, prm, s); break;
        case 64: e = launch_all<64>(pl, prm, s); break;
        case 128: e = launch_all<128>(pl, prm, s); break;
        default: e = launch_all<256>(pl, prm, s); break;
    }
    if (e != hipSuccess) return hip_fail(e);
    return KF_OK;
}

// ---- Static split-KV scratch of kf_attn_fwd_noalloc. ----
// One array per device, resident until the process ends; the entry point
// uses it in place of a caller workspace and never allocates.  In host code
// `scratch` names a host-side stand-in, not device memory: only the address
// hipGetSymbolAddress returns (kept per device) is passed to kernels.
__device__ __align__(256) char scratch[kStaticScratchBytes];

// Device address of this device's `scratch` (device current on the calling
// thread), resolved once per device and kept for the life of the process;
// nullptr and the HIP error on failure.  hipDeviceReset() unloads this
// library's code objects and with them the array, so the kept address is
// stale after it: kf_attn_fwd_noalloc is not for processes that reset a
// device they have already called it on.
void* static_scratch(hipError_t* err) {
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && (dev < 0 || dev >= kMaxDevices)) e = hipErrorInvalidDevice;
    if (e != hipSuccess) {
        *err = e;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
            return nullptr;
        }
        addr[dev] = ptr;
    }
    return addr[dev];
}

// Paged geometry: page_size a power of two in [16, 2^20], positive counts,
// key capacity max_pages_per_seq * page_size within int.  Returns the
// status and, on success, log2(page_size) and the capacity.
int paged_geometry(int page_size, int max_pages_per_seq, int num_pages, int* shift, int* cap) {
    if (max_pages_per_seq <= 0 || num_pages <= 0) return KF_ERR_SIZE;
    if (page_size < 16 || page_size > (1 << 20) || (page_size & (page_size - 1)) != 0)
        return KF_ERR_SIZE;
    const long long c = (long long)page_size * max_pages_per_seq;
    if (c > INT_MAX) return KF_ERR_SIZE;
    int sh = 0;
    while ((1 << sh) < page_size) ++sh;
    *shift = sh;
    *cap = (int)c;
    return KF_OK;
}

int describe_plan(int B, int q_len, int kv_len, int H_q, int H_kv, int D, const DeviceShape& dev,
                  kf_attn_plan_t* plan) {
    if (!plan) return KF_ERR_NULL;
    Plan pl;
    const int st = make_plan(B, q_len, kv_len, H_q, H_kv, D, dev, &pl);
    if (st != KF_OK) return st;
    plan->path = pl.path;
    plan->rows_per_group = pl.R;
    plan->num_splits = pl.n_splits;
    plan->kv_per_split = pl.kv_per_split;
    // The unmasked dispatch (kf_attn_fwd); causal calls of kf_attn_fwd_ex
    // run the 256-row kernel's grid at D = 64 / 128 and this grid at D = 256.
    plan->grid_blocks = pl.wide_row_tiles > 0 ? pl.wide_grid : pl.grid;
    plan->block_threads = pl.wide_row_tiles > 0 ? kf::WideCfg<128>::kThreads : pl.threads;
    plan->workspace_bytes = pl.ws_bytes;
    plan->splits_per_block = prefill_path(pl.path) ? 0 : pl.short_stages > 0 ? kf::kShortWaves : 1;
    return KF_OK;
}

}  // namespace

extern "C" {

int kf_attn_plan(int B, int q_len, int kv_len, int H_q, int H_kv, int D, kf_attn_plan_t* plan) {
    return describe_plan(B, q_len, kv_len, H_q, H_kv, D, current_device_shape(), plan);
}

int kf_attn_plan_for_cus(int B, int q_len, int kv_len, int H_q, int H_kv, int D, int num_cus,
                         kf_attn_plan_t* plan) {
    if (num_cus <= 0) return KF_ERR_SIZE;
    return describe_plan(B, q_len, kv_len, H_q, H_kv, D, DeviceShape{num_cus, kDefaultXcds}, plan);
}

int kf_attn_kernel_names(int B, int q_len, int kv_len, int H_q, int H_kv, int D, int flags,
                         const int* kv_lens, char* buf, size_t buf_bytes) {
    if (!buf || buf_bytes == 0) return KF_ERR_NULL;
    Plan pl;
    const int st = make_plan(B, q_len, kv_len, H_q, H_kv, D, current_device_shape(), &pl);
    if (st != KF_OK) return st;
    char tmp[192];
    int n;
    if (prefill_path(pl.path)) {
        const bool causal = (flags & KF_ATTN_CAUSAL) != 0;
        const bool mask = causal || kv_lens;
        if (pl.wide_row_tiles > 0 && causal && D < 256 && pl.wide_causal)
            n = snprintf(tmp, sizeof(tmp), "kf_attn_prefill_wide_kernel<%d, true, 1, true>", D);
        else if (pl.wide_row_tiles > 0 && (!causal || D >= 256))
            n = snprintf(tmp, sizeof(tmp), "kf_attn_prefill_wide_kernel<%d, %s, %d, false>", D,
                         mask ? "true" : "false", pl.wide_kv_groups);
        else if (D >= 256 && pl.path == KF_PATH_PREFILL_SPLIT)
            n = snprintf(tmp, sizeof(tmp), "kf_attn_prefill_parts_kernel<%d, %s>", D, mask ? "true" : "false");
        else
            n = snprintf(tmp, sizeof(tmp), "kf_attn_prefill_kernel<%d, %s, %d, %d>", D,
                         mask ? "true" : "false", pl.waves, pl.kv_groups);
        if (pl.path == KF_PATH_PREFILL_SPLIT)
            n += snprintf(tmp + n, sizeof(tmp) - (size_t)n, " + kf_attn_split_merge_kernel<%d, %d, %d>", D,
                          pl.merge_per, pl.merge_cw);
    } else {
        if (pl.short_stages > 0)
            n = snprintf(tmp, sizeof(tmp), "kf_attn_decode_short_kernel<%d, %d>", D, pl.short_stages);
        else
            n = snprintf(tmp, sizeof(tmp), "kf_attn_decode_kernel<%d, false>", D);
        if (pl.path == KF_PATH_DECODE_SPLIT)
            n += snprintf(tmp + n, sizeof(tmp) - (size_t)n, " + kf_attn_split_merge_kernel<%d, %d, %d>", D,
                          pl.merge_per, pl.merge_cw);
    }
    if (n < 0 || (size_t)n + 1 > buf_bytes) return KF_ERR_SIZE;
    memcpy(buf, tmp, (size_t)n + 1);
    return KF_OK;
}

size_t kf_attn_workspace_bytes(int B, int q_len, int kv_len, int H_q, int H_kv, int D) {
    Plan pl;
    if (make_plan(B, q_len, kv_len, H_q, H_kv, D, current_device_shape(), &pl) != KF_OK) return 0;
    return pl.ws_bytes;
}

int kf_attn_fwd(const void* Q, const void* K, const void* V, float* O, float* row_max,
                float* row_sumexp, int B, int q_len, int kv_len, int H_q, int H_kv, int D,
                void* workspace, size_t workspace_bytes, void* stream) {
    return kf_attn_fwd_ex(Q, K, V, O, row_max, row_sumexp, B, q_len, kv_len, H_q, H_kv, D,
                          nullptr, 0, workspace, workspace_bytes, stream);
}

int kf_attn_fwd_ex(const void* Q, const void* K, const void* V, void* O, float* row_max,
                   float* row_sumexp, int B, int q_len, int kv_len, int H_q, int H_kv, int D,
                   const int* kv_lens, int flags, void* workspace, size_t workspace_bytes,
                   void* stream) {
    Plan pl;
    const DeviceShape dev = current_device_shape();
    const int st = make_plan(B, q_len, kv_len, H_q, H_kv, D, dev, &pl);
    if (st != KF_OK) return st;
    // A split prefill is an optimisation, not a requirement: without a
    // workspace that holds its partials it runs with as many KV partitions
    // as the given workspace holds, or unsplit (no workspace at all), so a
    // prefill call never fails for want of a workspace.  Split decode plans
    // keep their workspace requirement.
    if (pl.path == KF_PATH_PREFILL_SPLIT && (!workspace || workspace_bytes < pl.ws_bytes))
        (void)make_plan(B, q_len, kv_len, H_q, H_kv, D, dev, &pl, false, workspace ? workspace_bytes : 0);
    kf::AttnParams prm{};
    prm.kv_lens = kv_lens;
    return run(pl, prm, Q, K, V, O, row_max, row_sumexp, q_len, kv_len, H_kv, D, flags,
               workspace, workspace_bytes, stream);
}

int kf_attn_fwd_noalloc(const void* Q, const void* K, const void* V, void* O, float* row_max,
                        float* row_sumexp, int B, int q_len, int kv_len, int H_q, int H_kv, int D,
                        const int* kv_lens, int flags, void* stream) {
    Plan pl;
    // Split prefill partitions are limited to what the scratch holds.
    int st = make_plan(B, q_len, kv_len, H_q, H_kv, D, current_device_shape(), &pl, false,
                       kStaticScratchBytes);
    if (st != KF_OK) return st;
    // The argument errors of kf_attn_fwd_ex come before any scratch question.
    st = check_args(flags, Q, K, V, O, kv_lens, nullptr);
    if (st != KF_OK) return st;
    if (pl.ws_bytes > kStaticScratchBytes) return KF_ERR_SCRATCH;
    void* ws = nullptr;
    if (pl.ws_bytes > 0) {
        hipError_t e = hipSuccess;
        ws = static_scratch(&e);
        if (!ws) return hip_fail(e);
    }
    kf::AttnParams prm{};
    prm.kv_lens = kv_lens;
    return run(pl, prm, Q, K, V, O, row_max, row_sumexp, q_len, kv_len, H_kv, D, flags, ws,
               pl.ws_bytes, stream);
}

size_t kf_attn_noalloc_scratch_bytes(void) { return kStaticScratchBytes; }

size_t kf_attn_decode_paged_workspace_bytes(int B, int q_len, int H_q, int H_kv, int D,
                                            int page_size, int max_pages_per_seq) {
    int sh, cap;
    if (paged_geometry(page_size, max_pages_per_seq, 1, &sh, &cap) != KF_OK) return 0;
    Plan pl;
    if (make_plan(B, q_len, cap, H_q, H_kv, D, current_device_shape(), &pl, true) != KF_OK ||
        prefill_path(pl.path))
        return 0;
    return pl.ws_bytes;
}

int kf_attn_decode_paged(const void* Q, const void* K_pages, const void* V_pages,
                         const int* block_table, const int* kv_lens, void* O, float* row_max,
                         float* row_sumexp, int B, int q_len, int H_q, int H_kv, int D,
                         int page_size, int max_pages_per_seq, int num_pages, int flags,
                         void* workspace, size_t workspace_bytes, void* stream) {
    int sh, cap;
    int st = paged_geometry(page_size, max_pages_per_seq, num_pages, &sh, &cap);
    if (st != KF_OK) return st;
    Plan pl;
    st = make_plan(B, q_len, cap, H_q, H_kv, D, current_device_shape(), &pl, true);
    if (st != KF_OK) return st;
    if (prefill_path(pl.path)) return KF_ERR_SIZE;  // more than 32 query rows per KV head
    if (!block_table || !kv_lens) return KF_ERR_NULL;
    kf::AttnParams prm{};
    prm.kv_lens = kv_lens;
    prm.block_table = block_table;
    prm.max_pages = max_pages_per_seq;
    prm.page_shift = sh;
    prm.num_pages = num_pages;
    return run(pl, prm, Q, K_pages, V_pages, O, row_max, row_sumexp, q_len, cap, H_kv, D, flags,
               workspace, workspace_bytes, stream);
}

int kf_launch_flash_attn(const uint16_t* Q, const uint16_t* K, const uint16_t* V, float* O,
                         int B, int S, int H_q, int H_kv, int D, void* stream) {
    Plan pl;
    if (make_plan(B, S, S, H_q, H_kv, D, current_device_shape(), &pl) != KF_OK)
        return (int)hipErrorInvalidValue;
    if (!Q || !K || !V || !O || !aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O))
        return (int)hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    void* ws = nullptr;
    hipError_t e = hipSuccess;
    if (pl.ws_bytes > 0) {
        e = hipMalloc(&ws, pl.ws_bytes);
        if (e != hipSuccess) {
            g_last_hip_error = (int)e;
            return (int)e;
        }
    }
    const int st = kf_attn_fwd(Q, K, V, O, nullptr, nullptr, B, S, S, H_q, H_kv, D, ws,
                               pl.ws_bytes, stream);
    if (st == KF_ERR_HIP)
        e = (hipError_t)g_last_hip_error;
    else if (st != KF_OK)
        e = hipErrorInvalidValue;
    if (e == hipSuccess) e = hipStreamSynchronize(s);  // scratch must outlive the kernels
    if (ws) (void)hipFree(ws);
    if (e != hipSuccess) g_last_hip_error = (int)e;
    return (int)e;
}

const char* kf_status_string(int status) {
    switch (status) {
        case KF_OK: return "ok";
        case KF_ERR_HEAD_DIM: return "unsupported head dimension (D must be 16, 64, 128 or 256)";
        case KF_ERR_GQA: return "H_q must be a positive multiple of H_kv";
        case KF_ERR_SIZE: return "invalid size (non-positive or beyond 32-bit in-head indexing)";
        case KF_ERR_NULL: return "required pointer is NULL";
        case KF_ERR_WORKSPACE: return "workspace missing or smaller than kf_attn_workspace_bytes()";
        case KF_ERR_ALIGN: return "device pointer not 16-byte aligned (workspace: 256-byte)";
        case KF_ERR_HIP: return "HIP runtime error (see kf_last_hip_error)";
        case KF_ERR_FLAGS: return "unknown or conflicting flag bits (KF_ATTN_CAUSAL, KF_ATTN_OUT_F16 or KF_ATTN_OUT_BF16, KF_ATTN_LSE)";
        case KF_ERR_SCRATCH: return "shape needs more split-KV scratch than kf_attn_fwd_noalloc's static maximum (kf_attn_noalloc_scratch_bytes); use kf_attn_fwd_ex with a workspace";
        default: return "unknown status";
    }
}

int kf_last_hip_error(void) { return g_last_hip_error; }

const char* kf_version(void) { return "kernelfoundry_amd 0.2.0 (gfx950)"; }

}  // extern "C"
