// attn_kernels.h -- gfx950 (CDNA4) flash-attention forward kernels.
//
// Four kernels, all hand-written for wave64 and the fp16 MFMA
// v_mfma_f32_32x32x16_f16:
//
//   kf_attn_prefill_kernel<D, kMask, NW>
//                              one workgroup = NW waves x 32 query rows of
//                              one KV head (NW = 8, 4 for D = 256, fewer for
//                              small grids); K/V streamed HBM -> LDS by
//                              LDS-DMA through a ring of LDS stages; online
//                              softmax in registers; kMask adds causal
//                              masking / per-sequence key counts.
//   kf_attn_decode_kernel<D, kPaged>
//                              split-KV ("flash-decoding") for <= 32 query
//                              rows per KV head (Q_len = 1 decode, GQA/MQA
//                              groups): every wave streams its own KV stages
//                              through a wave-private LDS slot; the waves of
//                              a workgroup merge in LDS; with several splits
//                              each workgroup writes an unnormalised partial;
//                              kPaged reads K/V through a block table.
//   kf_attn_decode_short_kernel<D, NST> / kf_attn_decode_short_paged_kernel<D, NST>
//                              split-KV for small decode jobs: every wave is
//                              one split of 32 or 64 keys and issues all of
//                              its loads at once (one memory round trip);
//                              the paged form reads K/V through a block table.
//   kf_attn_split_merge_kernel<D, NPER, CW>
//                              merges the split partials into O, Mi, Li.
//
// Behaviour follows the reference forward (kernels/flash_attn.cu:384-585):
// O = softmax(Q K^T / sqrt(D)) V per (b, h_q) with h_kv = h_q / (H_q / H_kv)
// (:406), fp16 inputs, fp32 accumulation and softmax, P rounded to fp16
// before the P.V product (:301-303; the row sum here adds those same fp16
// values, where the reference adds the fp32 P, :284-294: at most 2^-12
// relative apart), O divided by the row sum once at the end (:582-584), and the
// row statistics Mi = max_j s_ij and Li = sum_j exp(s_ij - Mi) written once
// (:559-579).  The tiling, data layout, MFMA formulation and split-KV path
// are this library's own (see the comments at each kernel).
//
// Query rows of one KV head.  With Q laid out [B, H_q, q_len, D] and the
// query heads of a group contiguous (h_q / ratio), the ratio * q_len query
// rows that read KV head (b, h_kv) are one contiguous block of Q (and of O,
// Mi, Li) starting at row (b * H_kv + h_kv) * ratio * q_len.  Every kernel
// works on that "group row" view, so GQA/MQA heads share each K/V stage.
//
// MFMA formulation (wave64, 32x32x16 fp16 -> fp32):
//   S^T = K . Q^T   A = K rows from LDS (lane l: kv row l%32, 8 d values),
//                   B = Q^T from registers (lane l: query row l%32, the same
//                   8 d values), C: lane l holds query row l%32 and the 16 kv
//                   rows 8*(r/4) + 4*(l/32) + r%4, r = 0..15.
//   O^T += V^T . P^T  A = V^T from LDS (lane l: d row l%32, 8 kv values),
//                   B = P^T taken straight from the S^T accumulator (lane l:
//                   query row l%32, 8 of its kv values), so P never leaves
//                   registers; C: lane l holds query row l%32 and 16 d values.
// Each lane therefore owns one query row: the row max needs one exchange
// with lane l^32 and the row sum none until the end.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>

namespace kf {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
// The running max used for exponentiation only moves when a new tile max
// exceeds it by more than this many powers of two; P then stays <= 2^8,
// exact in fp16's range, and most tiles skip the O rescale.
constexpr float kLazyRescaleLog2 = 8.0f;

// ---------------------------------------------------------------------------
// Kernel parameter blocks (passed by value).
// ---------------------------------------------------------------------------
struct AttnParams {
    const uint16_t* Q;
    const uint16_t* K;
    const uint16_t* V;
    float* O;           // final output (unsplit paths and combine)
    float* Mi;          // optional
    float* Li;          // optional
    float* Opart;       // split partials [B * H_kv][n_splits][R][D], unnormalised
    float* Mpart;       // [B * H_kv][n_splits][R]  max of scaled scores
    float* Lpart;       // [B * H_kv][n_splits][R]  sum of exp relative to Mpart
    int rows_per_group; // R = (H_q / H_kv) * q_len
    int kv_len;
    int row_tiles;      // prefill: ceil(R / rows per workgroup)
    int n_splits;       // KV partitions per group (split decode / split prefill), else 1
    int kv_per_split;   // keys per partition: a multiple of 32 (of 32 x KV groups on prefill)
    int rows_total;     // B * H_q * q_len
    float scale;        // 1 / sqrt(D), fp32 (the reference's softmax scale)
    float scale_log2;   // scale * log2(e)
    // Key masking (kf_attn_fwd_ex).  Sequence b uses keys [0, kv_lens[b])
    // of its K/V rows (kv_len rows are allocated per head); with `causal`,
    // query i of q_len additionally sees keys j <= i + kv_lens[b] - q_len
    // (bottom-right aligned).  Rows left without keys give O = 0,
    // Mi = -inf, Li = 0.
    const int* kv_lens; // [B] or null (all kv_len)
    int causal;         // 0 / 1
    int q_len;
    int heads_kv;       // H_kv: group index -> batch index
    // Paged K/V (kf_attn_decode_paged): K and V point to page pools
    // [num_pages][H_kv][page_size][D]; key j of sequence b lives in page
    // block_table[b * max_pages + j / page_size], row j % page_size.  A page
    // id outside [0, num_pages) contributes no keys (it is never read).
    const int* block_table;
    int max_pages;      // block_table row length; kv_len = max_pages * page_size
    int page_shift;     // log2(page_size), page_size >= 16
    int num_pages;
    // Output format: O elements fp32 / fp16 / bf16 (kOut*); with `lse` the
    // Mi slot receives LSE = Mi + ln(Li) and Li is not written.
    int out_dtype;
    int lse;
    // XCDs of the device (8 on an MI355X in SPX mode, 1 per CPX partition):
    // the dispatcher deals workgroup ids round-robin over them.
    int xcds;
};

enum : int { kOutF32 = 0, kOutF16 = 1, kOutBF16 = 2 };
// Internal store target of the split prefill: fp32 partial O at p.Opart.
constexpr int kOutPartial = 3;

// fp32 -> bf16 bits, round to nearest even (inputs are finite).
__device__ __forceinline__ uint32_t bf16_rne_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Store the 4 consecutive output elements O[e .. e+3] as kOut (e is a
// multiple of 4; O is 16-byte aligned).
template <int kOut>
__device__ __forceinline__ void store_out4_as(const AttnParams& p, size_t e, const f32x4& v) {
    if constexpr (kOut == kOutF32) {
        *reinterpret_cast<f32x4*>(p.O + e) = v;
    } else if constexpr (kOut == kOutPartial) {
        *reinterpret_cast<f32x4*>(p.Opart + e) = v;
    } else if constexpr (kOut == kOutF16) {
        const f16x4 h = __builtin_convertvector(v, f16x4);
        *reinterpret_cast<f16x4*>(reinterpret_cast<f16*>(p.O) + e) = h;
    } else {
        u32x2 w;
        w.x = bf16_rne_bits(v[0]) | (bf16_rne_bits(v[1]) << 16);
        w.y = bf16_rne_bits(v[2]) | (bf16_rne_bits(v[3]) << 16);
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.O) + e) = w;
    }
}

// The same in p.out_dtype.
__device__ __forceinline__ void store_out4(const AttnParams& p, size_t e, const f32x4& v) {
    if (p.out_dtype == kOutF32)
        store_out4_as<kOutF32>(p, e, v);
    else if (p.out_dtype == kOutF16)
        store_out4_as<kOutF16>(p, e, v);
    else
        store_out4_as<kOutBF16>(p, e, v);
}

// Row `ri` of O from the O^T accumulator tiles of one lane (d = 32 td + 8 i +
// 4 g .. +3 in o[td][4 i .. 4 i + 3]), scaled by inv, as kOut.
template <int kOut, int D, int NTD>
__device__ __forceinline__ void store_o_row(const AttnParams& p, size_t ri, const f32x16 (&o)[NTD],
                                            float inv, int g) {
#pragma unroll
    for (int td = 0; td < NTD; ++td)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = 32 * td + 8 * i + 4 * g;
            if (d < D)
                store_out4_as<kOut>(p, ri * D + d, f32x4{o[td][4 * i] * inv, o[td][4 * i + 1] * inv,
                                                         o[td][4 * i + 2] * inv, o[td][4 * i + 3] * inv});
        }
}

// store_o_row in p.out_dtype, the format chosen once for the whole row.
template <int D, int NTD>
__device__ __forceinline__ void store_o_row_any(const AttnParams& p, size_t ri, const f32x16 (&o)[NTD],
                                                float inv, int g) {
    if (p.out_dtype == kOutF16)
        store_o_row<kOutF16, D>(p, ri, o, inv, g);
    else if (p.out_dtype == kOutBF16)
        store_o_row<kOutBF16, D>(p, ri, o, inv, g);
    else
        store_o_row<kOutF32, D>(p, ri, o, inv, g);
}

// Row statistics of query row r: Mi and Li, or LSE = Mi + ln(Li) (-inf for a
// row without keys) into the Mi slot.
__device__ __forceinline__ void store_stats(const AttnParams& p, size_t r, float mi, float li) {
    if (p.lse) {
        if (p.Mi) p.Mi[r] = li > 0.f ? mi + __logf(li) : -INFINITY;
    } else {
        if (p.Mi) p.Mi[r] = mi;
        if (p.Li) p.Li[r] = li;
    }
}

// Keys of the sequence that KV-head group `grp` belongs to, clamped to
// [0, kv_len].
__device__ __forceinline__ int batch_kv_len(const AttnParams& p, int grp) {
    if (!p.kv_lens) return p.kv_len;
    return min(max(p.kv_lens[grp / p.heads_kv], 0), p.kv_len);
}

// Number of leading keys visible to query index qi (0 <= qi < q_len) of a
// sequence with kvb keys.
__device__ __forceinline__ int row_kv_limit(const AttnParams& p, int kvb, int qi) {
    if (!p.causal) return kvb;
    return min(max(qi + kvb - p.q_len + 1, 0), kvb);
}

// Smallest and largest query index among group rows [r0, r1] (r0 <= r1);
// group row r holds query index r % q_len.
__device__ __forceinline__ void qi_range(int r0, int r1, int q_len, int& lo, int& hi) {
    if (r0 / q_len != r1 / q_len) {
        lo = 0;
        hi = q_len - 1;
    } else {
        lo = r0 % q_len;
        hi = r1 % q_len;
    }
}

// ---------------------------------------------------------------------------
// Small device helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x16 mfma32(const f16x8& a, const f16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// exp2(m - rmax scale_log2): the factor that rebases a row's running sums
// (kept relative to the exp2-domain offset m) to its true row max.  One
// explicit fused multiply-add, so every kernel instantiation rounds it the
// same way (left to contraction, the compiler fuses it in some and not in
// others, and masked and unmasked results would differ in the last bit).
__device__ __forceinline__ float rebase_factor(float m, float rmax, float scale_log2) {
    return exp2_hw(__builtin_fmaf(-rmax, scale_log2, m));
}

// Cross-lane reductions on the VALU (no LDS round trip, unlike ds_bpermute):
// v_permlane32_swap(x, x) yields the lower half's values in both halves and
// the upper half's values in both halves, v_permlane16_swap the same for the
// even and odd 16-lane rows, and DPP row_ror:n rotates each 16-lane row by n.
// Every lane receives the result; max and + are commutative, so the lanes of
// a pair compute bit-identical values.
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Reduce v over the lanes that agree with this one modulo CW (a power of two
// <= 64): the offsets CW, 2 CW, ..., 32.
template <int CW, bool kMax>
__device__ __forceinline__ float reduce_mod(float v) {
    static_assert(CW >= 1 && CW <= 64 && (CW & (CW - 1)) == 0, "power of two");
    auto op = [](float a, float b) { return kMax ? fmaxf(a, b) : a + b; };
    auto ror = [](float x, auto ctrl) {  // DPP row_ror:n has control 0x120 + n
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, false));
    };
    if constexpr (CW <= 1) v = op(v, ror(v, std::integral_constant<int, 0x121>{}));
    if constexpr (CW <= 2) v = op(v, ror(v, std::integral_constant<int, 0x122>{}));
    if constexpr (CW <= 4) v = op(v, ror(v, std::integral_constant<int, 0x124>{}));
    if constexpr (CW <= 8) v = op(v, ror(v, std::integral_constant<int, 0x128>{}));
    if constexpr (CW <= 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    if constexpr (CW <= 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    return v;
}

__device__ __forceinline__ f16x8 as_f16x8(const u32x4& v) { return __builtin_bit_cast(f16x8, v); }

// Hardware workgroup id -> logical id such that each XCD receives one
// contiguous range of logical ids (the dispatcher deals ids round-robin over
// the nx XCDs).  Logical neighbours share K/V, so each XCD's L2 holds them.
// A bijection on [0, n) for any nx >= 1 (nx = 1: the identity).
__device__ __forceinline__ int xcd_remap(int hw, int n, int nx) {
    const int q = n / nx, r = n % nx;
    const int xcd = hw % nx, k = hw / nx;
    return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + k;
}

// Order LDS traffic between the lanes of one wave (wave-private buffers).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// LDS stage geometry for a stage of BC kv rows at head dim D.
//   K stage:  [BC][D] fp16, 16-byte chunks XOR-swizzled by row so that the
//             32 lanes reading one chunk column of 32 rows (ds_read_b128)
//             hit distinct bank groups.
//   V^T stage: [DV][BC + 4] fp16 (d-major), padded by 4 halfs so the
//             ds_read_b64 of 32 consecutive d rows are conflict-free.
// ---------------------------------------------------------------------------
template <int D, int BC>
struct StageGeom {
    static constexpr int kChunks = D / 8;                           // 16-byte chunks per row
    static constexpr int kSwz = (kChunks < 16 ? kChunks : 16) - 1;  // K chunk XOR mask
    static constexpr int kDV = D < 32 ? 32 : D;                     // V^T rows, MFMA M >= 32
    static constexpr int kVtStride = BC + 4;                        // halfs per V^T row
    static constexpr int kKHalfs = BC * D;
    static constexpr int kVtHalfs = kDV * kVtStride;
    static constexpr int kStageHalfs = kKHalfs + kVtHalfs;
    static constexpr int kNSB = BC / 32;   // 32-row score blocks per stage
    static constexpr int kNKK = D / 16;    // MFMA k-steps over D
    static constexpr int kNTD = kDV / 32;  // 32-row O^T tiles
};

// Register-staged loader: NT threads copy one BC-row K/V stage from HBM into
// registers (load) and then into LDS (store), K row-major swizzled and V
// transposed.  Rows at or beyond kv_end hold row kv_end - 1 (load) or zeros
// (load_halves, whose pages may be unallocated), so masked scores meet
// finite V rows (0 * NaN would be NaN).  The loads are non-temporal: each
// K/V byte is read once per launch, and streamed past the caches the
// B = 32 x 8192-key decode reads HBM at 6.8 instead of 6.0 TB/s.
template <int D, int BC, int NT>
struct StageLoader {
    using G = StageGeom<D, BC>;
    static constexpr int kKTotal = BC * G::kChunks;          // 16-byte K chunks
    static constexpr int kKIters = (kKTotal + NT - 1) / NT;
    static constexpr int kVGroups = BC / 4;                   // 4-row V groups
    static constexpr int kVTotal = kVGroups * G::kChunks;     // (group, chunk) pairs
    static constexpr int kVIters = (kVTotal + NT - 1) / NT;

    u32x4 k[kKIters];
    u32x4 v[kVIters][4];

    // Unpredicated loads: rows at or beyond kv_end (kv0 < kv_end) read row
    // kv_end - 1 instead, a valid row whose scores the caller masks to -inf
    // (P = 0 times finite data), and lanes past the stage (idx beyond the
    // chunk count, D = 16 V only) read chunk 0 and are never stored.  A
    // predicated load compiles to a branch per load, and the compiler then
    // waited for the first loads before issuing the rest.
    __device__ __forceinline__ void load(const uint16_t* __restrict__ Kh,
                                         const uint16_t* __restrict__ Vh, int kv0, int kv_end,
                                         int tid) {
        const int last = kv_end - 1;
#pragma unroll
        for (int i = 0; i < kKIters; ++i) {
            const int idx = tid + i * NT;
            const int idc = ((kKTotal % NT == 0) || idx < kKTotal) ? idx : 0;
            const int row = idc / G::kChunks, c = idc % G::kChunks;
            const int kv = min(kv0 + row, last);
            k[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Kh + (size_t)kv * D + c * 8));
        }
#pragma unroll
        for (int i = 0; i < kVIters; ++i) {
            const int idx = tid + i * NT;
            const int idc = ((kVTotal % NT == 0) || idx < kVTotal) ? idx : 0;
            const int grp = idc % kVGroups, c = idc / kVGroups;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kv = min(kv0 + 4 * grp + r, last);
                v[i][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Vh + (size_t)kv * D + c * 8));
            }
        }
    }

    // The same for a stage whose rows 0..15 start at element offset off_lo
    // and rows 16..31 at off_hi (consecutive rows D elements apart within a
    // half): a stage of a paged K/V cache.  Rows >= nrows and halves whose
    // page is invalid (ok_* false) are zero-filled (their pool memory may
    // hold anything, and 0 * NaN would be NaN) and never read as keys.  The
    // half bases and flags are wave-uniform: the loads are unpredicated, an
    // invalid half reads the pool's first page (always in bounds), and the
    // rare stage with an invalid half or a short tail is zeroed afterwards
    // in one wave-uniform branch (predicating every load cost a 64-bit
    // address per load and spilled registers at D = 256).
    __device__ __forceinline__ void load_halves(const uint16_t* __restrict__ Kp,
                                                const uint16_t* __restrict__ Vp, size_t off_lo,
                                                size_t off_hi, bool ok_lo, bool ok_hi, int nrows,
                                                int tid) {
        static_assert(BC == 32, "two 16-row halves");
        const size_t blo = ok_lo ? off_lo : 0, bhi = ok_hi ? off_hi : 0;
#pragma unroll
        for (int i = 0; i < kKIters; ++i) {
            const int idx = tid + i * NT;
            const int idc = ((kKTotal % NT == 0) || idx < kKTotal) ? idx : 0;
            const int row = idc / G::kChunks, c = idc % G::kChunks;
            const size_t off = (row >= 16 ? bhi : blo) + (size_t)(row & 15) * D + c * 8;
            k[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Kp + off));
        }
        // V: lane tid always reads rows 4 (idx % kVGroups) + r, of one half
        // when NT is a multiple of kVGroups (it is: NT = 64, kVGroups = 8).
        static_assert(NT % kVGroups == 0, "V rows of a lane in one half");
        const uint16_t* vb = Vp + (4 * (tid % kVGroups) >= 16 ? bhi : blo);
#pragma unroll
        for (int i = 0; i < kVIters; ++i) {
            const int idx = tid + i * NT;
            const int idc = ((kVTotal % NT == 0) || idx < kVTotal) ? idx : 0;
            const int grp = idc % kVGroups, c = idc / kVGroups;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 4 * grp + r;
                v[i][r] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(vb + (size_t)(row & 15) * D + c * 8));
            }
        }
        if (!(ok_lo && ok_hi) || nrows < BC) {
#pragma unroll
            for (int i = 0; i < kKIters; ++i) {
                const int row = ((tid + i * NT) % kKTotal) / G::kChunks;
                if (!(row < nrows && (row >= 16 ? ok_hi : ok_lo))) k[i] = u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int i = 0; i < kVIters; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 4 * ((tid + i * NT) % kVGroups) + r;
                    if (!(row < nrows && (row >= 16 ? ok_hi : ok_lo))) v[i][r] = u32x4{0u, 0u, 0u, 0u};
                }
        }
    }

    __device__ __forceinline__ void store(f16* __restrict__ Ks, f16* __restrict__ Vt, int tid) const {
#pragma unroll
        for (int i = 0; i < kKIters; ++i) {
            const int idx = tid + i * NT;
            if ((kKTotal % NT == 0) || idx < kKTotal) {
                const int row = idx / G::kChunks, c = idx % G::kChunks;
                const int phys = c ^ (row & G::kSwz);
                *reinterpret_cast<u32x4*>(Ks + row * D + phys * 8) = k[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kVIters; ++i) {
            const int idx = tid + i * NT;
            if ((kVTotal % NT == 0) || idx < kVTotal) {
                const int grp = idx % kVGroups, c = idx / kVGroups;
                f16* dst = Vt + (8 * c) * G::kVtStride + 4 * grp;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    // Word w of each of the 4 rows holds d = 8c+2w (low half)
                    // and d = 8c+2w+1 (high half); gather them per d.
                    u32x2 lo, hi;
                    lo.x = __builtin_amdgcn_perm(v[i][1][w], v[i][0][w], 0x05040100u);
                    lo.y = __builtin_amdgcn_perm(v[i][3][w], v[i][2][w], 0x05040100u);
                    hi.x = __builtin_amdgcn_perm(v[i][1][w], v[i][0][w], 0x07060302u);
                    hi.y = __builtin_amdgcn_perm(v[i][3][w], v[i][2][w], 0x07060302u);
                    *reinterpret_cast<u32x2*>(dst + (2 * w) * G::kVtStride) = lo;
                    *reinterpret_cast<u32x2*>(dst + (2 * w + 1) * G::kVtStride) = hi;
                }
            }
        }
    }
};

// Q^T fragments of one wave: query row `row` of the group, chunk
// 2*kk + (lane/32) for MFMA k-step kk.  Lanes of rows >= R load row R - 1:
// their score columns are computed but never stored.
template <int D>
__device__ __forceinline__ void load_q_frags(const uint16_t* __restrict__ Qg, int row, int R,
                                             int lane, f16x8 (&qf)[D / 16]) {
    const int g = lane >> 5;
    const int rc = min(row, R - 1);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
        qf[kk] = *reinterpret_cast<const f16x8*>(Qg + (size_t)rc * D + (2 * kk + g) * 8);
}

// One 32(kv) x 32(query) block of raw scores S^T = K . Q^T.
template <int D, int BC>
__device__ __forceinline__ f32x16 qk_block(const f16* __restrict__ Ks, int row0,
                                           const f16x8 (&qf)[D / 16], int lane) {
    using G = StageGeom<D, BC>;
    const int row = row0 + (lane & 31);
    const int g = lane >> 5;
    const f16* base = Ks + row * D;
    f32x16 s = {};
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
        const int phys = (2 * kk + g) ^ (row & G::kSwz);
        const f16x8 a = *reinterpret_cast<const f16x8*>(base + phys * 8);
        s = mfma32(a, qf[kk], s);
    }
    return s;
}

// qk_block with the Q^T fragments read from an LDS copy of the 32 query rows
// (row r's chunk c at chunk c ^ (r & 15), D / 8 chunks per row).
template <int D, int BC>
__device__ __forceinline__ f32x16 qk_block_qlds(const f16* __restrict__ Ks, const char* q_lds,
                                                int lane) {
    using G = StageGeom<D, BC>;
    const int row = lane & 31;
    const int g = lane >> 5;
    const f16* base = Ks + row * D;
    const char* qrow = q_lds + row * D * 2;
    f32x16 s = {};
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
        const int phys = (2 * kk + g) ^ (row & G::kSwz);
        const f16x8 a = *reinterpret_cast<const f16x8*>(base + phys * 8);
        const f16x8 q = *reinterpret_cast<const f16x8*>(qrow + ((2 * kk + g) ^ (row & 15)) * 16);
        s = mfma32(a, q, s);
    }
    return s;
}

// kv offset (within its 32-row block) of accumulator register r on lane l.
__device__ __forceinline__ int acc_row(int r, int lane) {
    return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

// Per-lane online-softmax state for one query row (lane l and l^32 share
// a row and keep identical m / rmax; each keeps its own partial sum l).
struct RowState {
    float m;     // running max used for exponentiation, log2 units
    float rmax;  // true running max of the raw (unscaled) scores
    float l;     // this lane's partial sum of exp2(s*scale_log2 - m)
    float thr;   // raw score above which m must move: (m + kLazyRescaleLog2) / scale_log2
};

// Online-softmax update for NSB score blocks: moves the running max (lazily),
// rescales O, exponentiates, packs fp16 P^T operands (p[j] covers kv
// 16j .. 16j+15 of the stage) and accumulates the row sum of those fp16 P
// values with v_dot2_f32_f16 (fp32 accumulation, two terms per instruction).
// Summing the rounded P keeps numerator and denominator on the same weights;
// it differs from a sum of the fp32 P by at most 2^-12 relative.
template <int NSB, int NTD>
__device__ __forceinline__ void softmax_update(f32x16 (&s)[NSB], RowState& st,
                                               f32x16 (&o)[NTD], float scale_log2,
                                               f16x8 (&p)[2 * NSB]) {
    float mx = s[0][0];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sb][r]);
    mx = max_xor32(mx);
    st.rmax = fmaxf(st.rmax, mx);
    const float mt = mx * scale_log2;
    const bool need = mt > st.m + kLazyRescaleLog2;
    if (__any(need)) {
        // Lanes that keep their max scale by exactly 1 (also when it is still
        // -inf: exp2(-inf - -inf) would be NaN).
        const float mnew = need ? mt : st.m;
        const float alpha = need ? exp2_hw(st.m - mt) : 1.0f;
        st.l *= alpha;
#pragma unroll
        for (int td = 0; td < NTD; ++td) o[td] *= alpha;
        st.m = mnew;
    }
    // A row that has seen no key yet (all masked) keeps m = -inf: exponents
    // must then give P = 0, not NaN.
    const float neg_m = st.m == -INFINITY ? 0.f : -st.m;
    const f16x2 ones = {(f16)1.0f, (f16)1.0f};
    float sum[2] = {0.f, 0.f};
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f32x8 e;
#pragma unroll
            for (int r = 0; r < 8; ++r) e[r] = exp2_hw(fmaf(s[sb][8 * h + r], scale_log2, neg_m));
            const f16x8 ph = __builtin_convertvector(e, f16x8);
            p[2 * sb + h] = ph;
            sum[h] = __builtin_amdgcn_fdot2(__builtin_shufflevector(ph, ph, 0, 1), ones, sum[h], false);
            sum[h] = __builtin_amdgcn_fdot2(__builtin_shufflevector(ph, ph, 2, 3), ones, sum[h], false);
            sum[h] = __builtin_amdgcn_fdot2(__builtin_shufflevector(ph, ph, 4, 5), ones, sum[h], false);
            sum[h] = __builtin_amdgcn_fdot2(__builtin_shufflevector(ph, ph, 6, 7), ones, sum[h], false);
        }
    }
    st.l += sum[0] + sum[1];
}

// O^T += V^T . P^T over NJ 16-row kv steps of a V^T stage, starting at kv
// column kv0 of the stage.
template <int D, int BC, int NJ>
__device__ __forceinline__ void pv_accum(const f16* __restrict__ Vt, int kv0,
                                         const f16x8 (&p)[NJ],
                                         f32x16 (&o)[StageGeom<D, BC>::kNTD], int lane) {
    using G = StageGeom<D, BC>;
    const int g = lane >> 5;
    const int d0 = lane & 31;
#pragma unroll
    for (int td = 0; td < G::kNTD; ++td) {
        const f16* rowp = Vt + (32 * td + d0) * G::kVtStride + kv0 + 4 * g;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const f16x4 lo = *reinterpret_cast<const f16x4*>(rowp + 16 * j);
            const f16x4 hi = *reinterpret_cast<const f16x4*>(rowp + 16 * j + 8);
            const f16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            o[td] = mfma32(a, p[j], o[td]);
        }
    }
}

// ---------------------------------------------------------------------------
// Prefill: NW waves x 32 query rows per workgroup.  K and V
// stages are copied HBM -> LDS by the gfx950 LDS-DMA loads
// (global_load_lds_dwordx4: each wave instruction fills one contiguous KiB
// of LDS, no VGPR staging) into named LDS arrays, so the prefetch of later
// stages overlaps the MFMA/softmax work on the current one.  Both K and V
// stay row-major in LDS with the 16-byte chunks of a row XOR-permuted by
// SwizzleRow<D>: K fragments are read with ds_read_b128, and the V^T
// fragments of the P.V MFMA with the transposing ds_read_b64_tr_b16, so V is
// never transposed by VALU work.
// ---------------------------------------------------------------------------

// Row-dependent XOR applied to the 16-byte chunk index of a K / V row in LDS.
// It depends only on row & 15, is a bijection on those 16 rows, and was
// chosen (exhaustive search over GF(2)-linear maps) so that both access
// patterns are bank-conflict-free with 32 or with 64 four-byte banks:
//   ds_read_b128 of a 16-byte chunk column over 32 consecutive rows (K), and
//   ds_read_b64_tr_b16 of 4 consecutive rows x 32 bytes per 16 lanes (V).
template <int D> struct SwizzleRow;
template <> struct SwizzleRow<16> {
    static __device__ __forceinline__ int h(int row) { return row & 1; }
};
template <> struct SwizzleRow<64> {
    static __device__ __forceinline__ int h(int row) {
        const int r0 = row & 1, r1 = (row >> 1) & 1, r2 = (row >> 2) & 1, r3 = (row >> 3) & 1;
        return r1 | ((r0 ^ r2) << 1) | ((r0 ^ r1 ^ r3) << 2);
    }
};
template <> struct SwizzleRow<128> {
    static __device__ __forceinline__ int h(int row) { const int r = row & 15; return r ^ ((r & 3) << 2); }
};
template <> struct SwizzleRow<256> : SwizzleRow<128> {};

// Per head dimension: waves per workgroup (32 query rows each).  Every
// variant overlaps S(t+1) = K Q^T with the softmax of tile t (a second score
// block in registers).  D = 256 holds 128 fp32 O accumulators per lane, so it
// runs 4 waves (one per SIMD, up to 512 registers; it uses ~450).  Grids too
// small to give every CU a workgroup use fewer rows per workgroup: KS = 2 or
// 4 KV groups (each wave takes 1 / KS of the keys of its rows, the parts
// merged in LDS at the end) and then fewer waves (NW = 4, 2).
template <int D> constexpr int kPrefillMaxWaves = D >= 256 ? 4 : 8;

constexpr int gcd_int(int a, int b) { return b == 0 ? a : gcd_int(b, a % b); }

template <int D, int NW = kPrefillMaxWaves<D>, int KS = 1> struct PrefillCfg {
    static constexpr int BC = 32;                   // KV rows per MFMA tile
    static constexpr int kWaves = NW;
    static constexpr int kGroups = KS;              // KV groups per workgroup
    static constexpr int kRowWaves = NW / KS;       // waves per KV group
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kRows = 32 * kRowWaves;    // query rows per workgroup
    static_assert(NW % KS == 0 && (KS == 1 || KS == 2 || KS == 4) && (KS == 1 || D <= 128),
                  "KV groups: 1, 2 or 4, D <= 128");
    // Register budget: 256 per wave (two waves per SIMD) for D <= 128,
    // whatever the workgroup size, so every variant keeps its accumulators in
    // VGPRs; 512 for D = 256.
    static constexpr int kWavesPerEU = D >= 256 ? 1 : 2;
    // Tiles per LDS stage: 8-wave workgroups without KV groups hold two tiles
    // per stage, so the workgroup barrier and the LDS-DMA issue come once per
    // 64 kv rows.  The others keep one tile per stage, which holds the
    // compiler to the 256-register budget at D <= 128.  Stages t, t+1 and the
    // one being filled rotate through three stage buffers per KV group (48 KB
    // per group at D = 128), except where that does not fit: four KV groups
    // (192 KB), and two 4-wave groups, whose workgroups should share a CU two
    // at a time.  Those use two buffers per KV group whose K and V halves are
    // refilled separately: tile t reads K(t+1) from one buffer and V(t) from
    // the other, while K(t+2) lands in the first buffer's K half and V(t+1)
    // in the second's V half (32 KB per group at D = 128).  V then has one
    // tile of lead instead of two, which measured 2 % (two 8-wave groups) to
    // 6 % (D = 256) slower where the three buffers fit.
    static constexpr int kSub = (kWaves >= 8 && KS == 1) ? 2 : 1;
    static constexpr int kStageRows = BC * kSub;
    static constexpr int kBuffers = (KS == 4 || (KS == 2 && NW == 4)) ? 2 : 3;
};

inline int prefill_max_waves(int D) { return D >= 256 ? kPrefillMaxWaves<256> : kPrefillMaxWaves<128>; }

template <int D, int BC, int NW>
struct DmaStage {
    static constexpr int kRowBytes = D * 2;
    static constexpr int kChunks = D / 8;                        // 16-byte chunks per row
    static constexpr int kRowsPerInstr = 1024 / kRowBytes;       // rows per wave instruction
    static constexpr int kInstrPerTensor = BC * kRowBytes / 1024;
    static constexpr int kInstrTotal = 2 * kInstrPerTensor;      // K instructions, then V
    static constexpr int kPerWave = (kInstrTotal + NW - 1) / NW;
    static constexpr int kTensorBytes = BC * kRowBytes;
    static constexpr int kStageBytes = 2 * kTensorBytes;         // K region, then V region
    static_assert(kRowsPerInstr * kRowBytes == 1024, "row size must divide 1 KiB");
    static_assert(kInstrPerTensor >= 1, "a stage must fill whole KiB");
};

typedef __attribute__((address_space(3))) void lds_void;
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ f16x4 lds_read_tr16(const char* lds_byte_ptr) {
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4*)(const_cast<char*>(lds_byte_ptr)));
    return __builtin_bit_cast(f16x4, v);
}

// Row max of NSB 32-row score blocks, shared with the partner lane l^32.
template <int NSB>
__device__ __forceinline__ float block_rowmax(const f32x16 (&s)[NSB]) {
    float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
    for (int b = 0; b < NSB; ++b)
#pragma unroll
        for (int r = (b == 0 ? 2 : 0); r < 16; ++r) mx = fmaxf(mx, s[b][r]);
    return max_xor32(mx);
}

template <int NSB>
__device__ __forceinline__ void block_mask(f32x16 (&s)[NSB], int lim, int lane) {
#pragma unroll
    for (int b = 0; b < NSB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (32 * b + acc_row(r, lane) >= lim) s[b][r] = -INFINITY;
}

// exp2 + fp16 pack of one 32-row score block; adds its fp16 P values to the
// row sum `acc` (v_dot2_f32_f16, two terms per instruction, chained straight
// into the running sum: no partial sums to initialise and add).
__device__ __forceinline__ void block_exp(const f32x16& s, float scale_log2, float neg_m,
                                          f16x8& p0, f16x8& p1, float& acc) {
    f32x8 e0, e1;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        e0[r] = exp2_hw(fmaf(s[r], scale_log2, neg_m));
        e1[r] = exp2_hw(fmaf(s[8 + r], scale_log2, neg_m));
    }
    p0 = __builtin_convertvector(e0, f16x8);
    p1 = __builtin_convertvector(e1, f16x8);
    const f16x2 ones = {(f16)1.0f, (f16)1.0f};
    float a = acc;
    a = __builtin_amdgcn_fdot2(__builtin_shufflevector(p0, p0, 0, 1), ones, a, false);
    a = __builtin_amdgcn_fdot2(__builtin_shufflevector(p0, p0, 2, 3), ones, a, false);
    a = __builtin_amdgcn_fdot2(__builtin_shufflevector(p0, p0, 4, 5), ones, a, false);
    a = __builtin_amdgcn_fdot2(__builtin_shufflevector(p0, p0, 6, 7), ones, a, false);
    a = __builtin_amdgcn_fdot2(__builtin_shufflevector(p1, p1, 0, 1), ones, a, false);
    a = __builtin_amdgcn_fdot2(__builtin_shufflevector(p1, p1, 2, 3), ones, a, false);
    a = __builtin_amdgcn_fdot2(__builtin_shufflevector(p1, p1, 4, 5), ones, a, false);
    a = __builtin_amdgcn_fdot2(__builtin_shufflevector(p1, p1, 6, 7), ones, a, false);
    acc = a;
}

// Move the running max for a new block max (lazily) and rescale O and l.
// The test against the raw threshold st.thr is one compare per tile; the
// scaled max and the new threshold are computed only when some lane moves.
template <int NTD>
__device__ __forceinline__ void block_update_max(RowState& st, float mx, float scale_log2,
                                                 float inv_scale_log2, f32x16 (&o)[NTD]) {
    st.rmax = fmaxf(st.rmax, mx);
    const bool need = mx > st.thr;
    if (__any(need)) {
        // Lanes that keep their max scale by exactly 1 (also when it is still
        // -inf, a fully masked row: exp2(-inf - -inf) would be NaN).
        const float mt = mx * scale_log2;
        const float mnew = need ? mt : st.m;
        const float alpha = need ? exp2_hw(st.m - mt) : 1.0f;
        st.l *= alpha;
#pragma unroll
        for (int td = 0; td < NTD; ++td) o[td] *= alpha;
        st.m = mnew;
        st.thr = (mnew + kLazyRescaleLog2) * inv_scale_log2;
    }
}

// KV-group merge (KS > 1) of the prefill kernels, spread over the groups.
// Each group rebases its state to its true row max: O_g beta_g, m_g = rmax
// scale (natural log), l_g beta_g (both half rows); a group that saw no key
// of a row has weight 0.  A lane's O is kC float4 chunks (chunk cc holds
// d = 32 (cc / 4) + 8 (cc % 4) + 4 (l / 32) .. +3); group h owns chunks
// [h kCPer, (h+1) kCPer).  Every group publishes (m_g, l_g) in merge_ml and
// the chunks it does not own in lane-private 1 KiB slots (slot_base(k), in
// the then free stage buffers); after one barrier every group merges and
// stores its own chunks,
//   O = sum_g w_g O_g / L,  L = sum_g w_g l_g,  w_g = exp(m_g - max m),
// summing over g = 0 .. KS-1 in that order whatever the owner, so the result
// does not depend on which group stores a chunk.  With KV partitions
// (p.n_splits > 1) the merged state goes to the split partials at index pi
// instead (O unnormalised, m, L), for the split merge.  Opens with the
// barrier after which every group is done with its stage regions.
template <int D, int KS, int kRowWaves, class SlotBase>
__device__ __forceinline__ void merge_kv_groups(const AttnParams& p, const RowState& st,
                                                const f32x16 (&o)[D / 32], SlotBase slot_base,
                                                float* merge_ml, int wave, int kgrp, int lane, int g,
                                                size_t ri, size_t pi, bool row_ok) {
    constexpr int kC = D / 32 * 4;                      // float4 chunks per lane
    constexpr int kCPer = kC / KS;                      // chunks each group stores
    static_assert(kC % KS == 0, "chunks per group");
    // Slot of chunk cc of row wave w written by group gw (!= owner h).
    auto slot = [&](int cc, int gw, int h) {
        const int k = (wave * kC + cc) * (KS - 1) + (gw < h ? gw : gw - 1);
        return reinterpret_cast<f32x4*>(slot_base(k)) + lane;
    };
    auto chunk = [&](int cc) {
        const int td = cc / 4, i = cc % 4;
        return f32x4{o[td][4 * i], o[td][4 * i + 1], o[td][4 * i + 2], o[td][4 * i + 3]};
    };
    const float l_pair = sum_xor32(st.l);
    const bool none = st.rmax == -INFINITY;
    const float m_g = none ? -INFINITY : st.rmax * p.scale;
    const float beta = none ? 0.f : rebase_factor(st.m, st.rmax, p.scale_log2);
    __syncthreads();  // every group is done with its stage regions
    merge_ml[(kgrp * kRowWaves + wave) * 64 + lane] = m_g;
    merge_ml[((KS + kgrp) * kRowWaves + wave) * 64 + lane] = l_pair * beta;
#pragma unroll
    for (int cc = 0; cc < kC; ++cc) {
        const int h = cc / kCPer;
        if (h != kgrp) *slot(cc, kgrp, h) = chunk(cc) * beta;
    }
    __syncthreads();
    float m_all = -INFINITY;
#pragma unroll
    for (int gg = 0; gg < KS; ++gg) m_all = fmaxf(m_all, merge_ml[(gg * kRowWaves + wave) * 64 + lane]);
    float wgt[KS];
    float L = 0.f;
#pragma unroll
    for (int gg = 0; gg < KS; ++gg) {
        const float mo = merge_ml[(gg * kRowWaves + wave) * 64 + lane];
        wgt[gg] = mo == -INFINITY ? 0.f : exp2_hw((mo - m_all) * kLog2e);
        L += wgt[gg] * merge_ml[((KS + gg) * kRowWaves + wave) * 64 + lane];
    }
    const bool partial = p.n_splits > 1;
    const float inv = partial ? 1.0f : L > 0.f ? 1.0f / L : 0.f;
    const size_t oi = partial ? pi : ri;
    auto merge_store = [&](auto out) {
        constexpr int kOut = decltype(out)::value;
#pragma unroll
        for (int cc = 0; cc < kC; ++cc) {
            if (cc / kCPer != kgrp) continue;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int gg = 0; gg < KS; ++gg) {
                const f32x4 v = gg == kgrp ? chunk(cc) * beta : *slot(cc, gg, kgrp);
                acc = wgt[gg] * v + acc;
            }
            const int d = 32 * (cc / 4) + 8 * (cc % 4) + 4 * g;
            if (row_ok && d < D) store_out4_as<kOut>(p, oi * D + d, acc * inv);
        }
    };
    if (partial)
        merge_store(std::integral_constant<int, kOutPartial>{});
    else if (p.out_dtype == kOutF16)
        merge_store(std::integral_constant<int, kOutF16>{});
    else if (p.out_dtype == kOutBF16)
        merge_store(std::integral_constant<int, kOutBF16>{});
    else
        merge_store(std::integral_constant<int, kOutF32>{});
    if (kgrp == 0 && row_ok && g == 0) {
        if (partial) {
            p.Mpart[pi] = m_all;
            p.Lpart[pi] = L;
        } else {
            store_stats(p, ri, m_all, L);
        }
    }
}

// kMask: causal masking and/or per-sequence key counts (p.causal,
// p.kv_lens); without it every row sees keys [0, kv_len).
//
// KS > 1 (KV groups): wave w works on row wave w % (NW / KS) of the
// workgroup's rows and on KV group w / (NW / KS), i.e. on the tiles
// [g tpg, (g+1) tpg) of the keys the workgroup needs.  Every group streams its
// keys through its own region of each LDS stage buffer; all groups run the
// same number of tiles (tiles past a group's keys are masked), so the
// workgroup barriers line up.  At the end each group's (O, max, sum) is
// rebased to its true max and group 0 merges them through LDS.
// kParts: the KV-partition code (split prefill) is compiled in.  At D = 256
// it is a kernel of its own (kf_attn_prefill_parts_kernel), since its
// registers would push the unsplit 4-wave kernel's past the architectural
// VGPRs.
template <int D, bool kMask, int NW, int KS, bool kParts>
__device__ __forceinline__ void prefill_body(AttnParams p) {
    using Cfg = PrefillCfg<D, NW, KS>;
    constexpr int BC = Cfg::BC;
    constexpr int kNSB = BC / 32;                 // 32-row score blocks per stage
    constexpr int kRowWaves = Cfg::kRowWaves;     // waves per KV group
    constexpr int kPrefillRows = Cfg::kRows;
    constexpr int kSub = Cfg::kSub;               // tiles per LDS stage
    constexpr int SR = Cfg::kStageRows;           // kv rows per LDS stage
    using S = DmaStage<D, SR, kRowWaves>;
    using SW = SwizzleRow<D>;
    constexpr int kNKK = D / 16;                  // MFMA k-steps over D
    constexpr int kNTD = (D < 32 ? 32 : D) / 32;  // 32-row O^T tiles
    __shared__ __attribute__((aligned(1024))) char buf0[KS * S::kStageBytes];
    __shared__ __attribute__((aligned(1024))) char buf1[KS * S::kStageBytes];
    __shared__ __attribute__((aligned(1024))) char buf2[Cfg::kBuffers == 3 ? KS * S::kStageBytes : 16];
    __shared__ __attribute__((aligned(16))) char zero_pad[16];  // D=16: V^T rows 16..31
    // 8-wave workgroups with KV groups: the workgroup's query rows, copied
    // once into LDS (K's row layout) instead of KS times from memory.
    constexpr bool kQLds = KS > 1 && NW == 8;
    __shared__ __attribute__((aligned(1024))) char q_lds[kQLds ? Cfg::kRows * D * 2 : 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Row wave.  Causal, 8 waves: waves w and w+4 share a SIMD and get row
    // blocks w and 7 - w, so that the fully masked tiles each wave skips
    // (see nt_w) add up to the same count on every SIMD.
    const int wave = KS == 1 ? ((kMask && NW == 8 && p.causal && wave_id >= 4) ? 11 - wave_id : wave_id)
                             : wave_id % kRowWaves;
    const int kgrp = KS == 1 ? 0 : wave_id / kRowWaves;        // KV group
    const int g = lane >> 5;
    const int blk = xcd_remap(blockIdx.x, gridDim.x, p.xcds);
    // KV partitions (p.n_splits > 1, kParts): workgroup blk takes partition
    // blk % n_splits of its row tile's keys and writes split partials.
    constexpr bool kSplits = kParts;
    const int nsp = kSplits ? p.n_splits : 1;
    const bool split_out = kSplits && nsp > 1;
    const int split = blk % nsp;
    int rt = blk / nsp % p.row_tiles;
    const int grp = blk / nsp / p.row_tiles;
    const int R = p.rows_per_group;
    const int kv_len = p.kv_len;
    const float c = p.scale_log2;
    // Causal: a row tile's work grows with its position inside its head.
    // Each XCD receives its groups' row tiles longest first, so late, short
    // tiles fill the CUs that finish early: logical k -> position
    // T - 1 - k / heads of head k % heads, T = row tiles per head (when
    // tiles do not straddle heads; otherwise plain descending order).
    if (kMask && p.causal) {
        const int q_len = p.q_len;
        if (q_len % kPrefillRows == 0) {
            const int T = q_len / kPrefillRows, heads = R / q_len;
            rt = (rt % heads) * T + (T - 1 - rt / heads);
        } else {
            rt = p.row_tiles - 1 - rt;
        }
    }

    // Keys this workgroup needs (blk_lim) and, per wave, the smallest row
    // limit (below it no masking is needed) and the largest (from it on
    // every score of the wave is masked).
    int kvb = kv_len, blk_lim = kv_len, wave_min = kv_len, wave_max = kv_len;
    if constexpr (kMask) {
        kvb = batch_kv_len(p, grp);
        blk_lim = wave_min = wave_max = kvb;
        if (p.causal) {
            const int q_len = p.q_len;
            const int r0 = rt * kPrefillRows, r1 = min(R, r0 + kPrefillRows) - 1;
            int lo, hi;
            qi_range(r0, r1, q_len, lo, hi);
            blk_lim = row_kv_limit(p, kvb, hi);
            const int w0 = r0 + wave * 32;
            if (w0 < R) {
                qi_range(w0, min(R, w0 + 32) - 1, q_len, lo, hi);
                wave_min = row_kv_limit(p, kvb, lo);
                wave_max = row_kv_limit(p, kvb, hi);
            } else {
                wave_min = blk_lim;
                wave_max = 0;
            }
        }
    }
    // The workgroup's keys: [s0, blk_lim) (its partition of them when split).
    // KV group kgrp covers [kv_base, kv_end) of them in tiles 0 .. ntiles - 1
    // (the same count for every group); row limits below are relative to
    // kv_base.
    const int s0 = split * p.kv_per_split;
    if (split_out) blk_lim = min(blk_lim, s0 + p.kv_per_split);
    const int ntiles_wg = max(blk_lim - s0 + BC - 1, 0) / BC;
    const int ntiles = KS == 1 ? ntiles_wg : (ntiles_wg + KS - 1) / KS;  // 32-row tiles
    const int nstages = (ntiles * BC + SR - 1) / SR;                     // LDS stages
    const int kv_base = s0 + kgrp * ntiles * BC;
    const int kv_end = min(kv_base + ntiles * BC, blk_lim);
    if (KS > 1 || kSplits) {
        wave_min = min(wave_min, kv_end) - kv_base;
        wave_max = min(wave_max, kv_end) - kv_base;
    }
    // Tiles with a key visible to some row of this wave.  The later ones are
    // fully masked for it: their scores would contribute exactly nothing, so
    // the wave skips them and only takes part in the stage barriers and
    // copies (one KV group; with several, every group runs all its tiles).
    const int nt_w = (kMask && KS == 1) ? min(ntiles, max(wave_max + BC - 1, 0) / BC) : ntiles;
    char* const b0 = buf0 + kgrp * S::kStageBytes;  // this group's stage regions
    char* const b1 = buf1 + kgrp * S::kStageBytes;
    char* const b2 = Cfg::kBuffers == 3 ? buf2 + kgrp * S::kStageBytes : buf2;  // unused at 2

    const uint16_t* Qg = p.Q + (size_t)grp * R * D;
    const char* Kh = reinterpret_cast<const char*>(p.K + (size_t)grp * kv_len * D);
    const char* Vh = reinterpret_cast<const char*>(p.V + (size_t)grp * kv_len * D);

    // ---- LDS-DMA copy plan: this wave issues instructions j = wave + W i. ----
    // Lane l of instruction j writes LDS bytes [16 l, 16 l + 16) of KiB
    // ii = (j mod kInstrPerTensor) of the K (j < kInstrPerTensor) or V region,
    // i.e. row r = ii * kRowsPerInstr + l / kChunks, physical chunk
    // l % kChunks, which holds logical chunk (l % kChunks) ^ h(r) of kv row r.
    // lane_base[i % kLBPeriod]: byte offset of lane l's source chunk
    // relative to the first row of instruction i.  The swizzle depends on
    // row & 15 only, so instruction i repeats the offsets of instruction
    // i - kLBPeriod: kLaneBases distinct row phases, visited with stride W.
    constexpr int kLaneBases = S::kRowsPerInstr >= 16 ? 1 : 16 / S::kRowsPerInstr;
    constexpr int kLBPeriod = kLaneBases / gcd_int(kRowWaves, kLaneBases);
    uint32_t lane_base[kLBPeriod];
#pragma unroll
    for (int i = 0; i < kLBPeriod; ++i) {
        const int ii = (wave + kRowWaves * i) % S::kInstrPerTensor;
        const int lr = lane / S::kChunks;
        const int r = ii * S::kRowsPerInstr + lr;
        lane_base[i] = (uint32_t)(lr * S::kRowBytes +
                                  (((lane % S::kChunks) ^ SW::h(r)) % S::kChunks) * 16);
    }
    // Copy K rows [kv0k, kv0k + SR) into the K half of kdst (when do_k) and
    // V rows [kv0v, kv0v + SR) into the V half of vdst (when do_v); kv0k /
    // kv0v relative to this group's kv_base, kv0k >= kv0v when both are
    // copied.  The flags are wave-uniform.
    auto issue = [&](char* kdst, int kv0k_rel, bool do_k, char* vdst, int kv0v_rel, bool do_v) {
        const int kv0k = kv_base + kv0k_rel, kv0v = kv_base + kv0v_rel;
        if ((do_k ? kv0k : kv0v) + SR <= kv_len) {
            // Full stage: wave-uniform row base (SGPRs) + the lane's constant
            // 32-bit offset; no per-lane address arithmetic.
#pragma unroll
            for (int i = 0; i < S::kPerWave; ++i) {
                const int j = wave + kRowWaves * i;
                if (S::kInstrTotal % kRowWaves == 0 || j < S::kInstrTotal) {
                    const bool is_v = j >= S::kInstrPerTensor;
                    if (!(is_v ? do_v : do_k)) continue;
                    const int ii = j % S::kInstrPerTensor;
                    const int kv0 = is_v ? kv0v : kv0k;
                    const char* base = (is_v ? Vh : Kh) +
                                       (size_t)(kv0 + ii * S::kRowsPerInstr) * S::kRowBytes;
                    char* d = (is_v ? vdst + S::kTensorBytes : kdst) + ii * 1024;
                    // Keep the 32-bit lane offset opaque so the address stays
                    // "SGPR base + VGPR offset" instead of a hoisted 64-bit sum.
                    uint32_t lb = lane_base[i % kLBPeriod];
                    asm volatile("" : "+v"(lb));
                    __builtin_amdgcn_global_load_lds(base + lb, (lds_void*)d, 16, 0, 0);
                }
            }
        } else {
            // Last, partial stage: rows past kv_len re-read row kv_len - 1
            // (finite data whose scores are masked to -inf, so P = 0).
            asm volatile("" ::: "memory");
            const int lr = lane / S::kChunks;
#pragma unroll
            for (int i = 0; i < S::kPerWave; ++i) {
                const int j = wave + kRowWaves * i;
                if (S::kInstrTotal % kRowWaves == 0 || j < S::kInstrTotal) {
                    const bool is_v = j >= S::kInstrPerTensor;
                    if (!(is_v ? do_v : do_k)) continue;
                    const int ii = j % S::kInstrPerTensor;
                    const int kv = min((is_v ? kv0v : kv0k) + ii * S::kRowsPerInstr + lr, kv_len - 1);
                    const uint32_t off = (uint32_t)kv * S::kRowBytes +
                                         (lane_base[i % kLBPeriod] - (uint32_t)(lr * S::kRowBytes));
                    char* d = (is_v ? vdst + S::kTensorBytes : kdst) + ii * 1024;
                    __builtin_amdgcn_global_load_lds((is_v ? Vh : Kh) + off, (lds_void*)d, 16, 0, 0);
                }
            }
        }
    };
    auto issue_stage = [&](char* dst, int kv0_rel) { issue(dst, kv0_rel, true, dst, kv0_rel, true); };

    // ---- Per-lane LDS read offsets (bytes within a stage). ----
    // K (A of S^T = K Q^T): row l%32, logical chunk 2 kk + g.
    int koff[kNKK];
#pragma unroll
    for (int kk = 0; kk < kNKK; ++kk) {
        const int r = lane & 31;
        koff[kk] = r * S::kRowBytes + (((2 * kk + g) ^ SW::h(r)) % S::kChunks) * 16;
    }
    // V (A of O^T += V^T P^T) via ds_read_b64_tr_b16: 16-lane group G = l/16,
    // w = l%16 supplies row 4 (G/2) + w/4 (+8 for the second half of the
    // 16-row k step) and the 8 bytes at d = 32 td + 16 (G%2) + 4 (w%4).
    int voff[kNTD][2];
    {
        const int G = lane >> 4, w = lane & 15;
#pragma unroll
        for (int td = 0; td < kNTD; ++td)
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int r = 4 * (G >> 1) + (w >> 2) + 8 * h2;
                const int d = 32 * td + 16 * (G & 1) + 4 * (w & 3);
                if (d < D) {
                    const int cc = d >> 3, half = (d >> 2) & 1;
                    voff[td][h2] = S::kTensorBytes + r * S::kRowBytes +
                                   ((cc ^ SW::h(r)) % S::kChunks) * 16 + half * 8;
                } else {
                    voff[td][h2] = -1;  // D=16 padding rows of V^T: read zeros
                }
            }
    }

    auto qk = [&](const char* stage, const f16x8 (&qf)[kNKK], f32x16 (&s)[kNSB]) {
        // K fragments are fetched in batches: 8 (32 VGPRs) at D <= 128 under
        // the 256-register budget; all 16 of a tile at D = 256, whose one wave
        // per SIMD has the registers (measured 4 % faster than batches of 4).
        constexpr int kBatch = kNKK < 8 ? kNKK : (D >= 256 ? 16 : 8);
#pragma unroll
        for (int b = 0; b < kNSB; ++b) {
            s[b] = f32x16{};
#pragma unroll
            for (int k0 = 0; k0 < kNKK; k0 += kBatch) {
                f16x8 kf[kBatch];
#pragma unroll
                for (int kk = 0; kk < kBatch; ++kk)
                    kf[kk] = *reinterpret_cast<const f16x8*>(stage + koff[k0 + kk] +
                                                             b * 32 * S::kRowBytes);
#pragma unroll
                for (int kk = 0; kk < kBatch; ++kk) s[b] = mfma32(kf[kk], qf[k0 + kk], s[b]);
            }
        }
    };
    // p[j] holds P^T for kv rows 16 j .. 16 j + 15 of the stage.
    auto pv = [&](const char* stage, const f16x8 (&pp)[2 * kNSB], f32x16 (&o)[kNTD]) {
#pragma unroll
        for (int td = 0; td < kNTD; ++td)
#pragma unroll
            for (int jj = 0; jj < 2 * kNSB; ++jj) {
                f16x4 lo, hi;
                if (D < 32 && voff[td][0] < 0) {
                    lo = lds_read_tr16(zero_pad);
                    hi = lo;
                } else {
                    lo = lds_read_tr16(stage + voff[td][0] + jj * 16 * S::kRowBytes);
                    hi = lds_read_tr16(stage + voff[td][1] + jj * 16 * S::kRowBytes);
                }
                const f16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                o[td] = mfma32(a, pp[jj], o[td]);
            }
    };
    // Adds the tile's fp16 P values to the row sum `acc`.
    auto softmax_exp = [&](const f32x16 (&s)[kNSB], float neg_m, f16x8 (&pp)[2 * kNSB],
                           float& acc) {
#pragma unroll
        for (int b = 0; b < kNSB; ++b) block_exp(s[b], c, neg_m, pp[2 * b], pp[2 * b + 1], acc);
    };

    const int row = rt * kPrefillRows + wave * 32 + (lane & 31);
    if (kMask && ntiles == 0) {
        // No key for any row of this workgroup (whole-workgroup uniform):
        // O = 0, Mi = -inf, Li = 0, or that partial (a partition the rows
        // do not reach; the merge gives it weight 0 but reads it).
        if (row < R && kgrp == 0) {
            const size_t ri = (size_t)grp * R + row;
            const size_t pi = ((size_t)grp * nsp + split) * R + row;
#pragma unroll
            for (int td = 0; td < kNTD; ++td)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int d = 32 * td + 8 * i + 4 * g;
                    if (d >= D) continue;
                    if (split_out)
                        *reinterpret_cast<f32x4*>(p.Opart + pi * D + d) = f32x4{0.f, 0.f, 0.f, 0.f};
                    else
                        store_out4(p, ri * D + d, f32x4{0.f, 0.f, 0.f, 0.f});
                }
            if (g == 0) {
                if (split_out) {
                    p.Mpart[pi] = -INFINITY;
                    p.Lpart[pi] = 0.f;
                } else {
                    store_stats(p, ri, -INFINITY, 0.f);
                }
            }
        }
        return;
    }
    // This lane's query row sees keys [0, lim_lane) (padding rows: blk_lim).
    int lim_lane = kv_len;
    if constexpr (kMask) lim_lane = row < R ? row_kv_limit(p, kvb, row % p.q_len) : blk_lim;
    if (KS > 1 || kSplits) lim_lane = min(lim_lane, kv_end) - kv_base;

    // ---- Prologue: stage 0 and the K of stage 1 (two-buffer ring) or all of
    // stage 1 (three buffers) in flight, Q fragments, S(0). ----
    issue_stage(b0, 0);
    if (nstages > 1) issue(b1, SR, true, b1, SR, Cfg::kBuffers == 3);
    f16x8 qf[kNKK];
    if constexpr (kQLds) {
        // LDS-DMA of rows [rt kPrefillRows, + kPrefillRows) of the group (rows
        // past R re-read row R - 1, as load_q_frags does); lane l of KiB j
        // fills row 4 j + l / kChunks (D = 128) at physical chunk l % kChunks.
        constexpr int kQInstr = kPrefillRows * S::kRowBytes / 1024;
        const char* Qb = reinterpret_cast<const char*>(Qg);
        const int lr = lane / S::kChunks;
#pragma unroll
        for (int j0 = 0; j0 < kQInstr; j0 += NW) {
            const int j = j0 + wave_id;
            if (kQInstr % NW == 0 || j < kQInstr) {
                const int r = j * S::kRowsPerInstr + lr;
                const int src = min(rt * kPrefillRows + r, R - 1);
                const uint32_t off = (uint32_t)src * S::kRowBytes +
                                     (uint32_t)((((lane % S::kChunks) ^ SW::h(r)) % S::kChunks) * 16);
                __builtin_amdgcn_global_load_lds(Qb + off, (lds_void*)(q_lds + j * 1024), 16, 0, 0);
            }
        }
    } else {
        load_q_frags<D>(Qg, row, R, lane, qf);
    }
    if constexpr (D < 32) {
        if (tid < 4) reinterpret_cast<uint32_t*>(zero_pad)[tid] = 0u;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if constexpr (kQLds) {
        // Row wave w's 32 rows start at LDS row 32 w; koff addresses row l % 32.
#pragma unroll
        for (int kk = 0; kk < kNKK; ++kk)
            qf[kk] = *reinterpret_cast<const f16x8*>(q_lds + wave * 32 * S::kRowBytes + koff[kk]);
    }

    RowState st{-INFINITY, -INFINITY, 0.f, -INFINITY};
    const float inv_c = 1.0f / c;
    f32x16 o[kNTD];
#pragma unroll
    for (int td = 0; td < kNTD; ++td) o[td] = f32x16{};
    f32x16 sc[kNSB];
    qk(b0, qf, sc);
    if (BC > wave_min) block_mask<kNSB>(sc, lim_lane, lane);
    block_update_max<kNTD>(st, block_rowmax<kNSB>(sc), c, inv_c, o);
    // Exponent offset; a row with no key yet (masked) keeps m = -inf and
    // must get P = 0, not NaN.
    auto neg_m = [&]() { return ((kMask || KS > 1) && st.m == -INFINITY) ? 0.f : -st.m; };

    // ---- One pipelined tile; S(t) and its running max are ready on entry.
    //   barrier; LDS-DMA of the next stage(s)
    //   S(t+1) = K(t+1) Q^T   | exp + fp16 pack of S(t)
    //   O += V(t) P(t)        | row max of S(t+1)
    //   rare: tail masking of S(t+1); lazy rescale of O
    // cur holds V(t), nxt holds K(t+1).  On the last tile the S(t+1) MFMAs
    // read a stale, in-bounds buffer and are discarded, which keeps the
    // overlapped regions free of branches (issue is in order: a wave can only
    // overlap MFMA and VALU work that is interleaved in its own stream).
    auto tile = [&](char* cur, char* nxt, char* fill, int t, bool sync) {
        f16x8 pp[2 * kNSB];
        if (sync) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if constexpr (Cfg::kBuffers == 2) {
                // One tile per stage, two buffers: K(t+1) and V(t) landed for
                // every wave; tile t-1 read K(t) from cur and V(t-1) from nxt,
                // so K(t+2) goes to cur's K half and V(t+1) to nxt's V half.
                const bool dk = t + 2 < nstages, dv = t + 1 < nstages;
                if (dk || dv) issue(cur, (t + 2) * SR, dk, nxt, (t + 1) * SR, dv);
            } else {
                // Three buffers: tile t is the last of its stage j = t / kSub,
                // tile t+1 the first of stage j+1, which has landed for every
                // wave; stage j-1 (last read by tile t-1) is free for j+2.
                const int js = t / kSub + 2;
                if (js < nstages) issue_stage(fill, js * SR);
            }
        }
        if (t >= nt_w) return;  // wave-uniform; never for the unmasked kernel
        f32x16 sn[kNSB];
        qk(nxt, qf, sn);
        softmax_exp(sc, neg_m(), pp, st.l);
        pv(cur, pp, o);
        float mx = block_rowmax<kNSB>(sn);
        if (t + 1 < nt_w) {
            if ((t + 2) * BC > wave_min) {  // S(t+1) needs masking (tail / causal)
                // Keep this a branch: if-converted, the compares and selects
                // of the mask would run on every tile.
                asm volatile("" ::: "memory");
                block_mask<kNSB>(sn, lim_lane - (t + 1) * BC, lane);
                mx = block_rowmax<kNSB>(sn);
            }
            block_update_max<kNTD>(st, mx, c, inv_c, o);
#pragma unroll
            for (int b = 0; b < kNSB; ++b) sc[b] = sn[b];
        }
    };
    if constexpr (kSub == 1 && Cfg::kBuffers == 2) {
        // Tile t reads V(t) from buffer t % 2 and K(t+1) from buffer (t+1) % 2.
        for (int t = 0; t < ntiles; t += 2) {
            tile(b0, b1, nullptr, t, true);
            if (t + 1 >= ntiles) break;
            tile(b1, b0, nullptr, t + 1, true);
        }
    } else if constexpr (kSub == 1) {
        // Stage t lives in buffer t % 3.
        for (int t = 0; t < ntiles; t += 3) {
            tile(b0, b1, b2, t, true);
            if (t + 1 >= ntiles) break;
            tile(b1, b2, b0, t + 1, true);
            if (t + 2 >= ntiles) break;
            tile(b2, b0, b1, t + 2, true);
        }
    } else {
        static_assert(kSub == 2, "stages hold one or two tiles");
        // Tile t reads the (t % 2)-th half of stage t / 2, which lives in
        // buffer (t / 2) % 3; the loop body covers 3 stages.
        constexpr int H = BC * S::kRowBytes;
        for (int t = 0; t < ntiles; t += 6) {
            tile(b0, b0 + H, nullptr, t, false);
            if (t + 1 >= ntiles) break;
            tile(b0 + H, b1, b2, t + 1, true);
            if (t + 2 >= ntiles) break;
            tile(b1, b1 + H, nullptr, t + 2, false);
            if (t + 3 >= ntiles) break;
            tile(b1 + H, b2, b0, t + 3, true);
            if (t + 4 >= ntiles) break;
            tile(b2, b2 + H, nullptr, t + 4, false);
            if (t + 5 >= ntiles) break;
            tile(b2 + H, b0, b1, t + 5, true);
        }
    }

    if constexpr (KS > 1) {
        static_assert(kRowWaves * kNTD * 4 * (KS - 1) <= Cfg::kBuffers * KS * S::kStageBytes / 1024,
                      "merge slots");
        // Merge slot k: 1 KiB at k % per-buffer in stage buffer k / per-buffer.
        constexpr int kSlotsPerBuf = KS * S::kStageBytes / 1024;
        auto slot_base = [&](int k) {
            char* bb = k / kSlotsPerBuf == 0 ? buf0 : (k / kSlotsPerBuf == 1 ? buf1 : buf2);
            return bb + (k % kSlotsPerBuf) * 1024;
        };
        __shared__ float merge_ml[2 * KS * kRowWaves * 64];
        merge_kv_groups<D, KS, kRowWaves>(p, st, o, slot_base, merge_ml, wave, kgrp, lane, g,
                                          (size_t)grp * R + row,
                                          ((size_t)grp * nsp + split) * R + row, row < R);
        return;
    }

    // ---- Epilogue: combine the two half-row partial sums, normalise, store. ----
    const float l = sum_xor32(st.l);
    if (split_out) {
        // KV partition: the split partial, rebased to the true row max
        // (O beta, l beta, m = rmax scale; a row without keys here: 0, 0, -inf).
        const bool none = st.rmax == -INFINITY;
        const float beta = none ? 0.f : rebase_factor(st.m, st.rmax, p.scale_log2);
        if (row < R) {
            const size_t pi = ((size_t)grp * nsp + split) * R + row;
            store_o_row<kOutPartial, D>(p, pi, o, beta, g);
            if (g == 0) {
                p.Mpart[pi] = none ? -INFINITY : st.rmax * p.scale;
                p.Lpart[pi] = l * beta;
            }
        }
        return;
    }
    const bool empty = kMask && !(l > 0.f);  // no visible key
    if (row < R) {
        const float inv = empty ? 0.f : 1.0f / l;
        const size_t ri = (size_t)grp * R + row;
        store_o_row_any<D>(p, ri, o, inv, g);
        if (g == 0)
            store_stats(p, ri, st.rmax * p.scale,
                        empty ? 0.f : l * rebase_factor(st.m, st.rmax, p.scale_log2));
    }
}

template <int D, bool kMask, int NW = kPrefillMaxWaves<D>, int KS = 1>
__global__ __launch_bounds__((PrefillCfg<D, NW, KS>::kThreads), (PrefillCfg<D, NW, KS>::kWavesPerEU))
void kf_attn_prefill_kernel(AttnParams p) {
    prefill_body<D, kMask, NW, KS, (D <= 128)>(p);
}

// The split prefill at D = 256: the 4-wave kernel with KV partitions.
template <int D, bool kMask>
__global__ __launch_bounds__((PrefillCfg<D, 4, 1>::kThreads), (PrefillCfg<D, 4, 1>::kWavesPerEU))
void kf_attn_prefill_parts_kernel(AttnParams p) {
    static_assert(D == 256, "D <= 128 compiles the partitions into kf_attn_prefill_kernel");
    prefill_body<D, kMask, 4, 1, true>(p);
}

// ---------------------------------------------------------------------------
// Wide prefill: 8 waves x 64 query rows (two 32-row blocks per wave) = 512
// rows per workgroup at D = 64 / 128, 8 waves x 32 rows at D = 256 (two waves
// per SIMD where kf_attn_prefill_kernel runs one: 487 vs 689 us at S = 4096,
// 32 / 8 heads, bit-identical); unmasked (keys past kv_len in the last tile
// are masked).  Each K fragment read from LDS feeds the S^T MFMAs of
// both row blocks and each V^T fragment the O^T MFMAs of both, so LDS reads,
// LDS-DMA bytes and workgroup barriers per MFMA are half those of the
// 32-row kf_attn_prefill_kernel (measured at S = 4096, 32 / 8 heads: 6 %
// faster, bit-identical output).  At D = 128 the second row block's Q^T
// fragments are read from an LDS copy of those rows (in K's row layout) at
// every tile: held in registers they push the wave past its 256-register
// budget (two waves per SIMD) and spill.  Per tile, in one wave: S^T of both
// blocks (two interleaved MFMA chains sharing each K fragment), the row max /
// lazy rescale / exp2 / fp16 pack of each block, then O^T += V^T P^T for
// both.  K/V stages of 64 rows rotate through two LDS buffers: at the barrier
// that starts stage j every wave is done with stage j-1, whose buffer then
// receives stage j+1 (one stage of lead).
// ---------------------------------------------------------------------------
template <int D> struct WideCfg {
    static constexpr int kWaves = 8;
    static constexpr int kThreads = 64 * kWaves;
    // 32-row blocks per wave: two at D <= 128; one at D = 256, whose 128 fp32
    // O accumulators per block leave no room for a second.
    static constexpr int kRB = D >= 256 ? 1 : 2;
    static constexpr int kRows = 32 * kRB * kWaves;             // query rows per workgroup
    static constexpr int BC = 32;                               // kv rows per MFMA tile
    static constexpr int kStageRows = D >= 256 ? 32 : 64;       // kv rows per LDS stage
    static constexpr bool kQ1Lds = D == 128;                    // block-1 Q^T read from LDS
    // S(t+1) overlapped with the softmax of tile t (a second score block per
    // row block) where the registers allow it: D = 64.
    static constexpr bool kPipe = D <= 64;
    // D = 256: the per-lane LDS read offsets (16 for K, 16 for V) are derived
    // at each tile from one base each by XOR, not held in 32 registers.
    static constexpr bool kXorOff = D >= 256;
};

// kMask: causal masking and/or per-sequence key counts, as in
// kf_attn_prefill_kernel.  With one row block per wave (D = 256) causal
// masking is part of the masked kernel.  With two (D = 64 / 128) the masked
// kernel serves key counts, which give every row of a sequence one limit, and
// causal calls run kCausal2: each wave on 64 consecutive rows (block 1 =
// block 0 + 32 rows instead of the same rows in the second half of the
// workgroup), so that its blocks' key limits differ by one tile, each block
// masked against its own limits; a row of kCausal2 keeps its block limit
// unclamped (one register), which needs a wave's 64 rows inside one head.  At
// D = 128 kCausal2 derives its K and V^T read offsets by XOR: the registers
// that frees keep its tile loop from spilling.  kCausal2 = false leaves the
// other instantiations instruction for instruction as they compile without it.
// KS > 1 (D = 256): KV groups as in kf_attn_prefill_kernel — the waves form
// KS groups of NW / KS, each on the same rows and its own share of the keys,
// merged through LDS at the end; for grids too small for 256-row tiles.
// (The body sits in the kernel itself: moved into a shared device function,
// the unmasked kernel compiled to a different, 0.5 % slower schedule.)
template <int D, bool kMask, int KS, bool kCausal2 = false>
__global__ __launch_bounds__(WideCfg<D>::kThreads, 2)
void kf_attn_prefill_wide_kernel(AttnParams p) {
    static_assert(D == 64 || D == 128 || D == 256, "wide prefill: D = 64, 128 or 256");
    using Cfg = WideCfg<D>;
    constexpr int NW = Cfg::kWaves;
    constexpr int BC = Cfg::BC;
    constexpr int SR = Cfg::kStageRows;
    constexpr bool kQ1Lds = Cfg::kQ1Lds;
    constexpr bool kPipe = Cfg::kPipe;
    constexpr int kRB = Cfg::kRB;
    constexpr bool kXorOff = Cfg::kXorOff || (kCausal2 && D == 128);
    static_assert(KS == 1 || (KS == 2 && kRB == 1 && !kPipe && SR == BC), "KV groups: D = 256, two groups");
    static_assert(!kCausal2 || (kMask && kRB == 2 && KS == 1), "causal two-block layout");
    constexpr int kRowWaves = NW / KS;                 // waves per KV group
    constexpr int kRows = 32 * kRB * kRowWaves;        // query rows per workgroup
    using S = DmaStage<D, SR, kRowWaves>;
    using SW = SwizzleRow<D>;
    constexpr int kNKK = D / 16;
    constexpr int kNTD = D / 32;
    constexpr int kHalfRows = kRows / 2;           // rows of one row block, all waves
    // KS > 1: buf0 holds group g's two stage regions at 2 g and 2 g + 1
    // (the offset between them fits the LDS reads' immediate) and, after
    // the loop, the merge slots.
    __shared__ __attribute__((aligned(1024))) char buf0[(KS == 1 ? 1 : 2 * KS) * S::kStageBytes];
    __shared__ __attribute__((aligned(1024))) char buf1[KS == 1 ? S::kStageBytes : 16];
    __shared__ __attribute__((aligned(1024))) char buf2[kPipe ? S::kStageBytes : 16];
    // The stage buffers come first (the backend orders LDS variables by
    // alignment), so their addresses fit the 16-bit immediate offset of the
    // LDS reads and no K / V read needs address arithmetic (measured +1.6 %).
    __shared__ __attribute__((aligned(256))) char q1_lds[kQ1Lds ? kHalfRows * D * 2 : 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Row wave.  Causal: waves w and w + 4 share a SIMD and get row blocks w
    // and 7 - w, so that the fully masked tiles each wave skips add up to the
    // same count on every SIMD.
    // Causal masking: one row block per wave, or the two-block layout of
    // kCausal2 (compiled out of the other two-block kernels).
    const bool causal = kMask && (kRB == 1 || kCausal2) && p.causal;
    // Rows of one wave: 32 (one block), or 64 consecutive ones when causal
    // with two blocks; b1_off: the offset of block 1 from block 0.
    const int wave_rows = (kRB == 2 && causal) ? 64 : 32;
    const int b1_off = (kRB == 2 && causal) ? 32 : kRows / 2;
    const int wave = KS == 1 ? ((causal && wave_id >= 4) ? 11 - wave_id : wave_id) : wave_id % kRowWaves;
    const int kgrp = KS == 1 ? 0 : wave_id / kRowWaves;  // KV group
    const int g = lane >> 5;
    const int blk = xcd_remap(blockIdx.x, gridDim.x, p.xcds);
    int rt = blk % p.row_tiles;
    const int grp = blk / p.row_tiles;
    const int R = p.rows_per_group;
    const int kv_len = p.kv_len;
    const float c = p.scale_log2;
    // Causal: row tiles longest first on every XCD (as kf_attn_prefill_kernel).
    if (causal) {
        const int q_len = p.q_len;
        if (q_len % kRows == 0) {
            const int T = q_len / kRows, heads = R / q_len;
            rt = (rt % heads) * T + (T - 1 - rt / heads);
        } else {
            rt = p.row_tiles - 1 - rt;
        }
    }
    // Keys this workgroup needs (blk_lim) and, per wave, the smallest row
    // limit (below it no masking is needed) and the largest (from it on
    // every score of the wave is masked).
    int kvb = kv_len, blk_lim = kv_len, wave_min = kv_len, wave_max = kv_len;
    if constexpr (kMask) {
        kvb = batch_kv_len(p, grp);
        blk_lim = wave_min = wave_max = kvb;
        if (causal) {
            const int q_len = p.q_len;
            const int r0 = rt * kRows, r1 = min(R, r0 + kRows) - 1;
            int lo, hi;
            qi_range(r0, r1, q_len, lo, hi);
            blk_lim = row_kv_limit(p, kvb, hi);
            const int w0 = r0 + wave * wave_rows;
            if (w0 < R) {
                qi_range(w0, min(R, w0 + wave_rows) - 1, q_len, lo, hi);
                wave_min = row_kv_limit(p, kvb, lo);
                wave_max = row_kv_limit(p, kvb, hi);
            } else {
                wave_min = blk_lim;
                wave_max = 0;
            }
        }
    }
    // KV group kgrp covers the keys [kv_base, kv_end) of the workgroup's
    // range in tiles 0 .. ntiles - 1 (the same count for every group, so the
    // barriers line up); row limits below are relative to kv_base.
    const int ntiles_wg = (blk_lim + BC - 1) / BC;
    const int ntiles = KS == 1 ? ntiles_wg : (ntiles_wg + KS - 1) / KS;
    const int nstages = KS == 1 ? (blk_lim + SR - 1) / SR : (ntiles * BC + SR - 1) / SR;
    const int kv_base = kgrp * ntiles * BC;
    const int kv_end = min(kv_base + ntiles * BC, blk_lim);
    if constexpr (KS > 1) wave_min = min(wave_min, kv_end) - kv_base;
    // Tiles with a key visible to some row of this wave; the later ones are
    // skipped (their scores would add exactly nothing), the wave still
    // taking part in the stage barriers and copies.
    const int wmax = KS == 1 ? wave_max : min(wave_max, kv_end) - kv_base;
    const int nt_w = kMask ? min(ntiles, (wmax + BC - 1) / BC) : ntiles;
    char* const b0 = KS == 1 ? buf0 : buf0 + 2 * kgrp * S::kStageBytes;  // this group's stages
    char* const b1 = KS == 1 ? buf1 : b0 + S::kStageBytes;

    const uint16_t* Qg = p.Q + (size_t)grp * R * D;
    const char* Kh = reinterpret_cast<const char*>(p.K + (size_t)grp * kv_len * D);
    const char* Vh = reinterpret_cast<const char*>(p.V + (size_t)grp * kv_len * D);

    // LDS-DMA plan as in kf_attn_prefill_kernel: wave w of a group issues
    // the KiB instructions j = w + kRowWaves i of the group's stage (K
    // region, then V region).
    constexpr int kLaneBases = S::kRowsPerInstr >= 16 ? 1 : 16 / S::kRowsPerInstr;
    constexpr int kLBPeriod = kLaneBases / gcd_int(kRowWaves, kLaneBases);
    uint32_t lane_base[kLBPeriod];
#pragma unroll
    for (int i = 0; i < kLBPeriod; ++i) {
        const int ii = (wave + kRowWaves * i) % S::kInstrPerTensor;
        const int lr = lane / S::kChunks;
        const int r = ii * S::kRowsPerInstr + lr;
        lane_base[i] = (uint32_t)(lr * S::kRowBytes +
                                  (((lane % S::kChunks) ^ SW::h(r)) % S::kChunks) * 16);
    }
    auto issue_stage = [&](char* dst, int kv0_rel) {
        const int kv0 = kv_base + kv0_rel;
        if (kv0 + SR <= kv_len) {
#pragma unroll
            for (int i = 0; i < S::kPerWave; ++i) {
                const int j = wave + kRowWaves * i;
                if (S::kInstrTotal % kRowWaves == 0 || j < S::kInstrTotal) {
                    const bool is_v = j >= S::kInstrPerTensor;
                    const int ii = j % S::kInstrPerTensor;
                    const char* base = (is_v ? Vh : Kh) + (size_t)(kv0 + ii * S::kRowsPerInstr) * S::kRowBytes;
                    char* d = dst + (is_v ? S::kTensorBytes : 0) + ii * 1024;
                    uint32_t lb = lane_base[i % kLBPeriod];
                    asm volatile("" : "+v"(lb));
                    __builtin_amdgcn_global_load_lds(base + lb, (lds_void*)d, 16, 0, 0);
                }
            }
        } else {
            // Last, partial stage: rows past kv_len re-read row kv_len - 1
            // (finite data whose scores are masked to -inf, so P = 0).
            asm volatile("" ::: "memory");
            const int lr = lane / S::kChunks;
#pragma unroll
            for (int i = 0; i < S::kPerWave; ++i) {
                const int j = wave + kRowWaves * i;
                if (S::kInstrTotal % kRowWaves == 0 || j < S::kInstrTotal) {
                    const bool is_v = j >= S::kInstrPerTensor;
                    const int ii = j % S::kInstrPerTensor;
                    const int kv = min(kv0 + ii * S::kRowsPerInstr + lr, kv_len - 1);
                    const uint32_t off = (uint32_t)kv * S::kRowBytes +
                                         (lane_base[i % kLBPeriod] - (uint32_t)(lr * S::kRowBytes));
                    char* d = dst + (is_v ? S::kTensorBytes : 0) + ii * 1024;
                    __builtin_amdgcn_global_load_lds((is_v ? Vh : Kh) + off, (lds_void*)d, 16, 0, 0);
                }
            }
        }
    };

    // Per-lane LDS read offsets (bytes within a stage), as in
    // kf_attn_prefill_kernel: K row l%32, logical chunk 2 kk + g; V^T via
    // ds_read_b64_tr_b16.
    int koff[kNKK];
#pragma unroll
    for (int kk = 0; kk < kNKK; ++kk) {
        const int r = lane & 31;
        koff[kk] = r * S::kRowBytes + (((2 * kk + g) ^ SW::h(r)) % S::kChunks) * 16;
    }
    int voff[kNTD][2];
    {
        const int G = lane >> 4, w = lane & 15;
#pragma unroll
        for (int td = 0; td < kNTD; ++td)
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int r = 4 * (G >> 1) + (w >> 2) + 8 * h2;
                const int d = 32 * td + 16 * (G & 1) + 4 * (w & 3);
                const int cc = d >> 3, half = (d >> 2) & 1;
                voff[td][h2] = S::kTensorBytes + r * S::kRowBytes +
                               ((cc ^ SW::h(r)) % S::kChunks) * 16 + half * 8;
            }
    }

    // kXorOff: with phys chunk (2 kk + g) ^ h(r) = 2 kk ^ (g ^ h(r)), the K
    // offset of k-step kk is koff[0] ^ 32 kk; the V^T offsets are voff[0][0]
    // ^ 64 td for the first 8 rows and, since h(r + 8) = h(r) ^ 8 (D = 128 /
    // 256 swizzle), that ^ 128, plus 8 rows, for the second.
    static_assert(!kXorOff || D >= 128, "XOR offsets use the D >= 128 swizzle");
    const int kbase = koff[0], vbase = voff[0][0];

    // Row blocks: block 0 = rows [rt kRows + wave_rows w, + 32), block 1 =
    // block 0 + b1_off (the same rows in the second half of the workgroup's
    // rows, or, causal, the next 32).  Rows past R compute on row R - 1 and
    // are never stored.
    const int row0 = rt * kRows + wave * wave_rows + (lane & 31);
    const int row1 = row0 + b1_off;
    if (kMask && ntiles == 0) {
        // No key for any row of this workgroup (workgroup-uniform).
#pragma unroll
        for (int b = 0; b < kRB; ++b) {
            const int row = b == 0 ? row0 : row1;
            if (row < R && kgrp == 0) {
                const size_t ri = (size_t)grp * R + row;
#pragma unroll
                for (int td = 0; td < kNTD; ++td)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        store_out4(p, ri * D + 32 * td + 8 * i + 4 * g, f32x4{0.f, 0.f, 0.f, 0.f});
                if (g == 0) store_stats(p, ri, -INFINITY, 0.f);
            }
        }
        return;
    }
    // This lane's query row sees keys [0, lim_lane) (padding rows: blk_lim).
    // Causal with two blocks (the host keeps a wave's 64 rows inside one
    // head): lim_lane holds block 0's limit before clamping to [0, kvb], and
    // block 1's row, 32 queries on, sees keys [0, clamp(lim_lane + 32)).
    int lim_lane = kv_len;
    if constexpr (kMask) {
        if (kCausal2 && causal)
            lim_lane = row0 < R ? row0 % p.q_len + kvb - p.q_len + 1 : blk_lim;
        else
            lim_lane = !causal ? kvb : row0 < R ? row_kv_limit(p, kvb, row0 % p.q_len) : blk_lim;
    }
    if constexpr (KS > 1) lim_lane = min(lim_lane, kv_end) - kv_base;

    issue_stage(b0, 0);
    f16x8 q0[kNKK], q1[(kRB == 2 && !kQ1Lds) ? kNKK : 1];
    load_q_frags<D>(Qg, row0, R, lane, q0);
    if constexpr (kQ1Lds) {
        // LDS-DMA of rows [rt kRows + kHalfRows, + kHalfRows) (rows past R
        // re-read row R - 1), in K's row layout.
        constexpr int kQInstr = kHalfRows * S::kRowBytes / 1024;
        static_assert(kQInstr % NW == 0, "whole Q copy rounds");
        const char* Qb = reinterpret_cast<const char*>(Qg);
        const int lr = lane / S::kChunks;
#pragma unroll
        for (int j0 = 0; j0 < kQInstr; j0 += NW) {
            const int j = j0 + wave_id;
            const int r = j * S::kRowsPerInstr + lr;
            // LDS row r holds block-1 row r % 32 of wave r / 32.
            const int src = min(rt * kRows + (kCausal2 ? (r >> 5) * wave_rows + b1_off + (r & 31)
                                                        : kHalfRows + r), R - 1);
            const uint32_t off = (uint32_t)src * S::kRowBytes +
                                 (uint32_t)((((lane % S::kChunks) ^ SW::h(r)) % S::kChunks) * 16);
            __builtin_amdgcn_global_load_lds(Qb + off, (lds_void*)(q1_lds + j * 1024), 16, 0, 0);
        }
    } else if constexpr (kRB == 2) {
        load_q_frags<D>(Qg, row1, R, lane, q1);
    }
    const char* q1w = q1_lds + wave * 32 * S::kRowBytes;  // this wave's block-1 rows

    RowState st0{-INFINITY, -INFINITY, 0.f, -INFINITY};
    RowState st1{-INFINITY, -INFINITY, 0.f, -INFINITY};
    const float inv_c = 1.0f / c;
    f32x16 o0[kNTD], o1[kNTD];
#pragma unroll
    for (int td = 0; td < kNTD; ++td) {
        o0[td] = f32x16{};
        o1[td] = f32x16{};
    }

    // S^T of both row blocks for the tile whose K rows are at `stage`.
    auto qk2 = [&](const char* stage, f32x16 (&s0)[1], f32x16 (&s1)[1]) {
        s0[0] = f32x16{};
        if constexpr (kRB == 2) s1[0] = f32x16{};
        int kb = kbase;
        if constexpr (kXorOff) asm volatile("" : "+v"(kb));  // recomputed per tile
#pragma unroll
        for (int kk = 0; kk < kNKK; ++kk) {
            const int ko = kXorOff ? (kb ^ (32 * kk)) : koff[kk];
            const f16x8 kf = *reinterpret_cast<const f16x8*>(stage + ko);
            s0[0] = mfma32(kf, q0[kk], s0[0]);
            if constexpr (kRB == 2) {
                f16x8 qb;
                if constexpr (kQ1Lds)
                    qb = *reinterpret_cast<const f16x8*>(q1w + koff[kk]);
                else
                    qb = q1[kk];
                s1[0] = mfma32(kf, qb, s1[0]);
            }
        }
    };
    // Keys at or past the lane's limit in tile t -> -inf (unmasked: the keys
    // past kv_len in the last tile).  Register r of
    // lane l holds key 8 (r / 4) + 4 (l / 32) + r % 4 of the tile: compare
    // 8 (r / 4) + r % 4 (an inline constant) with the limit less 4 (l / 32),
    // so no per-register key index stays live across the loop.
    auto tail_mask = [&](f32x16 (&s0)[1], f32x16 (&s1)[1], int t) {
        if ((t + 1) * BC > wave_min) {
            asm volatile("" ::: "memory");
            const int lg = lim_lane - t * BC - 4 * g;
            if constexpr (kCausal2) {
                // One block at a time: a second limit live across the tile
                // would cost a register that this kernel does not have.
                int lb = (causal ? min(max(lim_lane, 0), kvb) : lim_lane) - t * BC - 4 * g;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (8 * (r >> 2) + (r & 3) >= lb) s0[0][r] = -INFINITY;
                lb = (causal ? min(max(lim_lane + 32, 0), kvb) : lim_lane) - t * BC - 4 * g;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (8 * (r >> 2) + (r & 3) >= lb) s1[0][r] = -INFINITY;
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (8 * (r >> 2) + (r & 3) >= lg) {
                        s0[0][r] = -INFINITY;
                        if constexpr (kRB == 2) s1[0][r] = -INFINITY;
                    }
            }
        }
    };
    // O^T += V^T P^T for both row blocks, V rows at stage + kTensorBytes.
    auto pv2 = [&](const char* stage, const f16x8 (&p0)[2], const f16x8 (&p1)[2]) {
        int vb = vbase;
        if constexpr (kXorOff) asm volatile("" : "+v"(vb));  // recomputed per tile
#pragma unroll
        for (int td = 0; td < kNTD; ++td) {
            const int vo0 = kXorOff ? (vb ^ (64 * td)) : voff[td][0];
            const int vo1 = kXorOff ? ((vb ^ (64 * td) ^ 128) + 8 * S::kRowBytes) : voff[td][1];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const f16x4 lo = lds_read_tr16(stage + vo0 + jj * 16 * S::kRowBytes);
                const f16x4 hi = lds_read_tr16(stage + vo1 + jj * 16 * S::kRowBytes);
                const f16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                o0[td] = mfma32(a, p0[jj], o0[td]);
                if constexpr (kRB == 2) o1[td] = mfma32(a, p1[jj], o1[td]);
            }
        }
    };
    constexpr int H = BC * S::kRowBytes;  // bytes of one tile's K (or V) rows

    if constexpr (!kPipe) {
        // One 32-key tile at `stage`: S^T of both blocks, the row max / lazy
        // rescale / exp2 of each, then P.V for both.
        auto tile = [&](const char* stage, int t) {
            if (kMask && t >= nt_w) return;  // fully masked for this wave (wave-uniform)
            f32x16 s0[1], s1[1];
            qk2(stage, s0, s1);
            tail_mask(s0, s1, t);
            f16x8 p0[2], p1[2];
            block_update_max<kNTD>(st0, block_rowmax<1>(s0), c, inv_c, o0);
            // A row that has seen no key yet (masked, or a KV group's tiles
            // past the keys) keeps m = -inf and must get P = 0, not NaN.
            block_exp(s0[0], c, ((kMask || KS > 1) && st0.m == -INFINITY) ? 0.f : -st0.m, p0[0], p0[1],
                      st0.l);
            if constexpr (kRB == 2) {
                block_update_max<kNTD>(st1, block_rowmax<1>(s1), c, inv_c, o1);
                block_exp(s1[0], c, (kCausal2 && st1.m == -INFINITY) ? 0.f : -st1.m, p1[0], p1[1], st1.l);
            }
            pv2(stage, p0, p1);
        };
        constexpr int kSub = SR / BC;  // tiles per stage
        static_assert(kSub == 1 || kSub == 2, "one or two tiles per stage");
        for (int js = 0; js < nstages; js += 2) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int j = js + u;
                if (j >= nstages) break;
                char* cur = u == 0 ? b0 : b1;
                char* nxt = u == 0 ? b1 : b0;
                // Stage j (and, at j = 0, the block-1 query rows) landed for
                // every wave; every wave is done with stage j-1 (in nxt).
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
                if (j + 1 < nstages) issue_stage(nxt, (j + 1) * SR);
                tile(cur, kSub * j);
                if (kSub == 2 && 2 * j + 1 < ntiles) tile(cur + H, 2 * j + 1);
            }
        }
    } else {
        // Pipelined as kf_attn_prefill_kernel's 8-wave layout: S(t+1) of both
        // blocks is computed while tile t's scores are exponentiated, then
        // P.V(t) and the row max of S(t+1).  Tile t reads V(t) from `cur`
        // and K(t+1) from `nxt`, which may be the next stage: three buffers,
        // the copy of stage j+2 issued at the barrier before the last tile of
        // stage j (stage j-1 is then free and stage j+1 has landed).
        if (nstages > 1) issue_stage(buf1, SR);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        f32x16 sc0[1], sc1[1];
        qk2(buf0, sc0, sc1);
        tail_mask(sc0, sc1, 0);
        block_update_max<kNTD>(st0, block_rowmax<1>(sc0), c, inv_c, o0);
        block_update_max<kNTD>(st1, block_rowmax<1>(sc1), c, inv_c, o1);
        auto tile = [&](char* cur, char* nxt, char* fill, int t, bool sync) {
            if (sync) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
                const int js = t / 2 + 2;
                if (js < nstages) issue_stage(fill, js * SR);
            }
            f32x16 sn0[1], sn1[1];
            qk2(nxt, sn0, sn1);  // the last tile's reads a stale buffer, discarded
            f16x8 p0[2], p1[2];
            // Causal: a row with no key yet keeps m = -inf and gets P = 0.
            block_exp(sc0[0], c, (kCausal2 && st0.m == -INFINITY) ? 0.f : -st0.m, p0[0], p0[1], st0.l);
            block_exp(sc1[0], c, (kCausal2 && st1.m == -INFINITY) ? 0.f : -st1.m, p1[0], p1[1], st1.l);
            pv2(cur, p0, p1);
            if (t + 1 < ntiles) {
                tail_mask(sn0, sn1, t + 1);
                block_update_max<kNTD>(st0, block_rowmax<1>(sn0), c, inv_c, o0);
                block_update_max<kNTD>(st1, block_rowmax<1>(sn1), c, inv_c, o1);
                sc0[0] = sn0[0];
                sc1[0] = sn1[0];
            }
        };
        // Tile t reads the (t % 2)-th half of stage t / 2, which lives in
        // buffer (t / 2) % 3; the loop body covers 3 stages.
        for (int t = 0; t < ntiles; t += 6) {
            tile(buf0, buf0 + H, nullptr, t, false);
            if (t + 1 >= ntiles) break;
            tile(buf0 + H, buf1, buf2, t + 1, true);
            if (t + 2 >= ntiles) break;
            tile(buf1, buf1 + H, nullptr, t + 2, false);
            if (t + 3 >= ntiles) break;
            tile(buf1 + H, buf2, buf0, t + 3, true);
            if (t + 4 >= ntiles) break;
            tile(buf2, buf2 + H, nullptr, t + 4, false);
            if (t + 5 >= ntiles) break;
            tile(buf2 + H, buf0, buf1, t + 5, true);
        }
    }

    if constexpr (KS > 1) {
        // Merge slot k: 1 KiB at k * 1024 of buf0 (every group's stages).
        static_assert(kRowWaves * kNTD * 4 * (KS - 1) <= 2 * KS * S::kStageBytes / 1024, "merge slots");
        auto slot_base = [&](int k) { return buf0 + k * 1024; };
        __shared__ float merge_ml[2 * KS * kRowWaves * 64];
        merge_kv_groups<D, KS, kRowWaves>(p, st0, o0, slot_base, merge_ml, wave, kgrp, lane, g,
                                          (size_t)grp * R + row0, (size_t)grp * R + row0, row0 < R);
        return;
    }

    // ---- Epilogue: both row blocks (masked rows without a visible key:
    // O = 0, Mi = -inf, Li = 0). ----
    const float l0 = sum_xor32(st0.l);
    if (row0 < R) {
        const size_t ri = (size_t)grp * R + row0;
        const bool empty = kMask && !(l0 > 0.f);  // masked: no visible key
        store_o_row_any<D>(p, ri, o0, empty ? 0.f : 1.0f / l0, g);
        if (g == 0)
            store_stats(p, ri, st0.rmax * p.scale,
                        empty ? 0.f : l0 * rebase_factor(st0.m, st0.rmax, p.scale_log2));
    }
    if (kRB == 2 && row1 < R) {
        const float l1 = sum_xor32(st1.l);
        const size_t ri = (size_t)grp * R + row1;
        const bool empty = kCausal2 && !(l1 > 0.f);  // causal: no visible key
        store_o_row_any<D>(p, ri, o1, empty ? 0.f : 1.0f / l1, g);
        if (g == 0)
            store_stats(p, ri, st1.rmax * p.scale,
                        empty ? 0.f : l1 * rebase_factor(st1.m, st1.rmax, p.scale_log2));
    }
}


// ---------------------------------------------------------------------------
// Decode (split-KV): <= 32 query rows per KV head.  Workgroup = NW waves on
// one (group, split); wave w streams 32-row stages w, w+NW, w+2NW, ... of the
// split through its own LDS slot (single buffer, next stage prefetched into
// registers while the current one is computed; no workgroup barrier in the
// loop).  The NW wave states merge in LDS at the end.  D <= 128 runs 8 waves,
// one workgroup per CU (its LDS), D = 256 4 waves (one per SIMD).
// ---------------------------------------------------------------------------
constexpr int kDecodeStage = 32;

template <int D> struct DecodeCfg {
    static constexpr int kWaves = D >= 256 ? 4 : 8;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kWavesPerEU = D >= 256 ? 1 : 2;
};
inline int decode_waves(int D) { return D >= 256 ? DecodeCfg<256>::kWaves : DecodeCfg<128>::kWaves; }

template <int D>
struct DecodeSmem {
    using G = StageGeom<D, kDecodeStage>;
    static constexpr int NW = DecodeCfg<D>::kWaves;
    static constexpr int kOStride = D + 4;  // floats per merged-O row (padded)
    static constexpr int kStageBytes = NW * G::kStageHalfs * 2;
    static constexpr int kMergeBytes = NW * 32 * kOStride * 4 + NW * 32 * 2 * 4;
    static constexpr int kBytes = kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes;
};

// Element offsets and validity of the two 16-row halves of a 32-row stage of
// a paged K/V cache (page_size a power of two >= 16, stage start k0 a
// multiple of 32, rows beyond kv_end not needed).
struct PagedStage {
    size_t lo, hi;
    bool ok_lo, ok_hi;
};

template <int D>
__device__ __forceinline__ PagedStage paged_stage(const AttnParams& p, int bseq, int hkv, int k0,
                                                  int kv_end) {
    PagedStage ps;
    const int* tbl = p.block_table + (size_t)bseq * p.max_pages;
    const int sh = p.page_shift;
    const int pi = k0 >> sh;
    const int id0 = tbl[pi];
    ps.ok_lo = (unsigned)id0 < (unsigned)p.num_pages;
    ps.lo = ((((size_t)(unsigned)id0 * p.heads_kv + hkv) << sh) + (size_t)(k0 & ((1 << sh) - 1))) * D;
    if (sh == 4) {  // 16-row pages: the second half is the next page
        const int id1 = k0 + 16 < kv_end ? tbl[pi + 1] : -1;
        ps.ok_hi = (unsigned)id1 < (unsigned)p.num_pages;
        ps.hi = (((size_t)(unsigned)id1 * p.heads_kv + hkv) << 4) * D;
    } else {
        ps.ok_hi = ps.ok_lo;
        ps.hi = ps.lo + 16 * D;
    }
    return ps;
}

// kPaged: K / V are page pools addressed through p.block_table.
template <int D, bool kPaged>
__global__ __launch_bounds__(DecodeCfg<D>::kThreads, DecodeCfg<D>::kWavesPerEU)
void kf_attn_decode_kernel(AttnParams p) {
    using G = StageGeom<D, kDecodeStage>;
    using SM = DecodeSmem<D>;
    constexpr int NW = DecodeCfg<D>::kWaves;
    constexpr int kThreads = DecodeCfg<D>::kThreads;
    // D = 256, and paged D = 128: the Q^T fragments (64 / 32 registers) are
    // read from an LDS copy of the group's 32 query rows at every stage
    // instead of being held, which keeps the register-staged K/V stage, the O
    // accumulators and the paged addressing within the register file (held
    // in registers they spilled to scratch: inside the stage loop at
    // D = 256, around it for paged D = 128).
    constexpr bool kQLds = D >= 256 || (kPaged && D >= 128);
    __shared__ __attribute__((aligned(16))) char smem_raw[SM::kBytes];
    __shared__ __attribute__((aligned(16))) char q_lds[kQLds ? 32 * D * 2 : 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5;
    const int blk = xcd_remap(blockIdx.x, gridDim.x, p.xcds);
    const int split = blk % p.n_splits;
    const int grp = blk / p.n_splits;
    const int R = p.rows_per_group;
    const int kv_len = p.kv_len;
    // Keys of this sequence; with causal masking row r (query index
    // r % q_len) sees the first row_kv_limit(...) of them, at least
    // kvb - q_len + 1 (the rows of a group cover every query index).
    const int kvb = batch_kv_len(p, grp);
    const int s0 = split * p.kv_per_split;
    const int s1 = min(kvb, s0 + p.kv_per_split);
    const int lim_min = p.causal ? max(kvb - p.q_len + 1, 0) : kvb;

    const uint16_t* Qg = p.Q + (size_t)grp * R * D;
    const uint16_t* Kh = kPaged ? p.K : p.K + (size_t)grp * kv_len * D;
    const uint16_t* Vh = kPaged ? p.V : p.V + (size_t)grp * kv_len * D;
    const int bseq = grp / p.heads_kv, hkv = grp % p.heads_kv;  // paged addressing

    const int row = lane & 31;
    f16x8 qf[kQLds ? 1 : D / 16];
    if constexpr (kQLds) {
        // Row r (rows >= R repeat row R - 1), 16-byte chunk c stored at chunk
        // c ^ (r & 15) of LDS row r, so that the 32 rows read by one fragment
        // load spread over the banks.
        constexpr int kChunks = D / 8;
        for (int i = tid; i < 32 * kChunks; i += kThreads) {
            const int r = i / kChunks, c = i % kChunks;
            const u32x4 v = *reinterpret_cast<const u32x4*>(Qg + (size_t)min(r, R - 1) * D + c * 8);
            *reinterpret_cast<u32x4*>(q_lds + (r * kChunks + (c ^ (r & 15))) * 16) = v;
        }
        __syncthreads();
    } else {
        load_q_frags<D>(Qg, row, R, lane, qf);
    }
    const int lim_lane = row < R ? row_kv_limit(p, kvb, row % p.q_len) : kvb;

    f16* Ks = reinterpret_cast<f16*>(smem_raw) + wave * G::kStageHalfs;
    f16* Vt = Ks + G::kKHalfs;
    if constexpr (D < 32) {
        for (int i = lane; i < (32 - D) * G::kVtStride; i += 64) Vt[D * G::kVtStride + i] = (f16)0.f;
    }

    RowState st{-INFINITY, -INFINITY, 0.f, -INFINITY};
    f32x16 o[G::kNTD];
#pragma unroll
    for (int td = 0; td < G::kNTD; ++td) o[td] = f32x16{};

    StageLoader<D, kDecodeStage, 64> ld;
    PagedStage pc{0, 0, true, true}, pn{0, 0, true, true};
    auto load_stage = [&](int k0, PagedStage& ps) {
        if constexpr (kPaged) {
            ps = paged_stage<D>(p, bseq, hkv, k0, s1);
            ld.load_halves(Kh, Vh, ps.lo, ps.hi, ps.ok_lo, ps.ok_hi, s1 - k0, lane);
        } else {
            ld.load(Kh, Vh, k0, s1, lane);
        }
    };
    // The split's stages come in rounds of NW (one stage per wave).  With few
    // splits per KV head (contiguous cache only), every workgroup starts at a
    // round of its own (a hash of group and split) and wraps around, so the
    // workgroups running at once do not all read the same relative offset of
    // their equally sized K / V ranges: B = 8 x 8192 keys measured 5.7 %
    // faster, D = 64 3-4 %, and one GPU that ran B = 64 x 4096 keys 13 %
    // slow in the plain order ran it at full speed.  Paged caches (random
    // page placement) and many splits (already staggered) keep the plain
    // order, which measured as fast or faster there.
    const int n_rounds = s1 > s0 ? (s1 - s0 + NW * kDecodeStage - 1) / (NW * kDecodeStage) : 0;
    const bool rotate = !kPaged && p.n_splits <= 4;
    const int r0 = (rotate && n_rounds > 1)
                       ? (int)(((unsigned)grp * 11u + (unsigned)split * 7u) % (unsigned)n_rounds)
                       : 0;
    auto stage_kv = [&](int i) {
        int r = r0 + i;
        if (r >= n_rounds) r -= n_rounds;
        return s0 + (r * NW + wave) * kDecodeStage;
    };
    auto next_valid = [&](int i) {
        while (i < n_rounds && stage_kv(i) >= s1) ++i;
        return i;
    };
    int ri = next_valid(0);
    int kv0 = ri < n_rounds ? stage_kv(ri) : s1;
    if (kv0 < s1) load_stage(kv0, pc);
    while (kv0 < s1) {
        wave_lds_sync();  // previous stage's LDS reads are done
        ld.store(Ks, Vt, lane);
        wave_lds_sync();
        ri = next_valid(ri + 1);
        const int kv_next = ri < n_rounds ? stage_kv(ri) : s1;
        if (kv_next < s1) load_stage(kv_next, pn);

        f32x16 s[1];
        if constexpr (kQLds)
            s[0] = qk_block_qlds<D, kDecodeStage>(Ks, q_lds, lane);
        else
            s[0] = qk_block<D, kDecodeStage>(Ks, 0, qf, lane);
        if (kv0 + kDecodeStage > min(s1, lim_min) || !(pc.ok_lo && pc.ok_hi)) {
            const int lim = min(s1, lim_lane) - kv0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ar = acc_row(r, lane);
                if (ar >= lim || !(ar < 16 ? pc.ok_lo : pc.ok_hi)) s[0][r] = -INFINITY;
            }
        }
        f16x8 pb[2];
        softmax_update<1, G::kNTD>(s, st, o, p.scale_log2, pb);
        pv_accum<D, kDecodeStage, 2>(Vt, 0, pb, o, lane);
        kv0 = kv_next;
        pc = pn;
    }

    // Rebase this wave's state onto its true max (natural-log scaled units).
    const float l_pair = sum_xor32(st.l);
    const bool empty = st.rmax == -INFINITY;
    const float m_nat = empty ? -INFINITY : st.rmax * p.scale;
    const float beta = empty ? 0.f : rebase_factor(st.m, st.rmax, p.scale_log2);

    __syncthreads();  // all waves are done with their stage slots
    float* Ob = reinterpret_cast<float*>(smem_raw);
    float* Mb = Ob + NW * 32 * SM::kOStride;
    float* Lb = Mb + NW * 32;
#pragma unroll
    for (int td = 0; td < G::kNTD; ++td)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = 32 * td + 8 * i + 4 * g;
            if (d < D) {
                f32x4 v = {o[td][4 * i] * beta, o[td][4 * i + 1] * beta,
                           o[td][4 * i + 2] * beta, o[td][4 * i + 3] * beta};
                *reinterpret_cast<f32x4*>(Ob + (wave * 32 + row) * SM::kOStride + d) = v;
            }
        }
    if (g == 0) {
        Mb[wave * 32 + row] = m_nat;
        Lb[wave * 32 + row] = l_pair * beta;
    }
    __syncthreads();

    // Merge the NW wave states: thread -> (query row, kSeg-wide d segment).
    constexpr int kTpr = D / 4 < 8 ? D / 4 : 8;  // threads per query row
    constexpr int kSeg = D / kTpr;                // multiple of 4
    static_assert(kThreads / kTpr >= 32, "merge must cover 32 rows in one pass");
    const int mrow = tid / kTpr;
    const int seg = tid % kTpr;
    if (mrow < R) {
        float m = Mb[mrow];
#pragma unroll
        for (int w = 1; w < NW; ++w) m = fmaxf(m, Mb[w * 32 + mrow]);
        float wt[NW];
        float l = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = Mb[w * 32 + mrow];
            wt[w] = mw == -INFINITY ? 0.f : exp2_hw((mw - m) * kLog2e);
            l += wt[w] * Lb[w * 32 + mrow];
        }
        const bool final_out = p.n_splits == 1;
        const float inv = final_out ? (l > 0.f ? 1.0f / l : 0.f) : 1.0f;
        // Final rows go to O; split partials (fp32) to [grp][split][row][D].
        const size_t ri = (size_t)grp * R + mrow;
        const size_t pi = ((size_t)grp * p.n_splits + split) * R + mrow;
#pragma unroll
        for (int j = 0; j < kSeg; j += 4) {
            const int d = seg * kSeg + j;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(Ob + (w * 32 + mrow) * SM::kOStride + d);
                acc += wt[w] * v;
            }
            if (final_out)
                store_out4(p, ri * D + d, acc * inv);
            else
                *reinterpret_cast<f32x4*>(p.Opart + pi * D + d) = acc;
        }
        if (seg == 0) {
            if (final_out) {
                store_stats(p, ri, m, l);
            } else {
                p.Mpart[pi] = m;
                p.Lpart[pi] = l;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Short-split decode: <= 32 query rows per KV head and NST * 32 keys per
// split.  Each wave is its own (group, split), 4 waves per workgroup: at
// entry it issues every load it needs -- the Q^T fragments, its K rows
// straight into the MFMA A-operand layout (lane l: key row l % 32, 16-byte
// chunk 2 kk + l / 32 for k-step kk; no LDS), and its V rows by LDS-DMA into
// a wave-private slot (row-major, chunks XOR-swizzled by SwizzleRow<D>, read
// back as V^T fragments with ds_read_b64_tr_b16).  All of the split's scores
// are in registers at once, so the softmax uses their exact maximum (no
// running rescale).  The wave writes its partial (O unnormalised, M, l) or,
// with one split, the final row; no workgroup barrier anywhere.
//
// kPaged (kf_attn_decode_short_paged_kernel): K / V are page pools read
// through p.block_table.  Pages hold >= 16 rows, so a split of <= 64 keys
// spans at most 4 pages; the wave reads their ids with wave-uniform (scalar)
// loads before its K / V loads and each lane addresses its rows through
// them.  A row on a page id outside [0, num_pages) is loaded from page 0
// instead (the invalid page is never read), its scores are masked to -inf
// and its V row is zeroed in the slot, so it contributes exactly nothing.
// ---------------------------------------------------------------------------
constexpr int kShortWaves = 4;  // waves (independent splits) per workgroup

template <int D> constexpr int kShortMaxStages = D >= 256 ? 1 : 2;

template <int D, int NST> struct ShortCfg {
    static constexpr int kKeys = 32 * NST;                // keys per split
    static constexpr int kVBytes = kKeys * D * 2;         // V slot per wave
};

template <int D, int NST, bool kPaged>
__device__ __forceinline__ void decode_short_body(const AttnParams& p, char* vbuf) {
    static_assert(NST >= 1 && NST <= kShortMaxStages<D>, "stages per split");
    constexpr int kRowBytes = D * 2;
    constexpr int kChunks = D / 8;                   // 16-byte chunks per row
    constexpr int kKeys = ShortCfg<D, NST>::kKeys;   // keys per split
    constexpr int kVBytes = ShortCfg<D, NST>::kVBytes;
    constexpr int kRowsPerInstr = 1024 / kRowBytes;  // rows per LDS-DMA instruction
    constexpr int kInstr = kVBytes / 1024;
    constexpr int kNKK = D / 16;                     // MFMA k-steps over D
    constexpr int kNTD = (D < 32 ? 32 : D) / 32;     // 32-row O^T tiles
    static_assert(kVBytes % 1024 == 0, "V slot in whole KiB");
    using SW = SwizzleRow<D>;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 5;
    const int row = lane & 31;
    const int R = p.rows_per_group;
    const int ns = p.n_splits;
    const int wid = xcd_remap(blockIdx.x, gridDim.x, p.xcds) * kShortWaves + wave;
    if (wid >= (p.rows_total / R) * ns) return;  // past the last split (wave-uniform)
    const int split = wid % ns, grp = wid / ns;
    const int kvb = batch_kv_len(p, grp);
    const int s0 = split * kKeys;
    const int s1 = min(kvb, s0 + kKeys);
    const size_t ri = (size_t)grp * R + row;                  // final row index
    const size_t pi = ((size_t)grp * ns + split) * R + row;   // partial index

    if (s0 >= s1) {
        // No key of this sequence in the split: an empty partial (or row).
        if (row < R) {
#pragma unroll
            for (int td = 0; td < kNTD; ++td)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int d = 32 * td + 8 * i + 4 * g;
                    if (d < D) {
                        if (ns == 1)
                            store_out4(p, ri * D + d, f32x4{0.f, 0.f, 0.f, 0.f});
                        else
                            *reinterpret_cast<f32x4*>(p.Opart + pi * D + d) = f32x4{0.f, 0.f, 0.f, 0.f};
                    }
                }
            if (g == 0) {
                if (ns == 1) {
                    store_stats(p, ri, -INFINITY, 0.f);
                } else {
                    p.Mpart[pi] = -INFINITY;
                    p.Lpart[pi] = 0.f;
                }
            }
        }
        return;
    }

    // ---- Loads, all issued before the first wait (one memory round trip):
    // V into LDS, then the Q^T fragments and K into registers.  All are
    // unpredicated: rows past s1 re-read row s1 - 1, whose scores are masked
    // below. ----
    const int last = s1 - 1;
    const uint16_t* Qg = p.Q + (size_t)grp * R * D;
    const uint16_t* Kh = kPaged ? p.K : p.K + (size_t)grp * p.kv_len * D;
    const char* Vh = reinterpret_cast<const char*>(kPaged ? p.V : p.V + (size_t)grp * p.kv_len * D);
    // Paged: the ids of the (at most 4) pages of keys [s0, last], the first
    // one pg0; an invalid id reads page 0 and flags its keys (bad_pages bit j).
    int pid[4] = {0, 0, 0, 0};
    int pg0 = 0, bad_pages = 0, hkv = 0;
    if constexpr (kPaged) {
        const int* tbl = p.block_table + (size_t)(grp / p.heads_kv) * p.max_pages;
        hkv = grp % p.heads_kv;
        pg0 = s0 >> p.page_shift;
        const int pgl = last >> p.page_shift;  // pgl - pg0 <= 3
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int id = tbl[min(pg0 + j, pgl)];
            const bool ok = (unsigned)id < (unsigned)p.num_pages;
            pid[j] = ok ? id : 0;
            if (!ok && pg0 + j <= pgl) bad_pages |= 1 << j;
        }
    }
    // Element offset of key row kv (s0 <= kv <= last) in K / V.
    auto row_off = [&](int kv) -> size_t {
        if constexpr (kPaged) {
            const int j = (kv >> p.page_shift) - pg0;
            const int id = j == 0 ? pid[0] : j == 1 ? pid[1] : j == 2 ? pid[2] : pid[3];
            return ((((size_t)id * p.heads_kv + hkv) << p.page_shift) +
                    (size_t)(kv & ((1 << p.page_shift) - 1))) * D;
        } else {
            return (size_t)kv * D;
        }
    };
    // Lane l of DMA instruction ii writes LDS bytes [16 l, 16 l + 16) of KiB ii
    // of the slot: row r = ii * kRowsPerInstr + l / kChunks, physical chunk
    // l % kChunks, which holds logical chunk (l % kChunks) ^ h(r) of key s0 + r.
    char* const vs = vbuf + wave * kVBytes;
#pragma unroll
    for (int ii = 0; ii < kInstr; ++ii) {
        const int r = ii * kRowsPerInstr + lane / kChunks;
        const int kv = min(s0 + r, last);
        const uint32_t chunk = (uint32_t)((((lane % kChunks) ^ SW::h(r)) % kChunks) * 16);
        const char* src;
        if constexpr (kPaged)
            src = Vh + row_off(kv) * 2 + chunk;
        else
            src = Vh + ((uint32_t)kv * kRowBytes + chunk);
        __builtin_amdgcn_global_load_lds(src, (lds_void*)(vs + ii * 1024), 16, 0, 0);
    }
    f16x8 qf[kNKK];
    load_q_frags<D>(Qg, row, R, lane, qf);
    f16x8 kf[NST][kNKK];
#pragma unroll
    for (int b = 0; b < NST; ++b) {
        const int kv = min(s0 + 32 * b + row, last);
        const uint16_t* kr = Kh + row_off(kv);
#pragma unroll
        for (int kk = 0; kk < kNKK; ++kk)
            kf[b][kk] = *reinterpret_cast<const f16x8*>(kr + (2 * kk + g) * 8);
    }
    __builtin_amdgcn_sched_barrier(0);  // no MFMA (and its wait) above the loads

    // ---- Scores S^T = K Q^T (kv x query row), masked past each row's keys. ----
    f32x16 s[NST];
#pragma unroll
    for (int b = 0; b < NST; ++b) {
        s[b] = f32x16{};
#pragma unroll
        for (int kk = 0; kk < kNKK; ++kk) s[b] = mfma32(kf[b][kk], qf[kk], s[b]);
    }
    const int lim_min = p.causal ? max(kvb - p.q_len + 1, 0) : kvb;  // keys every row sees
    if (s0 + kKeys > min(s1, lim_min)) {
        const int lim_lane = row < R ? row_kv_limit(p, kvb, row % p.q_len) : kvb;
        block_mask<NST>(s, min(s1, lim_lane) - s0, lane);
    }
    // Keys on an invalid page (paged, wave-uniform branch): score -inf.
    auto bad_key = [&](int k) {  // key s0 + k, 0 <= k < kKeys (rows past last: last's page)
        const int j = (min(s0 + k, last) >> p.page_shift) - pg0;
        return ((bad_pages >> j) & 1) != 0;
    };
    if (kPaged && bad_pages) {
#pragma unroll
        for (int b = 0; b < NST; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (bad_key(32 * b + acc_row(r, lane))) s[b][r] = -INFINITY;
    }

    // ---- Softmax against the exact row max; fp16 P^T fragments. ----
    const float mx = block_rowmax<NST>(s);  // raw scores; shared with lane l ^ 32
    const bool empty = mx == -INFINITY;     // no visible key for this row
    const float neg_m = empty ? 0.f : -mx * p.scale_log2;
    f16x8 pp[2 * NST];
    float lsum = 0.f;
#pragma unroll
    for (int b = 0; b < NST; ++b) block_exp(s[b], p.scale_log2, neg_m, pp[2 * b], pp[2 * b + 1], lsum);
    const float l = sum_xor32(lsum);

    // ---- O^T = V^T P^T; V^T fragments by ds_read_b64_tr_b16 from the slot. ----
    // 16-lane group G = l / 16, w = l % 16 supplies key row 4 (G / 2) + w / 4
    // (+8 for the second half of the 16-key step) and the 8 bytes at
    // d = 32 td + 16 (G % 2) + 4 (w % 4).  D = 16: groups with d >= 16 give
    // the zero rows 16..31 of V^T (their reads, of valid rows, are discarded).
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the slot's LDS-DMA has landed
    if (kPaged && bad_pages) {
        // V rows of invalid pages (loaded from page 0) -> zeros, so that their
        // P = 0 meets finite values.
        wave_lds_sync();
        for (int i = lane; i < kKeys * kChunks; i += 64)
            if (bad_key(i / kChunks)) *reinterpret_cast<u32x4*>(vs + i * 16) = u32x4{0u, 0u, 0u, 0u};
        wave_lds_sync();
    }
    const int G = lane >> 4, w = lane & 15;
    f32x16 o[kNTD];
#pragma unroll
    for (int td = 0; td < kNTD; ++td) {
        o[td] = f32x16{};
        const int d = 32 * td + 16 * (G & 1) + 4 * (w & 3);
        const bool dok = d < D;
        const int dc = dok ? d : d - 16;
        int voff[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int r = 4 * (G >> 1) + (w >> 2) + 8 * h2;
            voff[h2] = r * kRowBytes + (((dc >> 3) ^ SW::h(r)) % kChunks) * 16 + ((dc >> 2) & 1) * 8;
        }
#pragma unroll
        for (int jj = 0; jj < 2 * NST; ++jj) {
            const f16x4 lo = lds_read_tr16(vs + voff[0] + jj * 16 * kRowBytes);
            const f16x4 hi = lds_read_tr16(vs + voff[1] + jj * 16 * kRowBytes);
            f16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            if (D < 32 && !dok) a = f16x8{};
            o[td] = mfma32(a, pp[jj], o[td]);
        }
    }

    // ---- Output: this split's partial, or the final row with one split (the
    // choice, and the output format, made once: not per store). ----
    if (row < R) {
        const float m_nat = empty ? -INFINITY : mx * p.scale;
        if (ns > 1) {
#pragma unroll
            for (int td = 0; td < kNTD; ++td)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int d = 32 * td + 8 * i + 4 * g;
                    if (d < D)
                        *reinterpret_cast<f32x4*>(p.Opart + pi * D + d) =
                            f32x4{o[td][4 * i], o[td][4 * i + 1], o[td][4 * i + 2], o[td][4 * i + 3]};
                }
            if (g == 0) {
                p.Mpart[pi] = m_nat;
                p.Lpart[pi] = empty ? 0.f : l;
            }
        } else {
            const float inv = empty ? 0.f : 1.0f / l;
            store_o_row_any<D>(p, ri, o, inv, g);
            if (g == 0) store_stats(p, ri, m_nat, empty ? 0.f : l);
        }
    }
}

template <int D, int NST>
__global__ __launch_bounds__(64 * kShortWaves, D >= 256 ? 1 : 2)
void kf_attn_decode_short_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(1024))) char vbuf[kShortWaves * ShortCfg<D, NST>::kVBytes];
    decode_short_body<D, NST, false>(p, vbuf);
}

template <int D, int NST>
__global__ __launch_bounds__(64 * kShortWaves, D >= 256 ? 1 : 2)
void kf_attn_decode_short_paged_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(1024))) char vbuf[kShortWaves * ShortCfg<D, NST>::kVBytes];
    decode_short_body<D, NST, true>(p, vbuf);
}

// ---------------------------------------------------------------------------
// Split merge: one wave per (query row, block of CW float4 columns of O);
// CW is a power of two in [4, min(D/4, 64)] chosen by the host.  Lane l owns
// column c = cb * CW + l % CW and the splits k = l / CW + i * (64 / CW),
// i < NPER (NPER, a power of two <= kMergePer, covers n_splits).  Every load
// (partial O, M, l) is unconditional and issued before the first use, so the
// merge costs one memory round trip; the reductions over the 64 / CW lanes of
// a column are VALU cross-lane operations (reduce_mod).  Every wave of a row
// computes the row's max and l itself.  Waves are dealt to the XCDs like the
// decode workgroups (xcd_remap over a grid ordered by group), so a group's
// partials are read on the XCD whose L2 received them.  The planner never
// makes more splits than kMergeMaxSplits = kMergePer * 16.
//   O = sum_k w_k O_k / sum_k w_k l_k,  w_k = exp(M_k - max_j M_j),
//   Mi = max_k M_k,  Li = sum_k w_k l_k.
// ---------------------------------------------------------------------------
constexpr int kMergeThreads = 64;
constexpr int kMergePer = 16;                    // most splits per lane
constexpr int kMergeTarget = 8;                  // splits per lane the planner aims for
constexpr int kMergeMaxSplits = kMergePer * 16;  // CW = 4: 16 split lanes

// Float4 columns per merge wave for ns splits: the widest block whose
// 64 / CW split lanes cover ns with at most kMergeTarget splits each (at
// CW = 4, up to kMergePer).
constexpr int merge_cols(int D, int ns) {
    int cw = D / 4 < 64 ? D / 4 : 64;
    while (cw > 4 && (ns + 64 / cw - 1) / (64 / cw) > kMergeTarget) cw /= 2;
    return cw;
}

// Splits per lane (a power of two) for ns splits over 64 / cw split lanes.
// A block narrower than min(D/4, 64) is only chosen with kMergeTarget
// splits per lane, or kMergePer at CW = 4.
constexpr int merge_per_lane(int cw, int ns) {
    const int need = (ns + 64 / cw - 1) / (64 / cw);
    int per = 1;
    while (per < need) per *= 2;
    return per;
}

template <int D, int NPER, int CW>
__global__ __launch_bounds__(kMergeThreads)
void kf_attn_split_merge_kernel(AttnParams p) {
    static_assert(NPER >= 1 && NPER <= kMergePer, "splits per lane");
    static_assert(CW >= 4 && CW <= 64 && CW <= D / 4 && (CW & (CW - 1)) == 0, "column block");
    constexpr int kNCB = (D / 4) / CW;             // column blocks per row
    constexpr int kSL = 64 / CW;                   // split lanes per column
    const int lane = threadIdx.x;
    const int mb = xcd_remap(blockIdx.x, gridDim.x, p.xcds);
    const int row = mb / kNCB;                     // global query row
    const int cb = mb % kNCB;
    const int R = p.rows_per_group;
    const int grp = row / R, r = row % R;
    const int ns = p.n_splits;                     // 1 .. NPER * kSL
    const size_t base = (size_t)grp * ns * R + r;  // partial index of split 0
    const int c = cb * CW + lane % CW, sl = lane / CW;

    f32x4 o[NPER];
    float mk[NPER], lk[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        // Splits past ns read split ns - 1 and get weight 0 below.
        const size_t pi = base + (size_t)min(sl + i * kSL, ns - 1) * R;
        o[i] = *reinterpret_cast<const f32x4*>(p.Opart + pi * D + 4 * c);
        mk[i] = p.Mpart[pi];
        lk[i] = p.Lpart[pi];
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPER; ++i)
        if (sl + i * kSL < ns) m = fmaxf(m, mk[i]);
    m = reduce_mod<CW, true>(m);
    const bool none = m == -INFINITY;  // no split saw a key for this row
    float l = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const bool live = sl + i * kSL < ns && !none;
        const float w = live ? exp2_hw((mk[i] - m) * kLog2e) : 0.f;
        l += w * lk[i];
        acc += w * o[i];
    }
    l = reduce_mod<CW, false>(l);
    acc.x = reduce_mod<CW, false>(acc.x);
    acc.y = reduce_mod<CW, false>(acc.y);
    acc.z = reduce_mod<CW, false>(acc.z);
    acc.w = reduce_mod<CW, false>(acc.w);
    if (sl == 0) {
        store_out4(p, (size_t)row * D + 4 * c, acc * (l > 0.f ? 1.0f / l : 0.f));
        if (c == 0) store_stats(p, row, m, l);
    }
}

}  // namespace kf
