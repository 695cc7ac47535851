// attn_kernels.h -- gfx950 (CDNA4) flash-attention forward kernels.
//
// Two kernels, both hand-written for wave64 and the fp16 MFMA
// v_mfma_f32_32x32x16_f16:
//
//   kf_attn_prefill_kernel<D>  one workgroup = 4 waves = 128 query rows of one
//                              KV head; K/V streamed through double-buffered
//                              LDS stages; online softmax in registers.
//   kf_attn_decode_kernel<D>   split-KV ("flash-decoding") for <= 32 query
//                              rows per KV head (Q_len = 1 decode, GQA/MQA
//                              groups): every wave streams its own KV stages
//                              through a wave-private LDS slot; the 4 waves of
//                              a workgroup merge in LDS; with several splits
//                              each workgroup writes an unnormalised partial
//                              and the last one of its group to finish merges
//                              them into O, Mi, Li (one launch, no combine
//                              kernel).
//
// Behaviour follows the reference forward (kernels/flash_attn.cu:384-585):
// O = softmax(Q K^T / sqrt(D)) V per (b, h_q) with h_kv = h_q / (H_q / H_kv)
// (:406), fp16 inputs, fp32 accumulation and softmax, P rounded to fp16
// before the P.V product (:301-303) while the row sum uses the fp32 P
// (:284-294), O divided by the row sum once at the end (:582-584), and the
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
#include <stdint.h>

namespace kf {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
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
constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin

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
    unsigned long long* tickets;  // [B * H_kv] split-merge tickets (epoch << 32 | count)
    unsigned epoch;     // unique per call, never 0
    int rows_per_group; // R = (H_q / H_kv) * q_len
    int kv_len;
    int row_tiles;      // prefill: ceil(R / 128)
    int n_splits;       // decode: KV partitions per group
    int kv_per_split;   // decode: multiple of 32
    int rows_total;     // B * H_q * q_len
    float scale;        // 1 / sqrt(D), fp32 (the reference's softmax scale)
    float scale_log2;   // scale * log2(e)
};

// ---------------------------------------------------------------------------
// Small device helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x16 mfma32(const f16x8& a, const f16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ u32x4 load16(const uint16_t* p, bool pred) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (pred) v = *reinterpret_cast<const u32x4*>(p);
    return v;
}

__device__ __forceinline__ f16x8 as_f16x8(const u32x4& v) { return __builtin_bit_cast(f16x8, v); }

// Hardware workgroup id -> logical id such that each XCD receives one
// contiguous range of logical ids (the dispatcher deals ids round-robin over
// the 8 XCDs).  Logical neighbours share K/V, so each XCD's L2 holds them.
__device__ __forceinline__ int xcd_remap(int hw, int n) {
    const int q = n / kXcds, r = n % kXcds;
    const int xcd = hw % kXcds, k = hw / kXcds;
    return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + k;
}

// Count this workgroup into its group's split merge; true for the last of
// n arrivals in this call.  The word holds (epoch << 32 | count): a count
// left by an earlier call (other epoch) restarts at 1, so the workspace needs
// no zeroing between calls.  Every failed compare-and-swap means another
// workgroup's swap succeeded; with n arrivals per epoch the loop ends after
// at most n iterations.
__device__ __forceinline__ bool take_ticket(unsigned long long* word, unsigned epoch, int n) {
    unsigned long long old = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned cnt;
    for (;;) {
        const unsigned long long assumed = old;
        cnt = (unsigned)(assumed >> 32) == epoch ? (unsigned)(assumed & 0xffffffffu) + 1u : 1u;
        const unsigned long long want = ((unsigned long long)epoch << 32) | cnt;
        old = atomicCAS(word, assumed, want);
        if (old == assumed) break;
    }
    return cnt == (unsigned)n;
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
// transposed.  Rows at or beyond kv_end are zero-filled, so masked scores
// meet zero V rows (0 * garbage could be NaN).
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

    __device__ __forceinline__ void load(const uint16_t* __restrict__ Kh,
                                         const uint16_t* __restrict__ Vh, int kv0, int kv_end,
                                         int tid) {
#pragma unroll
        for (int i = 0; i < kKIters; ++i) {
            const int idx = tid + i * NT;
            const bool in = (kKTotal % NT == 0) || idx < kKTotal;
            const int row = idx / G::kChunks, c = idx % G::kChunks;
            const int kv = kv0 + row;
            k[i] = load16(Kh + (size_t)kv * D + c * 8, in && kv < kv_end);
        }
#pragma unroll
        for (int i = 0; i < kVIters; ++i) {
            const int idx = tid + i * NT;
            const bool in = (kVTotal % NT == 0) || idx < kVTotal;
            const int grp = idx % kVGroups, c = idx / kVGroups;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int kv = kv0 + 4 * grp + r;
                v[i][r] = load16(Vh + (size_t)kv * D + c * 8, in && kv < kv_end);
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

// Q^T fragments of one wave: query row `row` of the group (zero when
// row >= R), chunk 2*kk + (lane/32) for MFMA k-step kk.
template <int D>
__device__ __forceinline__ void load_q_frags(const uint16_t* __restrict__ Qg, int row, int R,
                                             int lane, f16x8 (&qf)[D / 16]) {
    const int g = lane >> 5;
    const bool ok = row < R;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
        qf[kk] = as_f16x8(load16(Qg + (size_t)row * D + (2 * kk + g) * 8, ok));
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
};

// Online-softmax update for NSB score blocks: moves the running max (lazily),
// rescales O, exponentiates, accumulates the fp32 row sum and packs fp16 P^T
// operands (p[j] covers kv 16j .. 16j+15 of the stage).
template <int NSB, int NTD>
__device__ __forceinline__ void softmax_update(f32x16 (&s)[NSB], RowState& st,
                                               f32x16 (&o)[NTD], float scale_log2,
                                               f16x8 (&p)[2 * NSB]) {
    float mx = s[0][0];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[sb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    st.rmax = fmaxf(st.rmax, mx);
    const float mt = mx * scale_log2;
    const bool need = mt > st.m + kLazyRescaleLog2;
    if (__any(need)) {
        const float mnew = need ? mt : st.m;
        const float alpha = exp2_hw(st.m - mnew);
        st.l *= alpha;
#pragma unroll
        for (int td = 0; td < NTD; ++td) o[td] *= alpha;
        st.m = mnew;
    }
    const float neg_m = -st.m;
    float sum = 0.f;
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f32x8 e;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                e[r] = exp2_hw(fmaf(s[sb][8 * h + r], scale_log2, neg_m));
                sum += e[r];
            }
            p[2 * sb + h] = __builtin_convertvector(e, f16x8);
        }
    }
    st.l += sum;
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
// Prefill: 4 waves x 32 query rows per workgroup, BC-row K/V stages shared by
// all 4 waves, double-buffered in LDS with register-staged prefetch.
// ---------------------------------------------------------------------------
template <int D> struct PrefillCfg;
template <> struct PrefillCfg<16>  { static constexpr int BC = 64;  static constexpr int kWavesPerEU = 2; };
template <> struct PrefillCfg<64>  { static constexpr int BC = 128; static constexpr int kWavesPerEU = 2; };
template <> struct PrefillCfg<128> { static constexpr int BC = 64;  static constexpr int kWavesPerEU = 2; };
template <> struct PrefillCfg<256> { static constexpr int BC = 32;  static constexpr int kWavesPerEU = 1; };

constexpr int kPrefillThreads = 256;
constexpr int kPrefillRows = 128;

template <int D>
__global__ __launch_bounds__(kPrefillThreads, PrefillCfg<D>::kWavesPerEU)
void kf_attn_prefill_kernel(AttnParams p) {
    constexpr int BC = PrefillCfg<D>::BC;
    using G = StageGeom<D, BC>;
    __shared__ __attribute__((aligned(16))) f16 smem[2 * G::kStageHalfs];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 5;
    const int blk = xcd_remap(blockIdx.x, gridDim.x);
    const int rt = blk % p.row_tiles;
    const int grp = blk / p.row_tiles;
    const int R = p.rows_per_group;
    const int kv_len = p.kv_len;

    const uint16_t* Qg = p.Q + (size_t)grp * R * D;
    const uint16_t* Kh = p.K + (size_t)grp * kv_len * D;
    const uint16_t* Vh = p.V + (size_t)grp * kv_len * D;

    const int row = rt * kPrefillRows + wave * 32 + (lane & 31);
    f16x8 qf[D / 16];
    load_q_frags<D>(Qg, row, R, lane, qf);

    if constexpr (D < 32) {
        // V^T rows D..31 pad the MFMA M dimension; keep them zero.
        for (int i = tid; i < 2 * (32 - D) * G::kVtStride; i += kPrefillThreads) {
            const int b = i / ((32 - D) * G::kVtStride);
            const int j = i % ((32 - D) * G::kVtStride);
            smem[b * G::kStageHalfs + G::kKHalfs + D * G::kVtStride + j] = (f16)0.f;
        }
    }

    StageLoader<D, BC, kPrefillThreads> ld;
    const int ntiles = (kv_len + BC - 1) / BC;
    ld.load(Kh, Vh, 0, kv_len, tid);
    ld.store(smem, smem + G::kKHalfs, tid);
    __syncthreads();

    RowState st{-INFINITY, -INFINITY, 0.f};
    f32x16 o[G::kNTD];
#pragma unroll
    for (int td = 0; td < G::kNTD; ++td) o[td] = f32x16{};

    for (int t = 0; t < ntiles; ++t) {
        const f16* Ks = smem + (t & 1) * G::kStageHalfs;
        const f16* Vt = Ks + G::kKHalfs;
        if (t + 1 < ntiles) ld.load(Kh, Vh, (t + 1) * BC, kv_len, tid);

        f32x16 s[G::kNSB];
#pragma unroll
        for (int sb = 0; sb < G::kNSB; ++sb) s[sb] = qk_block<D, BC>(Ks, 32 * sb, qf, lane);
        if ((t + 1) * BC > kv_len) {
            const int lim = kv_len - t * BC;
#pragma unroll
            for (int sb = 0; sb < G::kNSB; ++sb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (32 * sb + acc_row(r, lane) >= lim) s[sb][r] = -INFINITY;
        }
        f16x8 pb[2 * G::kNSB];
        softmax_update<G::kNSB, G::kNTD>(s, st, o, p.scale_log2, pb);
        pv_accum<D, BC, 2 * G::kNSB>(Vt, 0, pb, o, lane);

        if (t + 1 < ntiles) {
            f16* Kn = smem + ((t + 1) & 1) * G::kStageHalfs;
            ld.store(Kn, Kn + G::kKHalfs, tid);
        }
        __syncthreads();
    }

    // Epilogue: combine the two half-row partial sums, normalise, store.
    const float l = st.l + __shfl_xor(st.l, 32);
    if (row < R) {
        const float inv = 1.0f / l;
        float* Orow = p.O + ((size_t)grp * R + row) * D;
#pragma unroll
        for (int td = 0; td < G::kNTD; ++td)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 32 * td + 8 * i + 4 * g;
                if (d < D) {
                    f32x4 v = {o[td][4 * i] * inv, o[td][4 * i + 1] * inv,
                               o[td][4 * i + 2] * inv, o[td][4 * i + 3] * inv};
                    *reinterpret_cast<f32x4*>(Orow + d) = v;
                }
            }
        if (g == 0) {
            const size_t ri = (size_t)grp * R + row;
            if (p.Mi) p.Mi[ri] = st.rmax * p.scale;
            if (p.Li) p.Li[ri] = l * exp2_hw(st.m - st.rmax * p.scale_log2);
        }
    }
}

// ---------------------------------------------------------------------------
// Decode (split-KV): <= 32 query rows per KV head.  Workgroup = 4 waves on one
// (group, split); wave w streams 32-row stages w, w+4, w+8, ... of the split
// through its own LDS slot (single buffer, next stage prefetched into
// registers while the current one is computed; no workgroup barrier in the
// loop).  The 4 wave states merge in LDS at the end.
// ---------------------------------------------------------------------------
constexpr int kDecodeThreads = 256;
constexpr int kDecodeStage = 32;

template <int D> struct DecodeCfg { static constexpr int kWavesPerEU = D >= 256 ? 1 : 2; };

template <int D>
struct DecodeSmem {
    using G = StageGeom<D, kDecodeStage>;
    static constexpr int kOStride = D + 4;  // floats per merged-O row (padded)
    static constexpr int kStageBytes = 4 * G::kStageHalfs * 2;
    static constexpr int kMergeBytes = 4 * 32 * kOStride * 4 + 4 * 32 * 2 * 4;
    static constexpr int kBytes = kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes;
};

template <int D>
__global__ __launch_bounds__(kDecodeThreads, DecodeCfg<D>::kWavesPerEU)
void kf_attn_decode_kernel(AttnParams p) {
    using G = StageGeom<D, kDecodeStage>;
    using SM = DecodeSmem<D>;
    __shared__ __attribute__((aligned(16))) char smem_raw[SM::kBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 5;
    const int blk = xcd_remap(blockIdx.x, gridDim.x);
    const int split = blk % p.n_splits;
    const int grp = blk / p.n_splits;
    const int R = p.rows_per_group;
    const int kv_len = p.kv_len;
    const int s0 = split * p.kv_per_split;
    const int s1 = min(kv_len, s0 + p.kv_per_split);

    const uint16_t* Qg = p.Q + (size_t)grp * R * D;
    const uint16_t* Kh = p.K + (size_t)grp * kv_len * D;
    const uint16_t* Vh = p.V + (size_t)grp * kv_len * D;

    const int row = lane & 31;
    f16x8 qf[D / 16];
    load_q_frags<D>(Qg, row, R, lane, qf);

    f16* Ks = reinterpret_cast<f16*>(smem_raw) + wave * G::kStageHalfs;
    f16* Vt = Ks + G::kKHalfs;
    if constexpr (D < 32) {
        for (int i = lane; i < (32 - D) * G::kVtStride; i += 64) Vt[D * G::kVtStride + i] = (f16)0.f;
    }

    RowState st{-INFINITY, -INFINITY, 0.f};
    f32x16 o[G::kNTD];
#pragma unroll
    for (int td = 0; td < G::kNTD; ++td) o[td] = f32x16{};

    StageLoader<D, kDecodeStage, 64> ld;
    int kv0 = s0 + wave * kDecodeStage;
    if (kv0 < s1) ld.load(Kh, Vh, kv0, s1, lane);
    while (kv0 < s1) {
        wave_lds_sync();  // previous stage's LDS reads are done
        ld.store(Ks, Vt, lane);
        wave_lds_sync();
        const int kv_next = kv0 + 4 * kDecodeStage;
        if (kv_next < s1) ld.load(Kh, Vh, kv_next, s1, lane);

        f32x16 s[1];
        s[0] = qk_block<D, kDecodeStage>(Ks, 0, qf, lane);
        if (kv0 + kDecodeStage > s1) {
            const int lim = s1 - kv0;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (acc_row(r, lane) >= lim) s[0][r] = -INFINITY;
        }
        f16x8 pb[2];
        softmax_update<1, G::kNTD>(s, st, o, p.scale_log2, pb);
        pv_accum<D, kDecodeStage, 2>(Vt, 0, pb, o, lane);
        kv0 = kv_next;
    }

    // Rebase this wave's state onto its true max (natural-log scaled units).
    const float l_pair = st.l + __shfl_xor(st.l, 32);
    const bool empty = st.rmax == -INFINITY;
    const float m_nat = empty ? -INFINITY : st.rmax * p.scale;
    const float beta = empty ? 0.f : exp2_hw(st.m - st.rmax * p.scale_log2);

    __syncthreads();  // all waves are done with their stage slots
    float* Ob = reinterpret_cast<float*>(smem_raw);
    float* Mb = Ob + 4 * 32 * SM::kOStride;
    float* Lb = Mb + 4 * 32;
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

    // Merge the 4 wave states: thread -> (query row, kSeg-wide d segment).
    constexpr int kTpr = D / 4 < 8 ? D / 4 : 8;  // threads per query row
    constexpr int kSeg = D / kTpr;                // multiple of 4
    static_assert(kDecodeThreads / kTpr >= 32, "merge must cover 32 rows in one pass");
    const int mrow = tid / kTpr;
    const int seg = tid % kTpr;
    if (mrow < R) {
        float m = Mb[mrow];
#pragma unroll
        for (int w = 1; w < 4; ++w) m = fmaxf(m, Mb[w * 32 + mrow]);
        float wt[4];
        float l = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float mw = Mb[w * 32 + mrow];
            wt[w] = mw == -INFINITY ? 0.f : exp2_hw((mw - m) * kLog2e);
            l += wt[w] * Lb[w * 32 + mrow];
        }
        const bool final_out = p.n_splits == 1;
        const float inv = final_out ? 1.0f / l : 1.0f;
        // Final rows go to O; split partials to [grp][split][row][D].
        const size_t ri = (size_t)grp * R + mrow;
        const size_t pi = ((size_t)grp * p.n_splits + split) * R + mrow;
        float* dst = final_out ? p.O + ri * D : p.Opart + pi * D;
#pragma unroll
        for (int j = 0; j < kSeg; j += 4) {
            const int d = seg * kSeg + j;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(Ob + (w * 32 + mrow) * SM::kOStride + d);
                acc += wt[w] * v;
            }
            *reinterpret_cast<f32x4*>(dst + d) = acc * inv;
        }
        if (seg == 0) {
            if (final_out) {
                if (p.Mi) p.Mi[ri] = m;
                if (p.Li) p.Li[ri] = l;
            } else {
                p.Mpart[pi] = m;
                p.Lpart[pi] = l;
            }
        }
    }
    if (p.n_splits == 1) return;

    // Split-KV merge, fused: the last workgroup of this group to finish merges
    // every split's partial.  Release the partials device-wide (other XCDs'
    // L2s included), then take a ticket.
    __threadfence();
    __syncthreads();
    __shared__ int s_last;
    if (tid == 0) s_last = take_ticket(p.tickets + grp, p.epoch, p.n_splits);
    __syncthreads();
    if (!s_last) return;
    __threadfence();  // acquire: the other splits' partials are visible
    if (mrow < R) {
        const float* Mg = p.Mpart + (size_t)grp * p.n_splits * R + mrow;
        const float* Lg = p.Lpart + (size_t)grp * p.n_splits * R + mrow;
        const float* Og = p.Opart + ((size_t)grp * p.n_splits * R + mrow) * D + seg * kSeg;
        const int ns = p.n_splits;
        float m = -INFINITY;
        for (int k = 0; k < ns; ++k) m = fmaxf(m, Mg[(size_t)k * R]);
        float l = 0.f;
        f32x4 acc[kSeg / 4];
#pragma unroll
        for (int j = 0; j < kSeg / 4; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < ns; ++k) {
            const float w = exp2_hw((Mg[(size_t)k * R] - m) * kLog2e);
            l += w * Lg[(size_t)k * R];
            const float* ok = Og + (size_t)k * R * D;
#pragma unroll
            for (int j = 0; j < kSeg / 4; ++j) acc[j] += w * *reinterpret_cast<const f32x4*>(ok + 4 * j);
        }
        const float inv = 1.0f / l;
        const size_t ri = (size_t)grp * R + mrow;
        float* dst = p.O + ri * D + seg * kSeg;
#pragma unroll
        for (int j = 0; j < kSeg / 4; ++j) *reinterpret_cast<f32x4*>(dst + 4 * j) = acc[j] * inv;
        if (seg == 0) {
            if (p.Mi) p.Mi[ri] = m;
            if (p.Li) p.Li[ri] = l;
        }
    }
}

}  // namespace kf
