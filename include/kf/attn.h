/*
 * kf/attn.h -- C ABI of the MI355X (gfx950) flash-attention forward.
 *
 * This is the drop-in boundary for the reference's attention launchers:
 *   - launch_flash_attn      tests/test_flash_attn.cu:52-113  (synchronous,
 *                            q_len == kv_len == S, launcher-owned scratch)
 *   - launch_once            tests/bench_flash_attn.cu:39-54  (asynchronous,
 *                            separate q_len / kv_len, caller-owned Mi / Li)
 *   - flash_attn_kernel<D>   kernels/flash_attn.cu:384-398    (the device
 *                            entry those launchers wrap; not exported here)
 *
 * Plain C types only: device pointers, sizes and an opaque stream handle
 * (a hipStream_t passed as void*; NULL is the default stream).  No C++
 * exceptions cross this boundary; every entry point returns a status code.
 *
 * Tensor layout contract (identical to the reference's, flash_attn.cu:364-370):
 *   Q  [B, H_q,  q_len,  D]  fp16 bits (uint16_t), contiguous row-major
 *   K  [B, H_kv, kv_len, D]  fp16 bits
 *   V  [B, H_kv, kv_len, D]  fp16 bits
 *   O  [B, H_q,  q_len,  D]  fp32
 *   Mi [B, H_q,  q_len]      fp32, optional: max_j s_ij over the scaled scores
 *                            s = q.k / sqrt(D)
 *   Li [B, H_q,  q_len]      fp32, optional: sum_j exp(s_ij - Mi)
 * Query head h_q reads KV head h_q / (H_q / H_kv) (flash_attn.cu:406); H_q
 * must be a multiple of H_kv (the reference silently mis-groups otherwise).
 * kf_attn_fwd is non-causal with softmax scale 1/sqrt(D), as in the
 * reference; kf_attn_fwd_ex adds causal masking and per-sequence key
 * counts (ranked next steps of the reference's own roadmap,
 * docs/flash_attn.md:105 and reference_benchmarks/bench_flash_attn2.py:115-150).
 * D must be one of the reference's instantiations
 * {16, 64, 128, 256} (flash_attn.cu:587-600).  All device pointers must be
 * 16-byte aligned.
 */
#ifndef KF_ATTN_H
#define KF_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by the kf_* entry points. */
enum kf_status {
    KF_OK = 0,
    KF_ERR_HEAD_DIM = 1,   /* D is not 16, 64, 128 or 256                      */
    KF_ERR_GQA = 2,        /* H_q is not a positive multiple of H_kv            */
    KF_ERR_SIZE = 3,       /* a size is <= 0 or overflows the kernels' indexing */
    KF_ERR_NULL = 4,       /* a required pointer is NULL                        */
    KF_ERR_WORKSPACE = 5,  /* workspace missing or smaller than required        */
    KF_ERR_ALIGN = 6,      /* a device pointer is not 16-byte aligned           */
    KF_ERR_HIP = 7,        /* a HIP runtime call failed: kf_last_hip_error()    */
    KF_ERR_FLAGS = 8,      /* unknown bits in `flags`, or F16 and BF16 together  */
    KF_ERR_SCRATCH = 9     /* kf_attn_fwd_noalloc: shape needs more scratch than
                              its static maximum                                 */
};

/* kf_attn_fwd_ex / kf_attn_decode_paged flags. */
#define KF_ATTN_CAUSAL 1   /* query i sees keys j <= i + kv_b - q_len           */
#define KF_ATTN_OUT_F16 2  /* O is written as fp16 (RNE of the fp32 result)     */
#define KF_ATTN_OUT_BF16 4 /* O is written as bf16 (RNE of the fp32 result)     */
#define KF_ATTN_LSE 8      /* row_max receives LSE = Mi + ln(Li) (natural log;
                              -inf for a row without keys); row_sumexp unused */

/* Which kernels kf_attn_fwd runs for a shape (see kf_attn_plan). */
enum kf_path {
    KF_PATH_PREFILL = 0,   /* MFMA prefill kernel, one pass over KV             */
    KF_PATH_DECODE = 1,    /* split-KV decode kernel, writes final O directly   */
    KF_PATH_DECODE_SPLIT = 2, /* split-KV decode kernel + split-merge kernel     */
    KF_PATH_PREFILL_SPLIT = 3 /* MFMA prefill kernel over KV partitions (few query
                                 rows, many keys) + split-merge kernel          */
};

typedef struct kf_attn_plan_t {
    int path;              /* enum kf_path                                      */
    int rows_per_group;    /* H_q / H_kv * q_len query rows per KV head         */
    int num_splits;        /* KV partitions per (b, h_kv); 1 = unsplit          */
    int kv_per_split;      /* KV rows per partition                             */
    int grid_blocks;       /* workgroups of the main kernel                     */
    int block_threads;     /* threads per workgroup of the main kernel          */
    size_t workspace_bytes;/* bytes kf_attn_fwd needs in `workspace`            */
    int splits_per_block;  /* decode: KV partitions per workgroup (4 = the
                              short-split kernel, one partition per wave;
                              1 = the streaming decode kernel); 0 on prefill    */
} kf_attn_plan_t;

/* Describe the dispatch kf_attn_fwd would use on the device current on the
 * calling thread.  Validates like kf_attn_fwd (sizes only, no pointers).
 * The plan is sized for that device's compute units and XCDs, read once per
 * device with hipDeviceGetAttribute (the reference's launcher likewise sizes
 * its launch from the device, tests/test_flash_attn.cu:28-48); without a
 * visible device it is the plan for a whole MI355X (256 CUs, 8 XCDs).
 * kf_attn_fwd, kf_attn_fwd_ex, kf_attn_decode_paged and the workspace
 * queries plan the same way, so a workspace sized on the current device fits
 * calls on streams of that device. */
int kf_attn_plan(int B, int q_len, int kv_len, int H_q, int H_kv, int D,
                 kf_attn_plan_t* plan);

/* The plan for a device with num_cus compute units (no device query; for
 * planning ahead and for host-only tests).  No reference counterpart.
 * num_cus <= 0 -> KF_ERR_SIZE. */
int kf_attn_plan_for_cus(int B, int q_len, int kv_len, int H_q, int H_kv, int D, int num_cus,
                         kf_attn_plan_t* plan);

/* Names of the kernels kf_attn_fwd_ex launches for this shape on the current
 * device, in launch order and as a profiler lists them, e.g.
 * "kf_attn_prefill_kernel<128, false, 8, 1>" or
 * "kf_attn_decode_short_kernel<128, 1> + kf_attn_split_merge_kernel<128, 8, 4>";
 * `flags` (KF_ATTN_CAUSAL) and whether kv_lens is non-NULL (never read) pick
 * the masked prefill.  NUL-terminated into buf; KF_ERR_SIZE if buf_bytes is
 * too small.  No reference counterpart (its launchers print the launch
 * geometry, tests/test_flash_attn.cu:86-91). */
int kf_attn_kernel_names(int B, int q_len, int kv_len, int H_q, int H_kv, int D, int flags,
                         const int* kv_lens, char* buf, size_t buf_bytes);

/* Bytes of device workspace kf_attn_fwd needs for this shape (0 when the
 * shape runs without split-KV partials: split decode and split prefill need
 * them).  Returns 0 for invalid shapes too;
 * kf_attn_plan reports why. */
size_t kf_attn_workspace_bytes(int B, int q_len, int kv_len, int H_q, int H_kv, int D);

/* Attention forward, asynchronous on `stream`.
 *
 * Replaces launch_once (tests/bench_flash_attn.cu:39-54) and the kernel
 * launch inside launch_flash_attn (tests/test_flash_attn.cu:92-93):
 * separate q_len / kv_len (q_len = 1 is decode), optional Mi / Li outputs
 * (row_max / row_sumexp may be NULL), caller-owned workspace of at least
 * kf_attn_workspace_bytes() bytes (may be NULL when that is 0; 256-byte
 * aligned).  The workspace needs no initialisation; it must not be shared by
 * calls that can run concurrently (e.g. on two streams).  Only split decode
 * (KF_PATH_DECODE_SPLIT) requires it: a split prefill (KF_PATH_PREFILL_SPLIT)
 * given no workspace, or a smaller one, runs with as many KV partitions as
 * that workspace holds, or unsplit, instead of failing (its results then
 * differ in the last bits, within the same tolerance).
 * Validation happens before any HIP call; an invalid argument returns its
 * status code and launches nothing.  Unlike launch_once, which silently
 * does nothing for an unsupported D (bench_flash_attn.cu:48-52), this
 * returns KF_ERR_HEAD_DIM. */
int kf_attn_fwd(const void* Q, const void* K, const void* V, float* O,
                float* row_max, float* row_sumexp,
                int B, int q_len, int kv_len, int H_q, int H_kv, int D,
                void* workspace, size_t workspace_bytes, void* stream);

/* kf_attn_fwd with key masking; kf_attn_fwd(...) == kf_attn_fwd_ex(...,
 * NULL, 0, ...).  No counterpart in the reference, which has neither
 * (flash_attn.cu:384-585 is non-causal over all kv_len keys).
 *
 * kv_lens: NULL, or a device array [B] of int (4-byte aligned): sequence b
 *   uses only its first kv_b = kv_lens[b] keys (clamped to [0, kv_len]) of
 *   the kv_len rows allocated per head in K / V -- a pre-allocated KV cache
 *   filled to different lengths.
 * flags & KF_ATTN_CAUSAL: query i (0 <= i < q_len) of sequence b sees keys
 *   j <= i + kv_b - q_len, i.e. the mask is aligned to the bottom-right
 *   corner (the last query sees every key; with q_len == kv_len it is the
 *   usual lower triangle; q_len = 1 decode is unaffected).
 * A query row that sees no key (kv_b = 0, or causal rows with
 * i + kv_b - q_len < 0) gets O = 0, Mi = -inf, Li = 0.
 * O is fp32 [B, H_q, q_len, D] unless flags select KF_ATTN_OUT_F16 or
 * KF_ATTN_OUT_BF16 (then 2-byte elements, still 16-byte aligned; the
 * reference's PyTorch comparator outputs fp16, bench_flash_attn2.py:11-12);
 * KF_ATTN_LSE replaces the (Mi, Li) pair by one log-sum-exp per row in
 * row_max.  KF_ATTN_OUT_F16 | KF_ATTN_OUT_BF16 -> KF_ERR_FLAGS.  Shapes, workspace
 * and the kernels chosen are those of kf_attn_fwd (kf_attn_plan,
 * kf_attn_workspace_bytes apply unchanged). */
int kf_attn_fwd_ex(const void* Q, const void* K, const void* V, void* O,
                   float* row_max, float* row_sumexp,
                   int B, int q_len, int kv_len, int H_q, int H_kv, int D,
                   const int* kv_lens, int flags,
                   void* workspace, size_t workspace_bytes, void* stream);

/* kf_attn_fwd_ex without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference.
 *
 * The split-KV partials go to a static device array of the library, one per
 * device, of kf_attn_noalloc_scratch_bytes() bytes (16 MiB), held until the
 * process ends; the call makes no hipMalloc / hipFree or any other allocation.
 * Its address is resolved on the first call on each device (with that device
 * current on the calling thread) and kept for the life of the process; a
 * hipDeviceReset() of that device unloads the array, so the call must not be
 * used again on a device after resetting it.  Flag, pointer and alignment
 * errors are reported as by kf_attn_fwd_ex, before any scratch check.  A
 * shape whose plan needs more than that
 * (kf_attn_workspace_bytes) returns KF_ERR_SCRATCH and launches nothing,
 * except a split prefill (KF_PATH_PREFILL_SPLIT), which is planned with as
 * many KV partitions as the scratch holds -- possibly fewer than
 * kf_attn_fwd_ex takes, in which case the results differ from its in the
 * last bits (both within the same tolerance of the exact result).
 * Every call on one device shares that device's array: calls that can run
 * concurrently on one device (two streams, two threads) race on it and must
 * be serialised by the caller; consecutive calls on one stream are safe.  The
 * kernels need no initialised scratch.  Arguments otherwise as kf_attn_fwd_ex. */
int kf_attn_fwd_noalloc(const void* Q, const void* K, const void* V, void* O,
                        float* row_max, float* row_sumexp,
                        int B, int q_len, int kv_len, int H_q, int H_kv, int D,
                        const int* kv_lens, int flags, void* stream);

/* Size of kf_attn_fwd_noalloc's static per-device scratch (bytes). */
size_t kf_attn_noalloc_scratch_bytes(void);

/* Decode over a paged K/V cache, the block-table gather fused into the
 * split-KV decode kernel.  Replaces the gather + attention of the
 * reference's paged comparison (reference_benchmarks/bench_flash_attn2.py:
 * 153-215: pools [pool_blocks, H_kv, block_size, D], block ids per page),
 * which it names as the job of a specialised paged-attention kernel; the
 * reference has no such kernel.
 *
 * K_pages, V_pages: [num_pages, H_kv, page_size, D] fp16 page pools.
 * block_table: device int [B, max_pages_per_seq]; key j of sequence b is row
 *   j % page_size of page block_table[b * max_pages_per_seq + j / page_size].
 *   An id outside [0, num_pages) contributes no keys: the kernel never reads
 *   outside the pools.
 * kv_lens: device int [B], keys of each sequence, clamped to
 *   [0, max_pages_per_seq * page_size]; required.
 * page_size: a power of two in [16, 2^20].
 * Q, O, row_max, row_sumexp, flags (KF_ATTN_CAUSAL) as in kf_attn_fwd_ex,
 * with kv_len = max_pages_per_seq * page_size.  The decode path only: at
 * most 32 query rows per KV head ((H_q / H_kv) * q_len <= 32), else
 * KF_ERR_SIZE.  Workspace: kf_attn_decode_paged_workspace_bytes() bytes,
 * 256-byte aligned, no initialisation. */
size_t kf_attn_decode_paged_workspace_bytes(int B, int q_len, int H_q, int H_kv, int D,
                                            int page_size, int max_pages_per_seq);
int kf_attn_decode_paged(const void* Q, const void* K_pages, const void* V_pages,
                         const int* block_table, const int* kv_lens,
                         void* O, float* row_max, float* row_sumexp,
                         int B, int q_len, int H_q, int H_kv, int D,
                         int page_size, int max_pages_per_seq, int num_pages, int flags,
                         void* workspace, size_t workspace_bytes, void* stream);

/* The reference launcher's contract (tests/test_flash_attn.cu:52-113):
 * q_len = kv_len = S, scratch allocated and freed by the call, stream
 * synchronised before returning.  Returns a hipError_t value:
 * hipSuccess (0), hipErrorInvalidValue for an unsupported D or an invalid
 * shape, or the HIP error of a failed allocation / launch / sync. */
int kf_launch_flash_attn(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                         float* O, int B, int S, int H_q, int H_kv, int D,
                         void* stream);

/* Human-readable text for a kf_status value (static storage). */
const char* kf_status_string(int status);

/* hipError_t of the last failed HIP call made by a kf_* entry point on the
 * calling thread (0 if none). */
int kf_last_hip_error(void);

/* Library version string. */
const char* kf_version(void);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* KF_ATTN_H */
