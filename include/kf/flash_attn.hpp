// kf/flash_attn.hpp -- C++ host launchers with the reference's signatures.
//
// Header-only layer over the C ABI in kf/attn.h (link libkf_attn.so).  It
// keeps the call shapes of the reference harness so tests and benchmarks
// written against it compile unchanged apart from cuda* -> hip* types:
//
//   launch_flash_attn(Q, K, V, O, B, S, H_q, H_kv, D, stream)
//       tests/test_flash_attn.cu:52-59 -- synchronous, q_len == kv_len == S,
//       hipErrorInvalidValue for an unsupported D (:96-100).
//
//   launch_flash_attn(Q, K, V, O, B, q_len, kv_len, H_q, H_kv, D, stream, Mi, Li)
//       the asynchronous form the bench needs (tests/bench_flash_attn.cu:39-54:
//       separate q_len / kv_len, caller-owned Mi / Li).  Split-KV workspace is
//       cached per host thread and grown on demand; it is never allocated
//       inside a steady-state loop once the largest shape has been seen.
//
//   kf::attn_fwd_ex(...), kf::attn_decode_paged(...)
//       the same over kf_attn_fwd_ex / kf_attn_decode_paged (causal masking,
//       per-sequence key counts, paged K/V, fp16 / bf16 O, LSE), which have
//       no counterpart in the reference.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "kf/attn.h"

namespace kf {

// Map a kf_status to the hipError_t the reference launcher would return.
inline hipError_t status_to_hip(int st) {
    switch (st) {
        case KF_OK: return hipSuccess;
        case KF_ERR_HIP: return static_cast<hipError_t>(kf_last_hip_error());
        default: return hipErrorInvalidValue;
    }
}

// Per-thread cached workspace for the asynchronous launcher.
struct WorkspaceCache {
    void* ptr = nullptr;
    size_t bytes = 0;
    ~WorkspaceCache() {
        if (ptr) (void)hipFree(ptr);
    }
    hipError_t reserve(size_t need) {
        if (need <= bytes) return hipSuccess;
        if (ptr) {
            hipError_t e = hipDeviceSynchronize();
            if (e != hipSuccess) return e;
            (void)hipFree(ptr);
            ptr = nullptr;
            bytes = 0;
        }
        hipError_t e = hipMalloc(&ptr, need);
        if (e == hipSuccess) bytes = need;
        return e;
    }
};

inline WorkspaceCache& thread_workspace() {
    static thread_local WorkspaceCache cache;
    return cache;
}

}  // namespace kf

// Synchronous launcher with the reference signature (tests/test_flash_attn.cu:52-59).
inline hipError_t launch_flash_attn(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                                    float* O, int B, int S, int H_q, int H_kv, int D,
                                    hipStream_t stream = 0) {
    return static_cast<hipError_t>(
        kf_launch_flash_attn(Q, K, V, O, B, S, H_q, H_kv, D, static_cast<void*>(stream)));
}

// Asynchronous launcher with separate q_len / kv_len and optional Mi / Li.
inline hipError_t launch_flash_attn(const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                                    float* O, int B, int q_len, int kv_len, int H_q, int H_kv,
                                    int D, hipStream_t stream, float* Mi = nullptr,
                                    float* Li = nullptr) {
    kf_attn_plan_t plan;
    int st = kf_attn_plan(B, q_len, kv_len, H_q, H_kv, D, &plan);
    if (st != KF_OK) return kf::status_to_hip(st);
    kf::WorkspaceCache& ws = kf::thread_workspace();
    hipError_t e = ws.reserve(plan.workspace_bytes);
    if (e != hipSuccess) return e;
    st = kf_attn_fwd(Q, K, V, O, Mi, Li, B, q_len, kv_len, H_q, H_kv, D, ws.ptr, ws.bytes,
                     static_cast<void*>(stream));
    return kf::status_to_hip(st);
}

namespace kf {

// kf_attn_fwd_ex with the per-thread cached workspace: kv_lens (device int[B]
// or nullptr) and flags (KF_ATTN_CAUSAL, KF_ATTN_OUT_F16 / _BF16,
// KF_ATTN_LSE) as documented in kf/attn.h.
inline hipError_t attn_fwd_ex(const uint16_t* Q, const uint16_t* K, const uint16_t* V, void* O,
                              int B, int q_len, int kv_len, int H_q, int H_kv, int D,
                              const int* kv_lens, int flags, hipStream_t stream,
                              float* Mi = nullptr, float* Li = nullptr) {
    kf_attn_plan_t plan;
    int st = kf_attn_plan(B, q_len, kv_len, H_q, H_kv, D, &plan);
    if (st != KF_OK) return status_to_hip(st);
    WorkspaceCache& ws = thread_workspace();
    hipError_t e = ws.reserve(plan.workspace_bytes);
    if (e != hipSuccess) return e;
    st = kf_attn_fwd_ex(Q, K, V, O, Mi, Li, B, q_len, kv_len, H_q, H_kv, D, kv_lens, flags,
                        ws.ptr, ws.bytes, static_cast<void*>(stream));
    return status_to_hip(st);
}

// kf_attn_decode_paged with the per-thread cached workspace.
inline hipError_t attn_decode_paged(const uint16_t* Q, const uint16_t* K_pages,
                                    const uint16_t* V_pages, const int* block_table,
                                    const int* kv_lens, void* O, int B, int q_len, int H_q,
                                    int H_kv, int D, int page_size, int max_pages_per_seq,
                                    int num_pages, int flags, hipStream_t stream,
                                    float* Mi = nullptr, float* Li = nullptr) {
    const size_t need = kf_attn_decode_paged_workspace_bytes(B, q_len, H_q, H_kv, D, page_size,
                                                             max_pages_per_seq);
    WorkspaceCache& ws = thread_workspace();
    hipError_t e = ws.reserve(need);
    if (e != hipSuccess) return e;
    const int st = kf_attn_decode_paged(Q, K_pages, V_pages, block_table, kv_lens, O, Mi, Li, B,
                                        q_len, H_q, H_kv, D, page_size, max_pages_per_seq,
                                        num_pages, flags, ws.ptr, ws.bytes,
                                        static_cast<void*>(stream));
    return status_to_hip(st);
}

}  // namespace kf
