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
//       cached per host thread, device and stream and grown on demand; it is
//       never allocated inside a steady-state loop once the largest shape has
//       been seen on that stream.
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

// Split-KV workspace of the asynchronous launchers, cached per host thread,
// device and stream.  Launches queued on one stream run in order, so they can
// share a buffer; launches on two streams may run at the same time and
// launches on two devices need memory on their own device, so neither shares
// one.  A buffer is grown (freed and reallocated) only after its stream has
// drained.  Up to kMaxEntries (device, stream) pairs are kept per thread;
// beyond that the oldest is released after a synchronisation of its device.
// Entries are keyed by the stream handle: a stream destroyed while its
// launches still run may hand its handle to a new stream, which would then
// share the buffer, so synchronise a stream before destroying it.
struct WorkspaceCache {
    struct Entry {
        int device;
        hipStream_t stream;
        void* ptr;
        size_t bytes;
    };
    static constexpr int kMaxEntries = 16;
    Entry entries[kMaxEntries] = {};
    int count = 0;

    ~WorkspaceCache() {
        for (int i = 0; i < count; ++i)
            if (entries[i].ptr) (void)hipFree(entries[i].ptr);
    }

    // Drop entry i: its kernels may still run, so its device is drained
    // first (hipFree alone does not promise to wait for other streams).
    hipError_t release(int i) {
        int cur = 0;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (entries[i].ptr) {
            if ((e = hipSetDevice(entries[i].device)) != hipSuccess) return e;
            e = hipDeviceSynchronize();
            if (e == hipSuccess) e = hipFree(entries[i].ptr);
            const hipError_t e2 = hipSetDevice(cur);
            if (e != hipSuccess) return e;
            if (e2 != hipSuccess) return e2;
        }
        for (int j = i + 1; j < count; ++j) entries[j - 1] = entries[j];
        --count;
        return hipSuccess;
    }

    // A buffer of at least `need` bytes on the current device for `stream`
    // (nullptr and 0 when need is 0).
    hipError_t get(hipStream_t stream, size_t need, void** ptr, size_t* bytes) {
        *ptr = nullptr;
        *bytes = 0;
        if (need == 0) return hipSuccess;
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        Entry* en = nullptr;
        for (int i = 0; i < count && !en; ++i)
            if (entries[i].device == dev && entries[i].stream == stream) en = &entries[i];
        if (!en) {
            if (count == kMaxEntries && (e = release(0)) != hipSuccess) return e;
            en = &entries[count++];
            *en = Entry{dev, stream, nullptr, 0};
        }
        if (en->bytes < need) {
            if (en->ptr) {
                // Kernels queued on this stream may still read the old buffer.
                if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
                (void)hipFree(en->ptr);
                en->ptr = nullptr;
                en->bytes = 0;
            }
            if ((e = hipMalloc(&en->ptr, need)) != hipSuccess) return e;
            en->bytes = need;
        }
        *ptr = en->ptr;
        *bytes = en->bytes;
        return hipSuccess;
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
    void* ws = nullptr;
    size_t ws_bytes = 0;
    hipError_t e = kf::thread_workspace().get(stream, plan.workspace_bytes, &ws, &ws_bytes);
    if (e != hipSuccess) return e;
    st = kf_attn_fwd(Q, K, V, O, Mi, Li, B, q_len, kv_len, H_q, H_kv, D, ws, ws_bytes,
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
    void* ws = nullptr;
    size_t ws_bytes = 0;
    hipError_t e = thread_workspace().get(stream, plan.workspace_bytes, &ws, &ws_bytes);
    if (e != hipSuccess) return e;
    st = kf_attn_fwd_ex(Q, K, V, O, Mi, Li, B, q_len, kv_len, H_q, H_kv, D, kv_lens, flags,
                        ws, ws_bytes, static_cast<void*>(stream));
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
    void* ws = nullptr;
    size_t ws_bytes = 0;
    hipError_t e = thread_workspace().get(stream, need, &ws, &ws_bytes);
    if (e != hipSuccess) return e;
    const int st = kf_attn_decode_paged(Q, K_pages, V_pages, block_table, kv_lens, O, Mi, Li, B,
                                        q_len, H_q, H_kv, D, page_size, max_pages_per_seq,
                                        num_pages, flags, ws, ws_bytes,
                                        static_cast<void*>(stream));
    return status_to_hip(st);
}

}  // namespace kf
