// probe.hip -- measurement probes of libkf_probe.so (used by bench.py; not
// part of the attention library or its ABI; declared in probe.h beside it).
//
// The decode of BASELINE configs[1] (B = 1, KV = 4096) moves 16.8 MB, which
// HBM delivers in ~2 us: the step is bounded by what one kernel launch and
// one memory round trip cost, not by bandwidth.  These probes measure those
// two floors on the same device and the same buffers:
//   kf_probe_read   reads two buffers once with 16-byte loads, every load
//                   issued before the first use (one round trip per lane), and
//                   writes nothing unless the data XORs to a magic value --
//                   the fastest kernel that reads the decode's K and V;
//   kf_probe_empty  an empty dispatch (one wave): back to back, the cost of a
//                   kernel boundary on one stream.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "probe.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kReadThreads = 256;
constexpr int kReadChunks = 4;  // 16-byte chunks per thread and buffer

__global__ __launch_bounds__(kReadThreads) void kf_probe_read_kernel(const u32x4* __restrict__ a,
                                                                     const u32x4* __restrict__ b,
                                                                     size_t chunks,
                                                                     unsigned* __restrict__ sink) {
    const size_t base = (size_t)blockIdx.x * kReadThreads * kReadChunks + threadIdx.x;
    u32x4 va[kReadChunks], vb[kReadChunks];
#pragma unroll
    for (int i = 0; i < kReadChunks; ++i) {
        const size_t c = base + (size_t)i * kReadThreads;
        const size_t cc = c < chunks ? c : chunks - 1;  // in bounds, unpredicated
        va[i] = __builtin_nontemporal_load(a + cc);
        vb[i] = __builtin_nontemporal_load(b + cc);
    }
    unsigned x = 0;
#pragma unroll
    for (int i = 0; i < kReadChunks; ++i) x ^= va[i].x ^ va[i].y ^ va[i].z ^ va[i].w ^ vb[i].x ^ vb[i].y ^ vb[i].z ^ vb[i].w;
    if (x == 0x9e3779b9u) sink[0] = x;  // keeps the loads; practically never taken
}

__global__ __launch_bounds__(64) void kf_probe_empty_kernel() {}

}  // namespace

extern "C" {

int kf_probe_read(const void* a, const void* b, size_t bytes_each, unsigned* sink, void* stream) {
    if (!a || !b || !sink || bytes_each < 16 || (bytes_each & 15) != 0) return 1;
    if (((uintptr_t)a & 15) != 0 || ((uintptr_t)b & 15) != 0) return 1;
    const size_t chunks = bytes_each / 16;
    const size_t per_block = (size_t)kReadThreads * kReadChunks;
    const size_t blocks = (chunks + per_block - 1) / per_block;
    if (blocks > 0x7fffffff) return 1;
    (void)hipGetLastError();
    kf_probe_read_kernel<<<dim3((unsigned)blocks), dim3(kReadThreads), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const u32x4*>(a), static_cast<const u32x4*>(b), chunks, sink);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

int kf_probe_empty(void* stream) {
    (void)hipGetLastError();
    kf_probe_empty_kernel<<<dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream)>>>();
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
