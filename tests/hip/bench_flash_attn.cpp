// bench_flash_attn.cpp -- the reference's C++ benchmark (tests/bench_flash_attn.cu)
// switched over to libkf_attn.so, timed with HIP events.
//
// Same workload list, protocol and metrics as the reference bench:
//   * shapes: decode (Q_len = 1), short and long prefill, a head-dimension
//     sweep and MQA (tests/bench_flash_attn.cu:150-185);
//   * 5 untimed launches, then 50 launches between two HIP events on one
//     stream; latency = elapsed / 50 (:108-123);
//   * FLOPs 4 B H_q q_len kv_len D and bytes = fp16 Q, K, V + fp32 O
//     (:125-131);
//   * inputs U[-1, 1] from mt19937 with seeds 42 / 43 / 44, rounded to fp16
//     (:84-90).
// Launches go through the asynchronous launch_flash_attn overload of
// kf/flash_attn.hpp with caller-owned Mi / Li, like the reference's
// launch_once (:39-54).  Like the reference, every iteration re-reads the
// same K / V: the decode shapes here fit the 256 MB Infinity Cache, so their
// GB/s are cache figures (bench.py rotates input sets for HBM figures).
//
// Options (for the profiling targets of tests/hip/CMakeLists.txt, which
// profile one shape, as the reference's ncu targets profile one launch,
// tests/CMakeLists.txt:23-33):
//   --shape B,kv_len,H_q,H_kv,D[,q_len]   run that shape only (q_len 0 or
//                                          absent: q_len = kv_len);
//   --list   print every shape, one per line, as "B kv_len H_q H_kv D q_len
//            kernels_per_launch" (2 on the split paths: kernel + merge) and
//            exit without touching the GPU; rocprof_report.py uses it to
//            cut a kernel trace of the whole bench into its shapes.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "kf/flash_attn.hpp"

extern "C" unsigned short kf_oracle_float_to_half(float);

#define HIP_CHECK(expr)                                                                  \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess) {                                                          \
            std::fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__,         \
                         hipGetErrorString(e_));                                         \
            std::exit(EXIT_FAILURE);                                                     \
        }                                                                                \
    } while (0)

namespace {

constexpr int kWarmup = 5;
constexpr int kIters = 50;

struct Shape {
    int B, kv_len, H_q, H_kv, D, q_len;  // q_len 0: q_len = kv_len (prefill)
};

std::vector<uint16_t> uniform_fp16(size_t n, uint32_t seed) {
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    std::vector<uint16_t> out(n);
    for (auto& x : out) x = kf_oracle_float_to_half(dist(rng));
    return out;
}

template <typename T>
T* to_device(const std::vector<T>& h) {
    T* d = nullptr;
    HIP_CHECK(hipMalloc(&d, h.size() * sizeof(T)));
    HIP_CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

void bench(const Shape& s) {
    const int q_len = s.q_len > 0 ? s.q_len : s.kv_len;
    const size_t qn = (size_t)s.B * s.H_q * q_len * s.D;
    const size_t kvn = (size_t)s.B * s.H_kv * s.kv_len * s.D;
    const size_t rows = (size_t)s.B * s.H_q * q_len;

    uint16_t* dQ = to_device(uniform_fp16(qn, 42));
    uint16_t* dK = to_device(uniform_fp16(kvn, 43));
    uint16_t* dV = to_device(uniform_fp16(kvn, 44));
    float *dO, *dMi, *dLi;
    HIP_CHECK(hipMalloc(&dO, qn * sizeof(float)));
    HIP_CHECK(hipMalloc(&dMi, rows * sizeof(float)));
    HIP_CHECK(hipMalloc(&dLi, rows * sizeof(float)));

    hipStream_t stream;
    HIP_CHECK(hipStreamCreate(&stream));
    auto launch = [&] {
        HIP_CHECK(launch_flash_attn(dQ, dK, dV, dO, s.B, q_len, s.kv_len, s.H_q, s.H_kv, s.D,
                                    stream, dMi, dLi));
    };
    for (int i = 0; i < kWarmup; ++i) launch();
    HIP_CHECK(hipStreamSynchronize(stream));

    hipEvent_t t0, t1;
    HIP_CHECK(hipEventCreate(&t0));
    HIP_CHECK(hipEventCreate(&t1));
    HIP_CHECK(hipEventRecord(t0, stream));
    for (int i = 0; i < kIters; ++i) launch();
    HIP_CHECK(hipEventRecord(t1, stream));
    HIP_CHECK(hipEventSynchronize(t1));
    float total_ms = 0.f;
    HIP_CHECK(hipEventElapsedTime(&total_ms, t0, t1));
    const double ms = total_ms / kIters;

    const double flops = 4.0 * s.B * s.H_q * (double)q_len * s.kv_len * s.D;
    const double bytes = 2.0 * qn + 4.0 * kvn + 4.0 * qn;
    const double tflops = flops / (ms * 1e9);
    const double gbs = bytes / (ms * 1e6);
    if (q_len != s.kv_len)
        std::printf("  B=%-2d Q=%-4d KV=%-4d H_q=%-2d H_kv=%-2d D=%-3d | %8.4f ms | %8.2f TFLOPS | %8.1f GB/s\n",
                    s.B, q_len, s.kv_len, s.H_q, s.H_kv, s.D, ms, tflops, gbs);
    else
        std::printf("  B=%-2d S=%-4d         H_q=%-2d H_kv=%-2d D=%-3d | %8.4f ms | %8.2f TFLOPS | %8.1f GB/s\n",
                    s.B, s.kv_len, s.H_q, s.H_kv, s.D, ms, tflops, gbs);

    HIP_CHECK(hipEventDestroy(t0));
    HIP_CHECK(hipEventDestroy(t1));
    HIP_CHECK(hipStreamDestroy(stream));
    for (void* p : {(void*)dQ, (void*)dK, (void*)dV, (void*)dO, (void*)dMi, (void*)dLi})
        HIP_CHECK(hipFree(p));
}

}  // namespace

int main(int argc, char** argv) {
    bool list = false;
    Shape only{};
    bool have_only = false;
    for (int i = 1; i < argc; ++i) {
        if (std::strcmp(argv[i], "--list") == 0) {
            list = true;
        } else if (std::strcmp(argv[i], "--shape") == 0 && i + 1 < argc) {
            only.q_len = 0;
            const int n = std::sscanf(argv[++i], "%d,%d,%d,%d,%d,%d", &only.B, &only.kv_len, &only.H_q,
                                      &only.H_kv, &only.D, &only.q_len);
            if (n < 5) {
                std::fprintf(stderr, "--shape wants B,kv_len,H_q,H_kv,D[,q_len]\n");
                return EXIT_FAILURE;
            }
            have_only = true;
        } else {
            std::fprintf(stderr, "usage: %s [--list] [--shape B,kv_len,H_q,H_kv,D[,q_len]]\n", argv[0]);
            return EXIT_FAILURE;
        }
    }
    struct Group {
        const char* title;
        std::vector<Shape> shapes;
    };
    const Group groups[] = {
        {"decode: Q_len=1 (single new token), KV_len=full cache",
         {{1, 512, 32, 8, 128, 1}, {1, 1024, 32, 8, 128, 1}, {1, 2048, 32, 8, 128, 1},
          {1, 4096, 32, 8, 128, 1}, {8, 512, 32, 8, 128, 1}, {8, 1024, 32, 8, 128, 1}}},
        {"short-prefill: Q_len=KV_len, small S",
         {{1, 64, 32, 8, 128, 0}, {1, 128, 32, 8, 128, 0}, {1, 256, 32, 8, 128, 0},
          {8, 64, 32, 8, 128, 0}}},
        {"prefill: large S",
         {{1, 512, 32, 8, 128, 0}, {1, 1024, 32, 8, 128, 0}, {1, 2048, 32, 8, 128, 0},
          {1, 4096, 32, 8, 128, 0}}},
        {"head dim sweep: B=1 S=1024 H_q=32 H_kv=8",
         {{1, 1024, 32, 8, 64, 0}, {1, 1024, 32, 8, 128, 0}, {1, 1024, 32, 8, 256, 0}}},
        {"MQA: H_kv=1",
         {{1, 512, 32, 1, 128, 0}, {1, 1024, 32, 1, 128, 0}, {1, 512, 32, 1, 128, 1},
          {1, 1024, 32, 1, 128, 1}}},
    };
    if (list) {
        for (const Group& g : groups)
            for (const Shape& s : g.shapes) {
                const int q_len = s.q_len > 0 ? s.q_len : s.kv_len;
                kf_attn_plan_t pl;
                if (kf_attn_plan(s.B, q_len, s.kv_len, s.H_q, s.H_kv, s.D, &pl) != KF_OK) return EXIT_FAILURE;
                const bool split = pl.path == KF_PATH_DECODE_SPLIT || pl.path == KF_PATH_PREFILL_SPLIT;
                std::printf("%d %d %d %d %d %d %d\n", s.B, s.kv_len, s.H_q, s.H_kv, s.D, q_len, split ? 2 : 1);
            }
        return EXIT_SUCCESS;
    }
    std::printf("=== kernelfoundry_amd flash-attention benchmark, gfx950 (warmup=%d, iters=%d) ===\n",
                kWarmup, kIters);
    if (have_only) {
        std::printf("\n[--shape]\n");
        bench(only);
        return EXIT_SUCCESS;
    }
    for (const Group& g : groups) {
        std::printf("\n[%s]\n", g.title);
        for (const Shape& s : g.shapes) bench(s);
    }
    return EXIT_SUCCESS;
}
