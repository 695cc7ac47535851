/*
 * cpu_attn.c -- brute-force CPU attention (TEST INFRASTRUCTURE ONLY).
 *
 * Restatement of the reference's host-side check, ``cpu_attn`` in
 * tests/test_flash_attn.cu:119-169: a scalar triple loop computing standard
 * scaled-dot-product attention with GQA grouping h_kv = h_q / (H_q / H_kv)
 * (tests/test_flash_attn.cu:138).  Generalised here to q_len != kv_len (the
 * reference's version assumes q_len == kv_len) and extended to also return
 * the row statistics the reference kernel writes (Mi = max_j s_ij,
 * Li = sum_j exp(s_ij - Mi); kernels/flash_attn.cu:559-579).
 *
 * Two precisions: ``kf_oracle_attn_f32`` keeps the reference's fp32
 * arithmetic and loop order; ``kf_oracle_attn_f64`` is the same loop in
 * double and serves as the high-precision check.
 *
 * Only tests/ and the HIP test harness link this file, as the checker.  The
 * product library never does.
 */
#include <math.h>
#include <stddef.h>
#include <stdlib.h>

#define KF_ORACLE_DEFINE(NAME, T, EXP, SQRT)                                      \
int NAME(const T* Q, const T* K, const T* V, T* O, T* Mi, T* Li,               \
         int B, int q_len, int kv_len, int H_q, int H_kv, int D) {            \
    if (B <= 0 || q_len <= 0 || kv_len <= 0 || H_q <= 0 || H_kv <= 0 ||       \
        D <= 0 || (H_q % H_kv) != 0)                                          \
        return 1;                                                              \
    const T scale = (T)1 / SQRT((T)D);                                         \
    const int ratio = H_q / H_kv;                                              \
    T* scores = (T*)malloc(sizeof(T) * (size_t)kv_len);                        \
    if (!scores) return 2;                                                     \
    for (int b = 0; b < B; ++b) {                                              \
        for (int h = 0; h < H_q; ++h) {                                        \
            const int hk = h / ratio;                                          \
            const T* Kh = K + ((size_t)b * H_kv + hk) * (size_t)kv_len * D;    \
            const T* Vh = V + ((size_t)b * H_kv + hk) * (size_t)kv_len * D;    \
            for (int i = 0; i < q_len; ++i) {                                  \
                const size_t row = ((size_t)b * H_q + h) * (size_t)q_len + i;  \
                const T* q = Q + row * D;                                      \
                T mx = -INFINITY;                                              \
                for (int j = 0; j < kv_len; ++j) {                             \
                    const T* k = Kh + (size_t)j * D;                           \
                    T dot = 0;                                                 \
                    for (int d = 0; d < D; ++d) dot += q[d] * k[d];            \
                    scores[j] = dot * scale;                                   \
                    if (scores[j] > mx) mx = scores[j];                        \
                }                                                              \
                T sum = 0;                                                     \
                for (int j = 0; j < kv_len; ++j) {                             \
                    scores[j] = EXP(scores[j] - mx);                           \
                    sum += scores[j];                                          \
                }                                                              \
                T* o = O + row * D;                                            \
                for (int d = 0; d < D; ++d) o[d] = 0;                          \
                for (int j = 0; j < kv_len; ++j) {                             \
                    const T p = scores[j] / sum;                               \
                    const T* v = Vh + (size_t)j * D;                           \
                    for (int d = 0; d < D; ++d) o[d] += p * v[d];              \
                }                                                              \
                if (Mi) Mi[row] = mx;                                          \
                if (Li) Li[row] = sum;                                         \
            }                                                                  \
        }                                                                      \
    }                                                                          \
    free(scores);                                                              \
    return 0;                                                                  \
}

KF_ORACLE_DEFINE(kf_oracle_attn_f32, float, expf, sqrtf)
KF_ORACLE_DEFINE(kf_oracle_attn_f64, double, exp, sqrt)

/* IEEE binary16 bits -> float, exact (every half is representable). */
float kf_oracle_half_to_float(unsigned short h) {
    const unsigned sign = (h >> 15) & 1u;
    const unsigned exp = (h >> 10) & 0x1Fu;
    const unsigned man = h & 0x3FFu;
    float v;
    if (exp == 0)
        v = ldexpf((float)man, -24);
    else if (exp == 31)
        v = man ? NAN : INFINITY;
    else
        v = ldexpf((float)(man | 0x400u), (int)exp - 25);
    return sign ? -v : v;
}

/* float -> IEEE binary16 bits with round-to-nearest-even (the conversion of
 * __float2half used at tests/test_flash_attn.cu:173-178). */
unsigned short kf_oracle_float_to_half(float f) {
    union { float f; unsigned u; } x = { f };
    const unsigned sign = (x.u >> 16) & 0x8000u;
    const unsigned absu = x.u & 0x7FFFFFFFu;
    if (absu >= 0x7F800000u)                       /* inf or nan */
        return (unsigned short)(sign | 0x7C00u | (absu > 0x7F800000u ? 0x200u : 0u));
    if (absu >= 0x477FF000u)                       /* rounds to >= 65520: inf */
        return (unsigned short)(sign | 0x7C00u);
    if (absu < 0x33000001u)                        /* <= 2^-25: rounds to 0 */
        return (unsigned short)sign;
    int e = (int)(absu >> 23) - 127;
    unsigned man = (absu & 0x7FFFFFu) | 0x800000u;  /* 24-bit significand */
    int shift;                                     /* bits to drop */
    unsigned base;
    if (e < -14) {                                 /* subnormal half */
        shift = 13 + (-14 - e);
        base = 0;
    } else {
        shift = 13;
        base = (unsigned)(e + 15) << 10;
        man &= 0x7FFFFFu;                          /* drop the implicit bit */
    }
    unsigned q = man >> shift;
    const unsigned rem = man & ((1u << shift) - 1u);
    const unsigned half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (unsigned short)(sign | (base + q));    /* carry propagates into exp */
}
