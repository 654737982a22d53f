/*
 * Plain-C restatement of the reference GEMM path.  TEST INFRASTRUCTURE ONLY.
 *
 *   C_out = alpha * (A @ B) + beta * C_in,   A [M][K], B [K][N] fp16 (bit patterns),
 *   FP32 accumulation in k order, C_in read only when beta != 0 and C_in != NULL
 *   (wmma_gemm.hip:636-666, 1912-1924).  Split-K: k_per_split = ceil(K/split), partials
 *   summed in split order (wmma_xor_swizzle.hpp:293-353).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

static float h2f(uint16_t h) {
    const int sign = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 1024), e - 25);
    return (float)(sign ? -v : v);
}

void oracle_gemm(const uint16_t* A, const uint16_t* B, const float* C_in, float* C_out, int M, int N,
                 int K, float alpha, float beta, int split) {
    if (split < 1) split = 1;
    const int kps = (K + split - 1) / split;
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float total = 0.0f;
            for (int s = 0; s < split; ++s) {
                const int k0 = s * kps, k1 = (k0 + kps < K) ? k0 + kps : K;
                float part = 0.0f;
                for (int k = k0; k < k1; ++k) part += h2f(A[(size_t)i * K + k]) * h2f(B[(size_t)k * N + j]);
                total = (s == 0) ? part : total + part;
            }
            float r = alpha * total;
            if (beta != 0.0f && C_in) r += beta * C_in[(size_t)i * N + j];
            C_out[(size_t)i * N + j] = r;
        }
}
