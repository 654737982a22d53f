/*
 * Plain-C restatement of the INT4 layouts and the dequantised W4A16 product.
 * TEST INFRASTRUCTURE ONLY (see oracle/__init__.py); written independently of the
 * numpy restatement in oracle/int4.py so the two can check each other.
 *
 * GPTQ qweight int32 [K/8][N]: q[k][n] = (qweight[k/8][n] >> 4*(k%8)) & 15.
 * Prepacked int32 [N/16][K/64][32][4]: entry l, word w of block kc of 16-column slice s is
 * the GPTQ word of k-group 8*kc + 4*(l/16) + w, column 16*s + l%16, with nibble p holding
 * k-offset perm[p] = {0,2,4,6,1,3,5,7}[p].
 * dequant: fp16((q - z) * s) -- computed here from the fp16 bit pattern of s by exact
 * integer arithmetic and an explicit round-to-nearest-even to fp16.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static const int kPerm[8] = {0, 2, 4, 6, 1, 3, 5, 7};

void oracle_int4_pack_gptq(const uint8_t* q, int K, int N, int32_t* qweight) {
    for (int kg = 0; kg < K / 8; ++kg)
        for (int n = 0; n < N; ++n) {
            uint32_t w = 0;
            for (int j = 0; j < 8; ++j) w |= (uint32_t)(q[(size_t)(kg * 8 + j) * N + n] & 15u) << (4 * j);
            qweight[(size_t)kg * N + n] = (int32_t)w;
        }
}

void oracle_int4_prepack(const int32_t* qweight, int K, int N, int32_t* out) {
    const int KC = K / 64, NS = N / 16;
    size_t idx = 0;
    for (int s = 0; s < NS; ++s)
        for (int kc = 0; kc < KC; ++kc)
            for (int l = 0; l < 32; ++l)
                for (int w = 0; w < 4; ++w) {
                    const int kg = 8 * kc + 4 * (l / 16) + w;
                    const int n = 16 * s + l % 16;
                    const uint32_t src = (uint32_t)qweight[(size_t)kg * N + n];
                    uint32_t dst = 0;
                    for (int p = 0; p < 8; ++p) dst |= ((src >> (4 * kPerm[p])) & 15u) << (4 * p);
                    out[idx++] = (int32_t)dst;
                }
}

/* fp16 bits -> double (exact). */
static double half_to_double(uint16_t h) {
    const int sign = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 1024), e - 25);
    return sign ? -v : v;
}

/* double -> fp16 bits, round to nearest even (finite inputs well inside range). */
static uint16_t double_to_half(double x) {
    uint16_t sign = 0;
    if (x < 0) { sign = 0x8000; x = -x; }
    if (x == 0) return sign;
    int e;
    double fr = frexp(x, &e);      /* x = fr * 2^e, fr in [0.5, 1) */
    int exp16 = e - 1 + 15;         /* biased exponent for 1.f form */
    double scaled;
    if (exp16 <= 0) {               /* subnormal: units of 2^-24 */
        scaled = ldexp(x, 24);
        exp16 = 0;
    } else {
        scaled = ldexp(fr, 11);     /* 11-bit significand in [1024, 2048) */
    }
    double fl = floor(scaled);
    double rem = scaled - fl;
    uint32_t mant = (uint32_t)fl;
    if (rem > 0.5 || (rem == 0.5 && (mant & 1u))) mant++;
    if (exp16 == 0) {
        if (mant >= 1024) return sign | (uint16_t)(1u << 10) | (uint16_t)(mant - 1024);
        return sign | (uint16_t)mant;
    }
    if (mant == 2048) { mant = 1024; exp16++; }
    if (exp16 >= 31) return sign | 0x7c00;
    return sign | (uint16_t)(exp16 << 10) | (uint16_t)(mant - 1024);
}

/* W[k][n] as fp16 bits; zeros unpacked uint8 [K/G][N]; scales fp16 bits [K/G][N]. */
void oracle_int4_dequant(const uint8_t* q, const uint16_t* scales, const uint8_t* zeros, int K, int N,
                         int G, uint16_t* W) {
    for (int k = 0; k < K; ++k)
        for (int n = 0; n < N; ++n) {
            const size_t gi = (size_t)(k / G) * N + n;
            const double d = (double)((int)q[(size_t)k * N + n] - (int)zeros[gi]);
            W[(size_t)k * N + n] = double_to_half(d * half_to_double(scales[gi]));
        }
}

/* Y[M][N] = A[M][K] (fp16 bits) @ W (fp16 bits), fp32 sequential accumulation. */
void oracle_w4a16(const uint16_t* A, const uint16_t* W, int M, int N, int K, float* Y) {
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k)
                acc += (float)half_to_double(A[(size_t)m * K + k]) * (float)half_to_double(W[(size_t)k * N + n]);
            Y[(size_t)m * N + n] = acc;
        }
}
