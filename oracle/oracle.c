/*
 * CPU restatement of the reference's W4A16 arithmetic -- TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline);
 * no product code path calls it.
 *
 * Restates (reference = chris320211/Nibble):
 *   oracle_pack_int4          w4a16/quantization.py:4-28
 *   oracle_unpack_int4        w4a16/quantization.py:31-63
 *   oracle_quantize_groupwise w4a16/quantization.py:65-102
 *   oracle_dequantize_f32     w4a16/reference.py:6-46
 *   oracle_dequantize_f16     w4a16/reference.py:6-46 + .to(torch.float16)
 *                             (the contract of csrc/int4_linear_kernel.cu:412-418)
 *   oracle_linear             w4a16/reference.py:49-80
 *   oracle_f32_to_f16 / oracle_f16_to_f32: IEEE 754 binary16 conversions
 *                             (round to nearest even, subnormals, inf, nan)
 *
 * Each function is pinned in tests/test_oracle.py against the reference's
 * known-answer vectors (tests/golden/kat.json) and closed forms computed
 * independently with numpy.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- binary16 */

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: man * 2^-24, exact in fp32 */
            float f = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) { /* inf / nan (nan keeps a quiet payload bit) */
        if (man == 0) return sign | 0x7C00u;
        return sign | 0x7E00u | (uint16_t)(man >> 13);
    }
    const int e = (int)exp - 127; /* unbiased */
    if (e > 15) return sign | 0x7C00u;
    if (e >= -14) { /* normal range of binary16 */
        uint32_t hm = man >> 13;
        const uint32_t rest = man & 0x1FFFu;
        uint32_t he = (uint32_t)(e + 15);
        if (rest > 0x1000u || (rest == 0x1000u && (hm & 1u))) {
            hm += 1;
            if (hm == 0x400u) {
                hm = 0;
                he += 1;
                if (he == 31) return sign | 0x7C00u;
            }
        }
        return sign | (uint16_t)(he << 10) | (uint16_t)hm;
    }
    /* subnormal or zero: value = full * 2^(e-23), full = 1.man (24 bits);
       binary16 subnormal unit = 2^-24, so the count is full >> (-e - 1) */
    if (e < -25) return sign; /* below half the smallest subnormal */
    const uint32_t full = man | 0x800000u;
    const int shift = -e - 1; /* 14..24 */
    uint32_t q = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1; /* may carry into the smallest normal: correct */
    return sign | (uint16_t)q;
}

/* ------------------------------------------------------------- pack/unpack */

/* Returns 0, or 1 if a value is outside [-7, 7], 2 if K is odd. */
int oracle_pack_int4(const int8_t* q, int64_t N, int64_t K, uint8_t* out) {
    if (K % 2 != 0) return 2;
    for (int64_t i = 0; i < N * K; ++i)
        if (q[i] < -7 || q[i] > 7) return 1;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t j = 0; j < K / 2; ++j) {
            const uint8_t lo = (uint8_t)q[n * K + 2 * j] & 0x0Fu;
            const uint8_t hi = (uint8_t)q[n * K + 2 * j + 1] & 0x0Fu;
            out[n * (K / 2) + j] = (uint8_t)(lo | (hi << 4));
        }
    return 0;
}

static inline int8_t nibble_to_code(uint8_t v) { return (int8_t)(v >= 8 ? (int)v - 16 : (int)v); }

void oracle_unpack_int4(const uint8_t* p, int64_t N, int64_t Kh, int8_t* out) {
    for (int64_t n = 0; n < N; ++n)
        for (int64_t j = 0; j < Kh; ++j) {
            const uint8_t b = p[n * Kh + j];
            out[n * 2 * Kh + 2 * j] = nibble_to_code(b & 0x0Fu);
            out[n * 2 * Kh + 2 * j + 1] = nibble_to_code(b >> 4);
        }
}

/* --------------------------------------------------------------- quantizer */

/* fp32 weights [N, K] -> int8 codes [N, K] and binary16 scale bits [N, K/G].
   Returns 0, or 3 if G <= 0 or K % G != 0. */
int oracle_quantize_groupwise(const float* w, int64_t N, int64_t K, int64_t G, int8_t* q, uint16_t* scales) {
    if (G <= 0 || K % G != 0) return 3;
    const int64_t groups = K / G;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t g = 0; g < groups; ++g) {
            const float* src = w + n * K + g * G;
            float amax = 0.0f;
            for (int64_t i = 0; i < G; ++i) {
                const float a = fabsf(src[i]);
                if (a > amax || isnan(a)) amax = a;
            }
            float s = amax / 7.0f;
            if (amax == 0.0f) s = 1.0f;
            for (int64_t i = 0; i < G; ++i) {
                float v = nearbyintf(src[i] / s); /* round half to even (default rounding mode) */
                if (isnan(v)) v = 0.0f; /* NaN weights: the reference leaves the code unspecified */
                if (v < -7.0f) v = -7.0f;
                if (v > 7.0f) v = 7.0f;
                q[n * K + g * G + i] = (int8_t)v;
            }
            scales[n * groups + g] = oracle_f32_to_f16(s);
        }
    return 0;
}

/* -------------------------------------------------------------- dequantize */

void oracle_dequantize_f32(const uint8_t* p, const uint16_t* scales, int64_t N, int64_t K, int64_t G,
                           float* out) {
    const int64_t groups = K / G;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            const uint8_t b = p[n * (K / 2) + k / 2];
            const int8_t c = nibble_to_code((k & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 0x0Fu));
            out[n * K + k] = (float)c * oracle_f16_to_f32(scales[n * groups + k / G]);
        }
}

void oracle_dequantize_f16(const uint8_t* p, const uint16_t* scales, int64_t N, int64_t K, int64_t G,
                           uint16_t* out) {
    const int64_t groups = K / G;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            const uint8_t b = p[n * (K / 2) + k / 2];
            const int8_t c = nibble_to_code((k & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 0x0Fu));
            out[n * K + k] = oracle_f32_to_f16((float)c * oracle_f16_to_f32(scales[n * groups + k / G]));
        }
}

/* ------------------------------------------------------------------ linear */

/* x: binary16 bits [M, K]; returns binary16 bits [M, N] of
   fp16( fp32( sum_k fp32(x[m][k]) * W[n][k] ) ) with W the fp32 dequantized
   weights; the sum is accumulated in double so the oracle's own rounding
   error is far below the comparison tolerance. `threads` <= 0 = default. */
int oracle_linear(const uint16_t* x, const uint8_t* p, const uint16_t* scales, int64_t M, int64_t N, int64_t K,
                  int64_t G, uint16_t* out, int threads) {
    if (G <= 0 || K % G != 0 || K % 2 != 0) return 3;
    float* W = (float*)malloc((size_t)(N * K > 0 ? N * K : 1) * sizeof(float));
    float* X = (float*)malloc((size_t)(M * K > 0 ? M * K : 1) * sizeof(float));
    if (W == NULL || X == NULL) {
        free(W);
        free(X);
        return 4;
    }
#ifdef _OPENMP
    const int saved = omp_get_max_threads();
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    oracle_dequantize_f32(p, scales, N, K, G, W);
    for (int64_t i = 0; i < M * K; ++i) X[i] = oracle_f16_to_f32(x[i]);
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        const float* wr = W + n * K;
        for (int64_t m = 0; m < M; ++m) {
            const float* xr = X + m * K;
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) acc += (double)xr[k] * (double)wr[k];
            out[m * N + n] = oracle_f32_to_f16((float)acc);
        }
    }
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(saved);
#endif
    free(W);
    free(X);
    return 0;
}
