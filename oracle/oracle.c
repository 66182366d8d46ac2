/*
 * oracle.c — CPU restatement of MYTHOS.cpp's quantized matvec/matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Compiled with gcc -O2
 * -ffp-contract=off so that every `s += a*b` below is a separate multiply and
 * add unless the code calls fmaf() explicitly, which it does exactly where the
 * reference uses _mm256_fmadd_ps.
 *
 * Pinning (what fixes each function besides this restatement):
 *   - RNG, fp16 conversions, oil8/oil4 (scalar + AVX2), i2s_gemv/gemm/vnni,
 *     quantize_per_*, tl1, tl2, gemv, rms_norm, silu: golden vectors written by
 *     tests/golden/make_golden.py from the reference sources compiled in this
 *     container (oracle/_ref), plus the closed-form / exhaustive / brute-force
 *     checks in tests/test_oracle.py.
 *   - orc_oil8_gemv, orc_oil4_gemv_blocked, orc_i2s_gemv_f32: compositions of
 *     pinned functions (checked against them call by call in tests).
 *   - orc_oil4_gemm_prefill: checked against a float64 numpy contraction of the
 *     dequantized weights and against orc_oil4_gemv_blocked row by row.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* RNG: xoroshiro128+ seeded by two splitmix64 draws (src/random.cpp:7-51). */
/* ------------------------------------------------------------------------ */
static uint64_t splitmix64(uint64_t* state) {           /* src/random.cpp:7-12 */
    uint64_t z = (*state += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void orc_rng_seed(orc_rng* r, uint64_t seed) {          /* src/random.cpp:16-20 */
    uint64_t t = seed;
    r->s[0] = splitmix64(&t);
    r->s[1] = splitmix64(&t);
}
uint64_t orc_rng_next_u64(orc_rng* r) {                 /* src/random.cpp:22-30 */
    uint64_t s0 = r->s[0], s1 = r->s[1];
    uint64_t out = s0 + s1;
    s1 ^= s0;
    r->s[0] = rotl64(s0, 24) ^ s1 ^ (s1 << 16);
    r->s[1] = rotl64(s1, 37);
    return out;
}
float orc_rng_uniform(orc_rng* r) {                     /* src/random.cpp:34-36 */
    /* (u64 >> 11) converted to float first (rounds; may reach 2^53 -> 1.0f) */
    return (float)(orc_rng_next_u64(r) >> 11) * (1.0f / 9007199254740992.0f);
}
float orc_rng_normal(orc_rng* r) {                      /* src/random.cpp:38-43 */
    float u1 = orc_rng_uniform(r);
    float u2 = orc_rng_uniform(r);
    if (u1 < 1e-10f) u1 = 1e-10f;
    return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}
int orc_rng_uniform_int(orc_rng* r, int lo, int hi) {   /* src/random.cpp:45-51 */
    uint64_t range = (uint64_t)(hi - lo + 1);
    uint64_t limit = UINT64_MAX - (UINT64_MAX % range);
    uint64_t v;
    do { v = orc_rng_next_u64(r); } while (v >= limit);
    return lo + (int)(v % range);
}

/* ------------------------------------------------------------------------ */
/* FP16                                                                     */
/* ------------------------------------------------------------------------ */
/* src/kernel_oil4.cpp:15-29: exact for normals and subnormals (mant * 2^-24);
 * every NaN becomes the canonical quiet NaN. */
float orc_fp16_to_float(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    if (e == 0) {
        float v = (float)mant * 0.000000059604644775390625f;
        return sign ? -v : v;
    }
    if (e == 31) return mant == 0 ? (sign ? -INFINITY : INFINITY) : NAN;
    uint32_t bits = (sign << 31) | ((e + 112u) << 23) | (mant << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* src/codebook.cpp:36-64 (CodebookOIL4::half_to_float, used by dequantize /
 * OILReader::read_tensor).  Normals, zeros, inf and NaN payloads match
 * orc_fp16_to_float; subnormals do not: the normalisation loop leaves
 * `shift` = position p of the leading mantissa bit and sets the exponent
 * field to 113 - p (IEEE: 103 + p), and the shifted mantissa is truncated to
 * 16 bits.  Restated literally; only 0x0020-style values agree with IEEE. */
float orc_half_to_float_codebook(uint16_t h) {
    uint16_t sign = h & 0x8000u;
    int32_t e = (h >> 10) & 0x1f;
    uint16_t mant = h & 0x03ffu;
    uint32_t bits;
    if (e == 0) {
        if (mant == 0) {
            bits = (uint32_t)sign << 16;
        } else {
            int shift = 10;
            while ((mant & 0x0400u) == 0) { mant = (uint16_t)(mant << 1); shift--; }
            e = 1 - shift + 127 - 15;
            /* `mant = (mant & 0x03FF) << 13` is stored back into the uint16_t
             * `mant`, so only the low 16 bits of the shifted mantissa survive */
            mant = (uint16_t)((mant & 0x03ffu) << 13);
            bits = ((uint32_t)sign << 16) | ((uint32_t)e << 23) | (uint32_t)mant;
        }
    } else if (e == 31) {
        bits = ((uint32_t)sign << 16) | 0x7f800000u | ((uint32_t)mant << 13);
    } else {
        bits = ((uint32_t)sign << 16) | ((uint32_t)(e - 15 + 127) << 23) | ((uint32_t)mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* src/codebook.cpp:16-34: truncating (round-toward-zero) conversion. */
uint16_t orc_float_to_half_trunc(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    int32_t e = (int32_t)((u >> 23) & 0xff) - 127 + 15;
    uint32_t mant = u & 0x007fffffu;
    if (e <= 0) {
        if (e < -10) return sign;
        mant = (mant | 0x00800000u) >> (1 - e);
        return (uint16_t)(sign | (uint16_t)(mant >> 13));
    }
    if (e >= 31) return (uint16_t)(sign | 0x7c00u | (mant != 0 ? 0x0200u : 0));
    return (uint16_t)(sign | ((uint16_t)e << 10) | (uint16_t)(mant >> 13));
}

void orc_fp16_to_float_n(const uint16_t* h, float* f, int64_t n) {
    for (int64_t i = 0; i < n; i++) f[i] = orc_fp16_to_float(h[i]);
}

/* ------------------------------------------------------------------------ */
/* OIL8                                                                     */
/* ------------------------------------------------------------------------ */
/* src/kernel_oil8.cpp:14-27: per (m,n) the weight row is indices[(m*N+n)*K..]. */
void orc_oil8_gemm_scalar(const uint8_t* idx, const float* cb, const float* act,
                          float* out, int64_t M, int64_t N, int64_t K) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const uint8_t* w = idx + (m * N + n) * K;
            const float* a = act + n * K;
            float s = 0.0f;
            for (int64_t k = 0; k < K; k++) s += cb[w[k]] * a[k];
            out[m * N + n] = s;
        }
}

/* Horizontal sum of an 8-lane __m256 the way src/kernel_oil8.cpp:46-51
 * (and kernel_oil4.cpp:173-178) does it: lo+hi, then two hadd_ps. */
static float hsum8_avx(const float v[8]) {
    float s4[4];
    for (int i = 0; i < 4; i++) s4[i] = v[i] + v[i + 4];
    float h0 = s4[0] + s4[1], h1 = s4[2] + s4[3];
    return h0 + h1;
}

/* src/kernel_oil8.cpp:30-60: 8 FMA lanes over k-steps of 8, then the
 * horizontal sum, then a sequential tail. */
void orc_oil8_gemm_avx2(const uint8_t* idx, const float* cb, const float* act,
                        float* out, int64_t M, int64_t N, int64_t K) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const uint8_t* w = idx + (m * N + n) * K;
            const float* a = act + n * K;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int64_t k = 0;
            for (; k + 8 <= K; k += 8)
                for (int l = 0; l < 8; l++) acc[l] = fmaf(cb[w[k + l]], a[k + l], acc[l]);
            float r = hsum8_avx(acc);
            /* gcc -O3 -mfma (GNU dialect, -ffp-contract=fast) contracts the
             * tail's `result += cb*a` into an FMA */
            for (; k < K; k++) r = fmaf(cb[w[k]], a[k], r);
            out[m * N + n] = r;
        }
}

void orc_oil8_gemv(const uint8_t* idx, const float* cb, const float* x, float* y,
                   int64_t M, int64_t K, int64_t batch, int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t m = 0; m < M; m++)
        for (int64_t t = 0; t < batch; t++)
            orc_oil8_gemm_avx2(idx + m * K, cb, x + t * K, y + t * M + m, 1, 1, K);
}

/* ------------------------------------------------------------------------ */
/* OIL4                                                                     */
/* ------------------------------------------------------------------------ */
/* src/kernel_oil4.cpp:31-54.  Weight row (m,n) = packed[(m*N+n)*K/2 ..];
 * index of element k = low nibble of byte k/2 for even k, high nibble for
 * odd k (:45-48; also tools/convert.cpp:362-365). */
void orc_oil4_gemm_scalar(const uint8_t* nib, const uint16_t* cb16, const float* act,
                          float* out, int64_t M, int64_t N, int64_t K) {
    float c[16];
    for (int i = 0; i < 16; i++) c[i] = orc_fp16_to_float(cb16[i]);
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const uint8_t* w = nib + (m * N + n) * K / 2;
            const float* a = act + n * K;
            float s = 0.0f;
            for (int64_t k = 0; k < K; k++) {
                uint8_t i = (k % 2 == 0) ? (w[k / 2] & 0xf) : ((w[k / 2] >> 4) & 0xf);
                s += c[i] * a[k];
            }
            out[m * N + n] = s;
        }
}

/* src/kernel_oil4.cpp:57-114 as compiled with -mavx2: _mm_loadl_epi64 loads
 * 8 bytes (16 nibbles), so `idx_even` holds the 16 indices in k order and
 * `idx_odd` (unpackhi of zero upper halves) is all zeros.  Each 16-step adds
 * cb[idx]*a for the 16 weights and cb[0]*a again for the same 16
 * activations: y_avx2 = y_scalar + cb[0] * sum_{k < 16*floor(K/16)} a[k],
 * up to summation order. */
void orc_oil4_gemm_avx2(const uint8_t* nib, const uint16_t* cb16, const float* act,
                        float* out, int64_t M, int64_t N, int64_t K) {
    float c[16];
    for (int i = 0; i < 16; i++) c[i] = orc_fp16_to_float(cb16[i]);
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const uint8_t* w = nib + (m * N + n) * K / 2;
            const float* a = act + n * K;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int64_t k = 0;
            for (; k + 16 <= K; k += 16) {
                const uint8_t* p = w + k / 2;
                float w16[16];
                for (int j = 0; j < 8; j++) {
                    w16[2 * j] = c[p[j] & 0xf];
                    w16[2 * j + 1] = c[(p[j] >> 4) & 0xf];
                }
                for (int l = 0; l < 8; l++) acc[l] = fmaf(w16[l], a[l + k], acc[l]);
                for (int l = 0; l < 8; l++) acc[l] = fmaf(w16[8 + l], a[k + 8 + l], acc[l]);
                for (int l = 0; l < 8; l++) acc[l] = fmaf(c[0], a[k + l], acc[l]);
                for (int l = 0; l < 8; l++) acc[l] = fmaf(c[0], a[k + 8 + l], acc[l]);
            }
            float r = hsum8_avx(acc);
            for (; k < K; k++) {   /* contracted to an FMA, as in the oil8 tail */
                uint8_t i = (k % 2 == 0) ? (w[k / 2] & 0xf) : ((w[k / 2] >> 4) & 0xf);
                r = fmaf(c[i], a[k], r);
            }
            out[m * N + n] = r;
        }
}

/* Per-block codebooks (the BASELINE configs): element k of row m uses
 * codebook cb16[(m*(K/block) + k/block)*16 ..]; otherwise the scalar
 * semantics of src/kernel_oil4.cpp:31-54 (sequential FP32 accumulation). */
void orc_oil4_gemv_blocked(const uint8_t* nib, const uint16_t* cb16, int64_t block,
                           const float* x, float* y, int64_t M, int64_t K,
                           int64_t batch, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    const int64_t nb = K / block;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t m = 0; m < M; m++) {
        const uint8_t* w = nib + m * (K / 2);
        for (int64_t t = 0; t < batch; t++) {
            const float* a = x + t * K;
            float s = 0.0f;
            for (int64_t b = 0; b < nb; b++) {
                float c[16];
                const uint16_t* cb = cb16 + (m * nb + b) * 16;
                for (int i = 0; i < 16; i++) c[i] = orc_fp16_to_float(cb[i]);
                for (int64_t k = b * block; k < (b + 1) * block; k++) {
                    uint8_t i = (k % 2 == 0) ? (w[k / 2] & 0xf) : ((w[k / 2] >> 4) & 0xf);
                    s += c[i] * a[k];
                }
            }
            y[t * M + m] = s;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* int8 activation quantization (src/int8_quant.cpp:8-41)                   */
/* ------------------------------------------------------------------------ */
void orc_quantize_per_tensor(const float* src, int8_t* dst, int64_t n,
                             float* scale, float* inv_scale) {
    float max_abs = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float v = fabsf(src[i]);
        if (v > max_abs) max_abs = v;
    }
    if (max_abs < 1e-10f) max_abs = 1e-10f;
    float s = 127.0f / max_abs;
    float inv = max_abs / 127.0f;
    /* std::round = half away from zero; then truncation to int8 */
    for (int64_t i = 0; i < n; i++) dst[i] = (int8_t)roundf(src[i] * s);
    if (scale) *scale = s;
    if (inv_scale) *inv_scale = inv;
}
void orc_quantize_per_token(const float* src, int8_t* dst, int64_t rows, int64_t cols,
                            float* scale, float* inv_scale) {
    for (int64_t r = 0; r < rows; r++)
        orc_quantize_per_tensor(src + r * cols, dst + r * cols, cols,
                                scale ? scale + r : 0, inv_scale ? inv_scale + r : 0);
}
void orc_dequantize_per_tensor(const int8_t* src, float* dst, int64_t n, float inv_scale) {
    for (int64_t i = 0; i < n; i++) dst[i] = (float)src[i] * inv_scale;
}

/* ------------------------------------------------------------------------ */
/* I2_S ternary (src/kernel_i2s.cpp)                                        */
/* ------------------------------------------------------------------------ */
/* :16-21: code 00 -> -1, 01 -> 0, 10 and 11 -> +1; element 4i+j of a row is
 * bits 2j..2j+1 of byte i (LUT built at :26-30). */
int orc_i2s_decode(uint8_t packed, int shift) {
    int v = (packed >> shift) & 3;
    return v == 0 ? -1 : (v == 1 ? 0 : 1);
}
static inline int t2(const uint8_t* w, int64_t i) { return orc_i2s_decode(w[i / 4], (int)(i % 4) * 2); }

/* :32-40 with the LUT initialised (the reference reads g_i2s_lut without
 * call_once: before any i2s_gemm* call it is all zeros and the result is 0). */
void orc_i2s_gemv(const uint8_t* packed_w, float w_scale, const int8_t* act,
                  float act_scale, float* out, int64_t K) {
    float s = 0.0f;
    for (int64_t i = 0; i < K; i++) s += (float)t2(packed_w, i) * (float)act[i];
    *out = (s * w_scale) * act_scale;
}

/* :42-65: weights shared over n (row m at w + m*(K/4)), FP32 partial sum per
 * 128-element block, out[m*N+n]. */
void orc_i2s_gemm(const uint8_t* w, const float* a, float* o,
                  int64_t M, int64_t N, int64_t K) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            float s = 0.0f;
            for (int64_t k = 0; k < K; k += 128) {
                int64_t bk = (K - k < 128) ? K - k : 128;
                const uint8_t* wb = w + m * (K / 4) + k / 4;
                const float* ab = a + n * K + k;
                float bs = 0.0f;
                for (int64_t i = 0; i < bk; i++) bs += (float)t2(wb, i) * ab[i];
                s += bs;
            }
            o[m * N + n] = s;
        }
}

/* :201-235 (the OIL_AVX2 body; in the as-built reference the macro is never
 * defined and the function is an empty stub at :253-256).  All products are
 * integers, so with |sum| < 2^24 the FP32 result is the exact integer dot. */
void orc_i2s_gemm_vnni(const uint8_t* w, const int8_t* a, float* o,
                       int64_t M, int64_t N, int64_t K) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const uint8_t* wb = w + m * (K / 4);
            const int8_t* ab = a + n * K;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int64_t k = 0;
            for (; k + 32 <= K; k += 32)
                for (int j = 0; j < 32; j++)
                    acc[j % 8] = fmaf((float)t2(wb, k + j), (float)ab[k + j], acc[j % 8]);
            float tot = acc[0] + acc[1] + acc[2] + acc[3] + acc[4] + acc[5] + acc[6] + acc[7];
            for (; k < K; k++) tot += (float)t2(wb, k) * (float)ab[k];
            o[m * N + n] = tot;
        }
}

/* quantize_per_token (int8_quant.cpp:24-31) then i2s_gemv per row with
 * act_scale = inv_scale (= max_abs/127). */
void orc_i2s_gemv_f32(const uint8_t* packed, float w_scale, const float* x, float* y,
                      int64_t M, int64_t K, int64_t batch, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    for (int64_t t = 0; t < batch; t++) {
        int8_t q[K > 0 ? K : 1];
        float inv;
        orc_quantize_per_tensor(x + t * K, q, K, 0, &inv);
#pragma omp parallel for num_threads(nthreads) schedule(static)
        for (int64_t m = 0; m < M; m++)
            orc_i2s_gemv(packed + m * (K / 4), w_scale, q, inv, y + t * M + m, K);
    }
}

/* ------------------------------------------------------------------------ */
/* TL1 / TL2 (src/kernel_tl.cpp)                                            */
/* ------------------------------------------------------------------------ */
static void quant_rows_tl(const float* a, int8_t* q, float* scales, int64_t N, int64_t K) {
    /* src/kernel_tl.cpp:42-52 / :118-129: scales[n] = 127/max_abs */
    for (int64_t n = 0; n < N; n++) {
        float mx = 0.0f;
        for (int64_t k = 0; k < K; k++) {
            float v = fabsf(a[n * K + k]);
            if (v > mx) mx = v;
        }
        if (mx < 1e-10f) mx = 1e-10f;
        scales[n] = 127.0f / mx;
        for (int64_t k = 0; k < K; k++) q[n * K + k] = (int8_t)roundf(a[n * K + k] * scales[n]);
    }
}
static inline int8_t clamp_i8(int32_t v) { return (int8_t)(v < -128 ? -128 : (v > 127 ? 127 : v)); }

void orc_tl1_precompute_lut(const int8_t* act, int8_t* lut, int64_t K) {  /* :13-31 */
    for (int64_t g = 0; g < K / 2; g++) {
        int8_t a0 = act[2 * g], a1 = act[2 * g + 1];
        int idx = 0;
        for (int w0 = -1; w0 <= 1; w0++)
            for (int w1 = -1; w1 <= 1; w1++) lut[g * 9 + idx++] = clamp_i8(a0 * w0 + a1 * w1);
    }
}

/* :33-74.  Weight row (m,n) at w + (m*N+n)*K/4.  For each pair i (even,
 * i < K-1) the LUT entry is selected by the 2-bit code of element i alone
 * (`wi`, 0..3), not by the pair; out = (float)total / (127/max_abs). */
void orc_tl1_gemm(const uint8_t* w, const float* a, float* o,
                  int64_t M, int64_t N, int64_t K) {
    int8_t* q = (int8_t*)__builtin_alloca((size_t)(N * K > 0 ? N * K : 1));
    float* sc = (float*)__builtin_alloca((size_t)(N > 0 ? N : 1) * sizeof(float));
    quant_rows_tl(a, q, sc, N, K);
    int8_t* lut = (int8_t*)__builtin_alloca((size_t)((K / 2) * 9 + 1));
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const uint8_t* wr = w + (m * N + n) * K / 4;
            orc_tl1_precompute_lut(q + n * K, lut, K);
            int32_t tot = 0;
            for (int64_t i = 0; i < K - 1; i += 2) {
                int wi = (wr[i / 4] >> ((i % 4) * 2)) & 3;
                tot += lut[(i / 2) * 9 + wi];
            }
            o[m * N + n] = (float)tot / sc[n];
        }
}

void orc_tl2_precompute_lut(const int8_t* act, int8_t* lut, int64_t K) {  /* :88-107 */
    for (int64_t k = 0; k < K; k += 3) {   /* reads act[k+1], act[k+2]: K % 3 == 0 */
        int8_t a0 = act[k], a1 = act[k + 1], a2 = act[k + 2];
        int idx = 0;
        for (int w0 = -1; w0 <= 1; w0++)
            for (int w1 = -1; w1 <= 1; w1++)
                for (int w2 = -1; w2 <= 1; w2++)
                    lut[(k / 3) * 27 + idx++] = clamp_i8(a0 * w0 + a1 * w1 + a2 * w2);
    }
}

/* :109-168.  Defined here for K % 3 == 0 only (for other K the reference
 * reads activations past the row).  bytes_per_row = ceil(K/4); element k of
 * a row sits at byte k/4, bits 2(k%4) (the "3 bytes per 12 weights" grouping
 * is the plain I2_S packing), so total = exact int dot; out = (float)total /
 * (127/max_abs). */
void orc_tl2_gemm(const uint8_t* w, const float* a, float* o,
                  int64_t M, int64_t N, int64_t K) {
    int8_t* q = (int8_t*)__builtin_alloca((size_t)(N * K > 0 ? N * K : 1));
    float* sc = (float*)__builtin_alloca((size_t)(N > 0 ? N : 1) * sizeof(float));
    quant_rows_tl(a, q, sc, N, K);
    int64_t bpr = (K * 2 + 7) / 8;
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            const uint8_t* wr = w + (m * N + n) * bpr;
            const int8_t* ar = q + n * K;
            int64_t tot = 0;
            for (int64_t g = 0; g * 12 < K; g++) {
                int64_t rem = K - g * 12;
                int64_t nt = (rem + 2) / 3 < 4 ? (rem + 2) / 3 : 4;
                for (int64_t t = 0; t < nt; t++) {
                    int64_t base = g * 12 + t * 3;
                    for (int j = 0; j < 3; j++) {
                        int64_t e = base + j;      /* element index within the row */
                        int v = orc_i2s_decode(wr[e / 4], (int)(e % 4) * 2);
                        tot += (int64_t)ar[e] * v;
                    }
                }
            }
            o[m * N + n] = (float)tot / sc[n];
        }
}

/* ------------------------------------------------------------------------ */
/* Dense math (src/math.cpp)                                                */
/* ------------------------------------------------------------------------ */
void orc_gemv(float alpha, const float* A, const float* x, float beta, float* y,
              int64_t M, int64_t N) {                                   /* :52-72 */
    for (int64_t i = 0; i < M; i++) {
        float s = 0.0f;
        for (int64_t j = 0; j < N; j++) s += A[i * N + j] * x[j];
        y[i] = alpha * s + beta * y[i];
    }
}
void orc_rms_norm(const float* x, const float* gamma, float eps, float* y,
                  int64_t rows, int64_t dim) {                           /* :182-205 */
    for (int64_t i = 0; i < rows; i++) {
        const float* r = x + i * dim;
        double ss = 0.0;
        for (int64_t j = 0; j < dim; j++) ss += (double)r[j] * r[j];
        ss /= (double)dim;
        double inv = 1.0 / sqrt(ss + (double)eps);
        for (int64_t j = 0; j < dim; j++) y[i * dim + j] = (float)((double)r[j] * inv) * gamma[j];
    }
}
void orc_silu(const float* x, float* y, int64_t n) {                     /* :119-128 */
    for (int64_t i = 0; i < n; i++) y[i] = x[i] / (1.0f + expf(-x[i]));
}
void orc_gemm(float alpha, const float* A, const float* B, float beta, float* C,
              int64_t M, int64_t N, int64_t K) {                        /* :74-97 */
    for (int64_t i = 0; i < M; i++)
        for (int64_t j = 0; j < N; j++) {
            float s = 0.0f;
            for (int64_t k = 0; k < K; k++) s += A[i * K + k] * B[k * N + j];
            C[i * N + j] = alpha * s + beta * C[i * N + j];
        }
}
void orc_relu(const float* x, float* y, int64_t n) {                     /* :99-105 */
    for (int64_t i = 0; i < n; i++) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}
void orc_gelu(const float* x, float* y, int64_t n) {                     /* :107-117 */
    const float s = 0.7071067811865475f;
    for (int64_t i = 0; i < n; i++) {
        const float v = x[i];
        y[i] = 0.5f * v * (1.0f + erff(v * s));
    }
}
void orc_scale(float s, const float* x, float* y, int64_t n) {           /* :278-284 */
    for (int64_t i = 0; i < n; i++) y[i] = s * x[i];
}
void orc_layer_norm(const float* x, const float* gamma, const float* beta, float eps, float* y,
                    int64_t rows, int64_t dim) {                         /* :148-180 */
    for (int64_t i = 0; i < rows; i++) {
        const float* r = x + i * dim;
        double mu = 0.0;
        for (int64_t j = 0; j < dim; j++) mu += r[j];
        mu /= (double)dim;
        double var = 0.0;
        for (int64_t j = 0; j < dim; j++) {
            const double d = r[j] - mu;
            var += d * d;
        }
        var /= (double)dim;
        const double inv = 1.0 / sqrt(var + (double)eps);
        for (int64_t j = 0; j < dim; j++) y[i * dim + j] = (float)(((double)r[j] - mu) * inv) * gamma[j] + beta[j];
    }
}
/* softmax along the middle axis of [outer][dim][inner] (:207-249): float
 * max, float exp, double sum, (float)(e * (1/sum)). */
void orc_softmax_axis(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner) {
    for (int64_t o = 0; o < outer; o++)
        for (int64_t i = 0; i < inner; i++) {
            const float* s = x + o * dim * inner + i;
            float* d = y + o * dim * inner + i;
            float mx = -INFINITY;
            for (int64_t k = 0; k < dim; k++) mx = s[k * inner] > mx ? s[k * inner] : mx;
            double sum = 0.0;
            for (int64_t k = 0; k < dim; k++) {
                const float v = expf(s[k * inner] - mx);
                d[k * inner] = v;
                sum += v;
            }
            const double inv = 1.0 / sum;
            for (int64_t k = 0; k < dim; k++) d[k * inner] = (float)((double)d[k * inner] * inv);
        }
}

/* ------------------------------------------------------------------------ */
/* OIL4 prefill GEMM reference                                              */
/* ------------------------------------------------------------------------ */
static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* out[m][n] = sum_k bf16->f32(A[m][k]) * W[n][k], W dequantized with the
 * per-block OIL4 codebooks; i.e. the oil4 scalar semantics applied per token,
 * with the FP32 result rounded to bf16 (RNE). */
void orc_oil4_gemm_prefill(const uint16_t* a_bf16, const uint8_t* nib, const uint16_t* cb16,
                           int64_t block, uint16_t* c_bf16, float* c_f32,
                           int64_t M, int64_t N, int64_t K, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    const int64_t nb = K / block;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t n = 0; n < N; n++) {
        float wrow[K > 0 ? K : 1];
        const uint8_t* w = nib + n * (K / 2);
        for (int64_t k = 0; k < K; k++) {
            uint8_t i = (k % 2 == 0) ? (w[k / 2] & 0xf) : ((w[k / 2] >> 4) & 0xf);
            wrow[k] = orc_fp16_to_float(cb16[(n * nb + k / block) * 16 + i]);
        }
        for (int64_t m = 0; m < M; m++) {
            const uint16_t* a = a_bf16 + m * K;
            float s = 0.0f;
            for (int64_t k = 0; k < K; k++) s += bf16_to_f32(a[k]) * wrow[k];
            if (c_f32) c_f32[m * N + n] = s;
            if (c_bf16) c_bf16[m * N + n] = f32_to_bf16_rne(s);
        }
    }
}
