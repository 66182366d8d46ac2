/*
 * oracle.h — CPU restatement of MYTHOS.cpp's quantized matvec/matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path (libmythos_oil.so) never calls
 * into it and has no CPU fallback.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the MYTHOS.cpp source tree).  Pinning status of each function is recorded in
 * oracle.c next to the function (what fixes it: golden vectors from the
 * compiled reference, closed forms, brute force, exhaustive sweeps).
 *
 * Conventions: sizes are int64_t, pointers are plain host pointers, outputs are
 * overwritten (never accumulated), exactly as in the reference kernels.
 */
#ifndef MYTHOS_ORACLE_H
#define MYTHOS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded generator: src/random.cpp:7-51 ---------------------------- */
typedef struct { uint64_t s[2]; } orc_rng;
void     orc_rng_seed(orc_rng* r, uint64_t seed);
uint64_t orc_rng_next_u64(orc_rng* r);
float    orc_rng_uniform(orc_rng* r);
float    orc_rng_normal(orc_rng* r);
int      orc_rng_uniform_int(orc_rng* r, int lo, int hi);

/* ---- FP16 conversions ---------------------------------------------------- */
float    orc_fp16_to_float(uint16_t h);          /* src/kernel_oil4.cpp:15-29 */
float    orc_half_to_float_codebook(uint16_t h); /* src/codebook.cpp:36-64   */
uint16_t orc_float_to_half_trunc(float f);       /* src/codebook.cpp:16-34   */
void     orc_fp16_to_float_n(const uint16_t* h, float* f, int64_t n);

/* ---- OIL8: src/kernel_oil8.cpp ------------------------------------------ */
void orc_oil8_gemm_scalar(const uint8_t* idx, const float* cb, const float* act,
                          float* out, int64_t M, int64_t N, int64_t K);
void orc_oil8_gemm_avx2(const uint8_t* idx, const float* cb, const float* act,
                        float* out, int64_t M, int64_t N, int64_t K);
/* weight-shared batched GEMV: y[t][m] = sum_k cb[idx[m][k]] * x[t][k]
 * (= `batch` reference calls with N=1 and per-token act/out offsets) */
void orc_oil8_gemv(const uint8_t* idx, const float* cb, const float* x, float* y,
                   int64_t M, int64_t K, int64_t batch, int nthreads);

/* ---- OIL4: src/kernel_oil4.cpp ------------------------------------------ */
void orc_oil4_gemm_scalar(const uint8_t* nib, const uint16_t* cb16, const float* act,
                          float* out, int64_t M, int64_t N, int64_t K);
void orc_oil4_gemm_avx2(const uint8_t* nib, const uint16_t* cb16, const float* act,
                        float* out, int64_t M, int64_t N, int64_t K);
/* per-block codebooks: cb16[m][K/block][16]; y[t][m] */
void orc_oil4_gemv_blocked(const uint8_t* nib, const uint16_t* cb16, int64_t block,
                           const float* x, float* y, int64_t M, int64_t K,
                           int64_t batch, int nthreads);

/* ---- int8 activation quantization: src/int8_quant.cpp:8-41 ------------- */
void orc_quantize_per_tensor(const float* src, int8_t* dst, int64_t n,
                             float* scale, float* inv_scale);
void orc_quantize_per_token(const float* src, int8_t* dst, int64_t rows, int64_t cols,
                            float* scale, float* inv_scale);
void orc_dequantize_per_tensor(const int8_t* src, float* dst, int64_t n, float inv_scale);

/* ---- ternary I2_S: src/kernel_i2s.cpp ----------------------------------- */
int  orc_i2s_decode(uint8_t packed, int shift);                 /* :16-21 */
void orc_i2s_gemv(const uint8_t* packed_w, float w_scale, const int8_t* act,
                  float act_scale, float* out, int64_t K);      /* :32-40 */
void orc_i2s_gemm(const uint8_t* w, const float* a, float* o,
                  int64_t M, int64_t N, int64_t K);             /* :42-65 */
void orc_i2s_gemm_vnni(const uint8_t* w, const int8_t* a, float* o,
                       int64_t M, int64_t N, int64_t K);        /* :201-235 */
/* Fused decode op (quantize_per_token -> i2s_gemv per row), y[t][m]. */
void orc_i2s_gemv_f32(const uint8_t* packed, float w_scale, const float* x, float* y,
                      int64_t M, int64_t K, int64_t batch, int nthreads);

/* ---- ternary LUT kernels: src/kernel_tl.cpp ----------------------------- */
void orc_tl1_precompute_lut(const int8_t* act, int8_t* lut, int64_t K);
void orc_tl1_gemm(const uint8_t* w, const float* a, float* o,
                  int64_t M, int64_t N, int64_t K);
void orc_tl2_precompute_lut(const int8_t* act, int8_t* lut, int64_t K);
void orc_tl2_gemm(const uint8_t* w, const float* a, float* o,
                  int64_t M, int64_t N, int64_t K);

/* ---- dense FP32 math (src/math.cpp) --------------------------------------- */
void orc_gemv(float alpha, const float* A, const float* x, float beta, float* y,
              int64_t M, int64_t N);                             /* :52-72 */
void orc_gemm(float alpha, const float* A, const float* B, float beta, float* C,
              int64_t M, int64_t N, int64_t K);                         /* src/math.cpp:74-97 */
void orc_relu(const float* x, float* y, int64_t n);                      /* src/math.cpp:99-105 */
void orc_gelu(const float* x, float* y, int64_t n);                      /* src/math.cpp:107-117 */
void orc_scale(float s, const float* x, float* y, int64_t n);            /* src/math.cpp:278-284 */
void orc_layer_norm(const float* x, const float* gamma, const float* beta, float eps, float* y,
                    int64_t rows, int64_t dim);                          /* src/math.cpp:148-180 */
void orc_softmax_axis(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner); /* :207-249 */
void orc_rms_norm(const float* x, const float* gamma, float eps, float* y,
                  int64_t rows, int64_t dim);                    /* :182-205 */
void orc_silu(const float* x, float* y, int64_t n);              /* :119-128 */

/* ---- config-5 decoder (decoder.c) ---------------------------------------- */
void orc_softmax(const float* x, float* y, int64_t rows, int64_t dim);  /* src/math.cpp:207-249 */
void orc_add(const float* a, const float* b, float* c, int64_t n);      /* src/math.cpp:251-258 */
void orc_mul(const float* a, const float* b, float* c, int64_t n);      /* src/math.cpp:269-276 */
void orc_silu_mul(const float* g, const float* u, float* y, int64_t n); /* transformer.cpp:377-386 */
void orc_rope_tables(int64_t head_dim, int64_t max_seq, float theta,
                     float* cos_t, float* sin_t);                       /* transformer.cpp:102-117 */
void orc_rope_apply(float* x, int64_t heads, int64_t head_dim, int64_t pos,
                    const float* cos_t, const float* sin_t);            /* transformer.cpp:119-139 */
void orc_attention_decode(const float* q, const float* kc, const float* vc, float* out,
                          int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t ctx,
                          int64_t kv_stride);                           /* transformer.cpp:188-348 */
int32_t orc_argmax(const float* logits, int64_t n);                    /* src/sampler.cpp:12-22 */

typedef struct {
    int64_t vocab, hidden, layers, heads, kv_heads, head_dim, ffn, max_seq, cb_block;
    float eps, theta;
    int64_t kv_bf16;      /* 1: K/V rounded to bf16 (nearest even) when appended */
} orc_decoder_config;

typedef struct {          /* one block; weights in [out][in] rows */
    const float* attn_norm;
    const float* ffn_norm;
    const uint8_t *wq, *wk, *wv, *wo;           /* OIL8 */
    const float *cbq, *cbk, *cbv, *cbo;
    const uint8_t *wgate, *wup;                 /* OIL4, codebooks [out][in/cb_block][16] */
    const uint16_t *cbgate, *cbup;
    const uint8_t* wdown;                       /* I2_S */
    float down_scale;
} orc_decoder_layer;

typedef struct {
    const float* emb;                           /* [vocab][hidden] FP32 */
    const float* final_norm;
    const uint8_t* lm_idx;                      /* OIL8 [vocab][hidden] */
    const float* lm_cb;
    const float* rope_cos;                      /* [max_seq][head_dim/2] */
    const float* rope_sin;
    const orc_decoder_layer* layers;
} orc_decoder_model;

/* One token of one sequence at position pos: writes that position's K/V into
 * kcache/vcache ([layers][kv_heads][max_seq][head_dim]) and the logits
 * [vocab].  down_mode 0: I2_S with int8 activations; 1: FP32 activations. */
void orc_decoder_step(const orc_decoder_config* c, const orc_decoder_model* m, float* kcache,
                      float* vcache, int64_t pos, int32_t token, float* logits, int down_mode,
                      int nthreads);

/* The attention half of layer l for one token: x <- x + O(attention(rmsnorm(x)))
 * (src/transformer.cpp:396-403) over the layer's cache kc/vc
 * [kv_heads][max_seq][head_dim].  append = 1 computes the position's K/V and
 * writes them into the cache first; append = 0 takes the cache as it is
 * (position pos already filled, e.g. with another implementation's values). */
void orc_decoder_attn_half(const orc_decoder_config* c, const orc_decoder_model* m, int64_t l, float* kc,
                           float* vc, int64_t pos, float* x, int append, int nthreads);

/* i2s_gemv (src/kernel_i2s.cpp:32-40) over M rows for given int8 activations
 * q [K] and act_scale inv: y[m]. */
void orc_i2s_gemv_rows(const uint8_t* packed, float w_scale, const int8_t* q, float inv, float* y, int64_t M,
                       int64_t K, int nthreads);

/* float -> bf16 -> float, round to nearest even (NaN kept a NaN). */
float orc_bf16_round(float f);

/* ---- OIL4 prefill GEMM reference: C[m][n] = bf16(sum_k A[m][k] * W[n][k]) ---- */
void orc_oil4_gemm_prefill(const uint16_t* a_bf16, const uint8_t* nib, const uint16_t* cb16,
                           int64_t block, uint16_t* c_bf16, float* c_f32,
                           int64_t M, int64_t N, int64_t K, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
