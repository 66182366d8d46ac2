/*
 * decoder.c — CPU restatement of the config-5 decoder step (mixed-format
 * Llama-style stack) and of the dense ops it uses.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker of the GPU decoder in
 * libmythos_oil.so, never called by it.
 *
 * The composition follows the reference's inference path
 *   DenseModel::forward          src/model.cpp:45-75
 *   TransformerBlock::forward    src/transformer.cpp:396-406 (pre-norm, two residuals)
 *   Attention::forward           src/transformer.cpp:154-362 (inference branch, scalar code)
 *   RotaryEmbedding              src/transformer.cpp:102-139 (rotate-half, theta 10000)
 *   FFN::forward                 src/transformer.cpp:373-387 (silu(gate) * up, then down)
 *   Embedding::forward           src/transformer.cpp:29-46 (ids outside [0, vocab) -> 0)
 *   Sampler::greedy              src/sampler.cpp:12-22 (first maximum)
 * with these clean semantics where the reference's own code is not usable as
 * a definition (each is exercised against the compiled reference where they
 * agree, see tests/test_decoder_oracle.py):
 *   - weights in the kernels' [out][in] rows (the reference Linear keeps them
 *     input-major, src/transformer.cpp:62-70);
 *   - every layer rotates at the token's own position (the reference reads
 *     layer 0's cache length for every layer, src/kv_cache.cpp:190-192, so its
 *     layers >= 1 rotate one position late when fed one token at a time; RoPE
 *     scores depend only on position differences, so the result is the same
 *     up to rounding);
 *   - softmax with exp (the scalar branch, src/transformer.cpp:277-290, not the
 *     AVX2 branch's 4th-order Taylor polynomial, :255-276);
 *   - one KV cache per sequence (the reference's cache is batch-1,
 *     src/kv_cache.cpp:64-65);
 *   - projections with the quantized kernels: Q/K/V/O and lm_head OIL8
 *     (orc_oil8_gemv), gate/up OIL4 with per-block codebooks
 *     (orc_oil4_gemv_blocked), down ternary I2_S with the activations
 *     quantized per token to int8 (orc_i2s_gemv_f32); down_mode 1 instead
 *     multiplies the FP32 activations with the dequantized ternary weights,
 *     the reference Linear's arithmetic (scalar_gemm, src/kernel_i2s.cpp:91-102).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* math::softmax (src/math.cpp:207-249) over the last axis: float max, float
 * exp, double sum, (float)(e * (1/sum)). */
void orc_softmax(const float* x, float* y, int64_t rows, int64_t dim) {
    for (int64_t r = 0; r < rows; r++) {
        const float* s = x + r * dim;
        float* d = y + r * dim;
        float mx = -INFINITY;
        for (int64_t i = 0; i < dim; i++) mx = fmaxf(mx, s[i]);
        double sum = 0.0;
        for (int64_t i = 0; i < dim; i++) {
            const float v = expf(s[i] - mx);
            d[i] = v;
            sum += v;
        }
        const double inv = 1.0 / sum;
        for (int64_t i = 0; i < dim; i++) d[i] = (float)((double)d[i] * inv);
    }
}

void orc_add(const float* a, const float* b, float* c, int64_t n) {       /* src/math.cpp:251-258 */
    for (int64_t i = 0; i < n; i++) c[i] = a[i] + b[i];
}

void orc_mul(const float* a, const float* b, float* c, int64_t n) {       /* src/math.cpp:269-276 */
    for (int64_t i = 0; i < n; i++) c[i] = a[i] * b[i];
}

/* FFN activation: math::silu then math::mul (src/transformer.cpp:377-386). */
void orc_silu_mul(const float* g, const float* u, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const float s = g[i] / (1.0f + expf(-g[i]));
        y[i] = s * u[i];
    }
}

/* RotaryEmbedding constructor tables (src/transformer.cpp:102-117), float
 * arithmetic: inv_freq = 1/theta^(2j/hd), angle = pos * inv_freq. */
void orc_rope_tables(int64_t head_dim, int64_t max_seq, float theta, float* cos_t, float* sin_t) {
    const int64_t h2 = head_dim / 2;
    for (int64_t i = 0; i < max_seq; i++)
        for (int64_t j = 0; j < h2; j++) {
            const float inv_freq = 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
            const float val = (float)i * inv_freq;
            cos_t[i * h2 + j] = cosf(val);
            sin_t[i * h2 + j] = sinf(val);
        }
}

/* RotaryEmbedding::apply (src/transformer.cpp:119-139) on one token's
 * [heads][head_dim] vector at position pos: pairs (d, d + D/2). */
void orc_rope_apply(float* x, int64_t heads, int64_t head_dim, int64_t pos, const float* cos_t,
                    const float* sin_t) {
    const int64_t h2 = head_dim / 2;
    for (int64_t h = 0; h < heads; h++) {
        float* v = x + h * head_dim;
        for (int64_t d = 0; d < h2; d++) {
            const float x1 = v[d], x2 = v[d + h2];
            const float c = cos_t[pos * h2 + d], s = sin_t[pos * h2 + d];
            v[d] = x1 * c - x2 * s;
            v[d + h2] = x1 * s + x2 * c;
        }
    }
}

/* Attention for one query token over ctx cached positions, the scalar
 * inference code of src/transformer.cpp:188-348 with S = 1:
 * score = (sum_d q*k) * (1/sqrt(D)); w = exp(score - max) / sum (float sum,
 * multiply by 1/sum); out = sum_t w[t] * v[t].  Head h reads kv head
 * h % kv_heads.  kc/vc: [kv_heads][kv_stride][head_dim]. */
void orc_attention_decode(const float* q, const float* kc, const float* vc, float* out, int64_t heads,
                          int64_t kv_heads, int64_t head_dim, int64_t ctx, int64_t kv_stride) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* w = (float*)malloc((size_t)(ctx > 0 ? ctx : 1) * sizeof(float));
    for (int64_t h = 0; h < heads; h++) {
        const int64_t kh = h % kv_heads;
        const float* qh = q + h * head_dim;
        const float* kb = kc + kh * kv_stride * head_dim;
        const float* vb = vc + kh * kv_stride * head_dim;
        for (int64_t t = 0; t < ctx; t++) {
            float s = 0.0f;
            for (int64_t d = 0; d < head_dim; d++) s += qh[d] * kb[t * head_dim + d];
            w[t] = s * scale;
        }
        float mx = -INFINITY;
        for (int64_t t = 0; t < ctx; t++)
            if (w[t] > mx) mx = w[t];
        float sum = 0.0f;
        for (int64_t t = 0; t < ctx; t++) {
            w[t] = expf(w[t] - mx);
            sum += w[t];
        }
        const float inv = 1.0f / sum;
        for (int64_t t = 0; t < ctx; t++) w[t] *= inv;
        for (int64_t d = 0; d < head_dim; d++) {
            float s = 0.0f;
            for (int64_t t = 0; t < ctx; t++) s += w[t] * vb[t * head_dim + d];
            out[h * head_dim + d] = s;
        }
    }
    free(w);
}

/* Sampler::greedy (src/sampler.cpp:12-22): the first index of the maximum;
 * NaNs never compare greater. */
int32_t orc_argmax(const float* logits, int64_t n) {
    int32_t best = 0;
    float bv = -INFINITY;
    for (int64_t i = 0; i < n; i++)
        if (logits[i] > bv) {
            bv = logits[i];
            best = (int32_t)i;
        }
    return best;
}

/* Dense ternary down projection, the reference Linear's arithmetic on the
 * dequantized weight W[m][k] = t(m,k) * w_scale: y[m] = sum_k a[k] * W[m][k]
 * accumulated in k order in float (scalar_gemm, src/kernel_i2s.cpp:91-102). */
static void ternary_dense(const uint8_t* packed, float w_scale, const float* a, float* y, int64_t M, int64_t K,
                          int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t m = 0; m < M; m++) {
        const uint8_t* row = packed + m * (K / 4);
        float s = 0.0f;
        for (int64_t k = 0; k < K; k++) {
            const float w = (float)orc_i2s_decode(row[k / 4], (int)(2 * (k % 4))) * w_scale;
            s += a[k] * w;
        }
        y[m] = s;
    }
}

/* Round to the nearest bf16 (ties to even), back to float. */
float orc_bf16_round(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return f;  /* NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    memcpy(&f, &u, 4);
    return f;
}

void orc_i2s_gemv_rows(const uint8_t* packed, float w_scale, const int8_t* q, float inv, float* y, int64_t M,
                       int64_t K, int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int64_t m = 0; m < M; m++) orc_i2s_gemv(packed + m * (K / 4), w_scale, q, inv, y + m, K);
}

void orc_decoder_attn_half(const orc_decoder_config* c, const orc_decoder_model* m, int64_t l, float* kc,
                           float* vc, int64_t pos, float* x, int append, int nthreads) {
    const int64_t H = c->hidden, D = c->head_dim;
    const int64_t QD = c->heads * D, KD = c->kv_heads * D;
    const orc_decoder_layer* L = &m->layers[l];
    float* buf = (float*)malloc(sizeof(float) * (size_t)(2 * H + 4 * QD));
    float* h = buf;            /* normed input */
    float* t = h + H;          /* projection output */
    float* q = t + H;
    float* k = q + QD;
    float* v = k + QD;
    float* att = v + QD;
    if (nthreads < 1) nthreads = 1;
    orc_rms_norm(x, L->attn_norm, c->eps, h, 1, H);
    orc_oil8_gemv(L->wq, L->cbq, h, q, QD, H, 1, nthreads);
    orc_rope_apply(q, c->heads, D, pos, m->rope_cos, m->rope_sin);
    if (append) {
        orc_oil8_gemv(L->wk, L->cbk, h, k, KD, H, 1, nthreads);
        orc_oil8_gemv(L->wv, L->cbv, h, v, KD, H, 1, nthreads);
        orc_rope_apply(k, c->kv_heads, D, pos, m->rope_cos, m->rope_sin);
        if (c->kv_bf16)        /* a bf16 cache stores the rounded values */
            for (int64_t i = 0; i < KD; i++) {
                k[i] = orc_bf16_round(k[i]);
                v[i] = orc_bf16_round(v[i]);
            }
        for (int64_t kh = 0; kh < c->kv_heads; kh++) {    /* KVCache::append, src/kv_cache.cpp:122-133 */
            memcpy(kc + (kh * c->max_seq + pos) * D, k + kh * D, sizeof(float) * (size_t)D);
            memcpy(vc + (kh * c->max_seq + pos) * D, v + kh * D, sizeof(float) * (size_t)D);
        }
    }
    orc_attention_decode(q, kc, vc, att, c->heads, c->kv_heads, D, pos + 1, c->max_seq);
    orc_oil8_gemv(L->wo, L->cbo, att, t, H, QD, 1, nthreads);
    orc_add(t, x, x, H);
    free(buf);
}

void orc_decoder_step(const orc_decoder_config* c, const orc_decoder_model* m, float* kcache, float* vcache,
                      int64_t pos, int32_t token, float* logits, int down_mode, int nthreads) {
    const int64_t H = c->hidden, F = c->ffn, D = c->head_dim;
    float* buf = (float*)malloc(sizeof(float) * (size_t)(3 * H + 3 * F));
    float* x = buf;            /* residual stream */
    float* h = x + H;          /* normed input */
    float* t = h + H;          /* projection output */
    float* g = t + H;
    float* u = g + F;
    float* a = u + F;
    if (nthreads < 1) nthreads = 1;

    const int64_t id = (token < 0 || token >= c->vocab) ? 0 : token;
    memcpy(x, m->emb + id * H, sizeof(float) * (size_t)H);
    for (int64_t l = 0; l < c->layers; l++) {
        const orc_decoder_layer* L = &m->layers[l];
        float* kc = kcache + l * c->kv_heads * c->max_seq * D;
        float* vc = vcache + l * c->kv_heads * c->max_seq * D;
        orc_decoder_attn_half(c, m, l, kc, vc, pos, x, 1, nthreads);
        orc_rms_norm(x, L->ffn_norm, c->eps, h, 1, H);
        orc_oil4_gemv_blocked(L->wgate, L->cbgate, c->cb_block, h, g, F, H, 1, nthreads);
        orc_oil4_gemv_blocked(L->wup, L->cbup, c->cb_block, h, u, F, H, 1, nthreads);
        orc_silu_mul(g, u, a, F);
        if (down_mode == 1)
            ternary_dense(L->wdown, L->down_scale, a, t, H, F, nthreads);
        else
            orc_i2s_gemv_f32(L->wdown, L->down_scale, a, t, H, F, 1, nthreads);
        orc_add(t, x, x, H);
    }
    orc_rms_norm(x, m->final_norm, c->eps, h, 1, H);
    orc_oil8_gemv(m->lm_idx, m->lm_cb, h, logits, c->vocab, H, 1, nthreads);
    free(buf);
}
