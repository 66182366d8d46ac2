// decoder.hip — the mixed-format decoder stack (include/mythos_decoder.h).
//
// One decode step for B sequences is a fixed sequence of launches on one
// stream (per layer: RMSNorm, one OIL8 launch for Q, K and V, RoPE + KV append + attention
// in one kernel, O GEMV, residual add fused into the FFN RMSNorm, gate/up
// OIL4 GEMV (one launch over 2*ffn rows when gate and up are adjacent),
// SwiGLU fused with the per-token int8 quantisation, ternary down GEMV on the
// int8 activations; the next layer's RMSNorm takes the second residual add;
// after the last layer: final norm, lm_head, a two-stage greedy argmax whose
// last launch also advances the step counter).  Everything that changes from step to step
// (position, input token) is read from device memory: the step counter and
// the token history.  So the sequence captures into one HIP graph that is
// replayed for every step.  All buffers are allocated at create; the graph
// holds no memset nodes and no allocations.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <vector>

#include "launch.h"
#include "../../include/mythos_decoder.h"

// Block maxima of the batched SwiGLU per token (one per 256 columns of ffn):
// the fused batch path covers ffn <= 64 * 256.
constexpr int kAmxParts = 64;
// Prefill chunks of at least this many rows run the projections as MFMA
// GEMMs (fewer: the batched GEMVs, which read every weight once per 16 rows;
// a 64-row chunk fills half of a GEMM tile and still reads each weight once:
// the 64-token prompt at batch 1 10.6 -> 8.5 ms against a threshold of 128).
constexpr int64_t kPfGemmRows = 64;

struct mth_decoder {
    mth_decoder_config c{};
    int device = 0;
    std::vector<mth_decoder_layer> layers;
    std::vector<bool> layer_set;
    mth_decoder_globals g{};
    bool globals_set = false;

    void* block = nullptr;  // one device allocation for every buffer below
    float *x = nullptr, *h = nullptr, *t = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr;
    float *gu = nullptr, *a_inv = nullptr, *logits = nullptr;
    char *kc = nullptr, *vc = nullptr;  // [layers][B][kv_heads][max_seq][head_dim], FP32 or bf16
    size_t kv_elem = 4;
    float* taps = nullptr;              // mth_decoder_set_taps
    float *rope_cos = nullptr, *rope_sin = nullptr, *bt_partial = nullptr, *arg_v = nullptr;
    double* ssp = nullptr;  // per-workgroup sums of squares of the split RMSNorm (ResidOut): attention norm
    double* ssp2 = nullptr;  // the same for the FFN norm (batch 1)
    float* amx = nullptr;    // the SwiGLU's block maxima of |act| per token (batches: kAmxParts per token)
    int8_t* aq = nullptr;
    int *hist = nullptr, *step = nullptr, *ids = nullptr, *arg_i = nullptr;
    int64_t hist_stride = 0, layer_kv = 0;

    int64_t batch = 0, prompt_len = 0, steps = 0;
    hipStream_t cap_stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int64_t graph_batch = 0, graph_prompt = 0;
    size_t graph_nodes = 0;

    // prefill (mth_decoder_prefill): pf_rows rows of (sequence, position)
    int64_t pf_rows = 0;
    float *pf_x = nullptr, *pf_h = nullptr, *pf_t = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr;
    float *pf_att = nullptr, *pf_gu = nullptr, *pf_inv = nullptr;
    int8_t* pf_aq = nullptr;
    void* pf_ws = nullptr;  // the prefill GEMMs' scratch (A fragments, row shifts, permuted int8 activations)

    void drop_graph() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
    }
};

namespace {

using mth::api_fail;
using mth::api_ok;

size_t round_up(size_t n) { return (n + 255) & ~(size_t)255; }

// y[rows][M] = W x for an OIL4 weight, picking the batched kernel when it applies.
hipError_t oil4(const mth_decoder* d, const uint8_t* w, const uint16_t* cb, const float* x, float* y, int64_t M,
                int64_t K, hipStream_t s, int64_t rows = 0) {
    if (!rows) rows = d->batch;
    const bool aligned = (((uintptr_t)w | (uintptr_t)cb | (uintptr_t)x) & 15u) == 0;
    if (aligned && mth::oil4_bt_supported(M, K, d->c.cb_block, rows))
        return mth::launch_oil4_gemv_bt(w, cb, d->c.cb_block, x, y, M, K, rows, d->bt_partial, s);
    return mth::launch_oil4_gemv(w, cb, d->c.cb_block, x, y, M, K, rows, s);
}

// y[rows][M] = W x for an OIL8 weight: MFMA kernel for batches of 2 and more.
hipError_t oil8(const mth_decoder* d, const uint8_t* w, const float* cb, const float* x, float* y, int64_t M,
                int64_t K, hipStream_t s, int64_t rows = 0) {
    if (!rows) rows = d->batch;
    const bool aligned = (((uintptr_t)w | (uintptr_t)x) & 15u) == 0;
    if (aligned && mth::oil8_bt_supported(M, K, rows))
        return mth::launch_oil8_gemv_bt(w, cb, x, y, M, K, rows, d->bt_partial, s);
    return mth::launch_oil8_gemv(w, cb, x, y, M, K, rows, s);
}

// Q, K and V projections of the normed input h (rows) into q, k, v: one
// launch over the three matrices (each with its own codebook) where the
// kernels take them.
hipError_t qkv(const mth_decoder* d, const mth_decoder_layer& L, const float* h, float* q, float* k, float* v,
               int64_t rows, hipStream_t s) {
    const mth_decoder_config& c = d->c;
    const int64_t H = c.hidden, QD = c.heads * c.head_dim, KD = c.kv_heads * c.head_dim;
    const mth::Oil8Seg seg[3] = {{L.wq, L.cbq, q, QD}, {L.wk, L.cbk, k, KD}, {L.wv, L.cbv, v, KD}};
    // prompt chunks of >= kPfGemmRows rows: the FP32-row OIL8 GEMM on MFMA
    if (rows >= kPfGemmRows && d->pf_ws && ((uintptr_t)h & 15u) == 0 && mth::oil8_gemm_x32_supported(seg, 3, rows, H))
        return mth::launch_oil8_gemm_x32(h, seg, 3, rows, H, d->pf_ws, s);
    if (((uintptr_t)h & 15u) == 0) {
        if (rows >= 2) {
            if (mth::oil8_bt_segs_fusable(seg, 3, H, rows))
                return mth::launch_oil8_gemv_bt_segs(seg, 3, h, H, rows, d->bt_partial, s);
        } else if (mth::oil8_segs_fusable(seg, 3, H)) {
            return mth::launch_oil8_gemv_segs(seg, 3, h, H, rows, s);
        }
    }
    hipError_t e = oil8(d, L.wq, L.cbq, h, q, QD, H, s, rows);
    if (e == hipSuccess) e = oil8(d, L.wk, L.cbk, h, k, KD, H, s, rows);
    if (e == hipSuccess) e = oil8(d, L.wv, L.cbv, h, v, KD, H, s, rows);
    return e;
}

// gate and up adjacent in one [2*ffn][hidden] weight with adjacent codebooks
bool gate_up_fused(const mth_decoder* d, const mth_decoder_layer& L) {
    const int64_t H = d->c.hidden, F = d->c.ffn, nb = d->c.cb_block ? H / d->c.cb_block : 1;
    return L.wup == L.wgate + F * (H / 2) && (d->c.cb_block == 0 ? false : L.cbup == L.cbgate + F * nb * 16);
}

// The prompt as one forward pass (src/generator.cpp:36): every prompt
// position of every sequence is a row of the same layer stack (the batched
// GEMVs in groups of 16 rows, one RoPE + KV append and one causal attention
// launch per layer over all rows), in chunks of pf_rows rows (whole
// positions, all sequences); the attention of a chunk reads the earlier
// chunks' positions from the cache.  Then the final norm, lm_head and argmax
// of each sequence's last position: the decoder is left as after prompt_len
// decode steps (step counter prompt_len, the first generated token in the
// history, its logits in the logits buffer).
hipError_t enqueue_prefill(const mth_decoder* d, hipStream_t s) {
    const mth_decoder_config& c = d->c;
    const int64_t B = d->batch, P = d->prompt_len, H = c.hidden, F = c.ffn, QD = c.heads * c.head_dim;
    const bool bf16 = c.kv_dtype == 1;
    const int64_t C = std::max<int64_t>(1, d->pf_rows / B);  // positions per chunk
    hipError_t e;
#define TRY(call)                        \
    do {                                 \
        if ((e = (call)) != hipSuccess) return e; \
    } while (0)
    int64_t np = 0;
    for (int64_t p0 = 0; p0 < P; p0 += C) {
        np = std::min(C, P - p0);
        const int64_t R = B * np;
        TRY(mth::launch_embed_rows(d->g.emb, d->hist, (int)d->hist_stride, d->pf_x, R, (int)np, (int)p0, (int)H,
                                   (int)c.vocab, s));
        for (int64_t l = 0; l < c.layers; l++) {
            const mth_decoder_layer& L = d->layers[(size_t)l];
            char* kc = d->kc + l * d->layer_kv * d->kv_elem;
            char* vc = d->vc + l * d->layer_kv * d->kv_elem;
            TRY(mth::launch_rms_norm(d->pf_x, l == 0 ? nullptr : d->pf_t, L.attn_norm, d->pf_h, R, H, c.eps, s));
            TRY(qkv(d, L, d->pf_h, d->pf_q, d->pf_k, d->pf_v, R, s));
            TRY(mth::launch_rope_kv_rows(d->pf_q, d->pf_k, d->pf_v, d->rope_cos, d->rope_sin, kc, vc, bf16, R,
                                         (int)np, (int)p0, (int)c.heads, (int)c.kv_heads, (int)c.head_dim,
                                         (int)c.max_seq, s));
            TRY(mth::launch_attention_rows(d->pf_q, kc, vc, bf16, d->pf_att, R, (int)np, (int)p0, (int)c.heads,
                                           (int)c.kv_heads, (int)c.head_dim, (int)c.max_seq, s));
            {
                const mth::Oil8Seg so{L.wo, L.cbo, d->pf_t, H};
                if (R >= kPfGemmRows && ((uintptr_t)d->pf_att & 15u) == 0 && mth::oil8_gemm_x32_supported(&so, 1, R, QD))
                    TRY(mth::launch_oil8_gemm_x32(d->pf_att, &so, 1, R, QD, d->pf_ws, s));
                else
                    TRY(oil8(d, L.wo, L.cbo, d->pf_att, d->pf_t, H, QD, s, R));
            }
            TRY(mth::launch_rms_norm(d->pf_x, d->pf_t, L.ffn_norm, d->pf_h, R, H, c.eps, s));
            if (gate_up_fused(d, L)) {
                // chunks of >= kPfGemmRows rows: the FP32-row OIL4 GEMM on
                // MFMA (each weight read once per 128 rows, not per 16)
                if (R >= kPfGemmRows && mth::oil4_gemm_x32_supported(R, 2 * F, H, c.cb_block) &&
                    ((((uintptr_t)L.wgate | (uintptr_t)L.cbgate) & 15u) == 0))
                    TRY(mth::launch_oil4_gemm_x32(d->pf_h, L.wgate, L.cbgate, c.cb_block, d->pf_gu, R, 2 * F, H,
                                                  d->pf_ws, s));
                else
                    TRY(oil4(d, L.wgate, L.cbgate, d->pf_h, d->pf_gu, 2 * F, H, s, R));
                TRY(mth::launch_silu_mul_quant(d->pf_gu, d->pf_gu + F, d->pf_aq, d->pf_inv, nullptr, R, F, 2 * F,
                                               2 * F, s));
            } else {
                TRY(oil4(d, L.wgate, L.cbgate, d->pf_h, d->pf_gu, F, H, s, R));
                TRY(oil4(d, L.wup, L.cbup, d->pf_h, d->pf_gu + R * F, F, H, s, R));
                TRY(mth::launch_silu_mul_quant(d->pf_gu, d->pf_gu + R * F, d->pf_aq, d->pf_inv, nullptr, R, F, F, F,
                                               s));
            }
            if (R >= kPfGemmRows && mth::i2s_gemm_mfma_ok(H, R, F) &&
                ((((uintptr_t)L.wdown | (uintptr_t)d->pf_aq) & 15u) == 0))  // int8 MFMA GEMM, bit-exact
                TRY(mth::launch_i2s_gemm_rows(L.wdown, L.down_scale, d->pf_aq, d->pf_inv, d->pf_t, H, R, F, s));
            else if ((((uintptr_t)L.wdown | (uintptr_t)d->pf_aq) & 15u) == 0 && mth::i2s_bt_supported(H, F, R))
                TRY(mth::launch_i2s_gemv_bt(L.wdown, L.down_scale, d->pf_aq, d->pf_inv, d->pf_t, H, F, R,
                                            d->bt_partial, s));
            else
                TRY(mth::launch_i2s_gemv(L.wdown, L.down_scale, nullptr, d->pf_aq, d->pf_inv, d->pf_t, H, F, R, s));
        }
    }
    // each sequence's last position (row b*np + np-1 of the last chunk): its
    // residual stream and last FFN output, then the final norm and lm_head
    TRY(hipMemcpy2DAsync(d->x, (size_t)H * 4, d->pf_x + (np - 1) * H, (size_t)(np * H) * 4, (size_t)H * 4, (size_t)B,
                         hipMemcpyDeviceToDevice, s));
    TRY(hipMemcpy2DAsync(d->t, (size_t)H * 4, d->pf_t + (np - 1) * H, (size_t)(np * H) * 4, (size_t)H * 4, (size_t)B,
                         hipMemcpyDeviceToDevice, s));
    TRY(mth::launch_rms_norm(d->x, d->t, d->g.final_norm, d->h, B, H, c.eps, s));
    TRY(oil8(d, d->g.lm_idx, d->g.lm_cb, d->h, d->logits, c.vocab, H, s));
    // the argmax of step prompt_len - 1 writes the token after the prompt and
    // advances the step counter to prompt_len
    TRY(hipMemsetD32Async((hipDeviceptr_t)d->step, (int)(P - 1), 1, s));
    TRY(mth::launch_argmax(d->logits, B, c.vocab, d->ids, d->hist, d->step, (int)d->hist_stride, (int)d->prompt_len,
                           d->arg_v, d->arg_i, s));
#undef TRY
    return hipSuccess;
}

// One decode step of a single sequence with the RMSNorms split over the
// launches around them (see enqueue_step).
hipError_t enqueue_step_split_norm(const mth_decoder* d, hipStream_t s) {
    const mth_decoder_config& c = d->c;
    const int64_t H = c.hidden, F = c.ffn, QD = c.heads * c.head_dim, KD = c.kv_heads * c.head_dim;
    hipError_t e;
#define TRY(call)                        \
    do {                                 \
        if ((e = (call)) != hipSuccess) return e; \
    } while (0)
    using mth::plain_slices;
    // x: residual stream, h: x * gamma of the next norm.  The attention
    // norm's partial sums are written to ssp (embedding, down projections),
    // the FFN norm's to ssp2 (O projections), so the down projection with the
    // SwiGLU fused in reads one buffer and writes the other.
    mth::ResidOut ro{d->x, d->layers[0].attn_norm, d->h, d->ssp};
    mth::NormScale ns_attn{d->ssp, 1, (float)H, c.eps}, ns_ffn{d->ssp2, 1, (float)H, c.eps};
    TRY(mth::launch_embed(d->g.emb, d->hist, d->step, (int)d->hist_stride, d->x, 1, (int)H, (int)c.vocab, s, ro));
    for (int64_t l = 0; l < c.layers; l++) {
        const mth_decoder_layer& L = d->layers[(size_t)l];
        const bool last = l + 1 == c.layers;
        char* kc = d->kc + l * d->layer_kv * d->kv_elem;
        char* vc = d->vc + l * d->layer_kv * d->kv_elem;
        TRY(qkv(d, L, d->h, d->q, d->k, d->v, 1, s));
        TRY(mth::launch_rope_attention_slices(plain_slices(d->q, QD), plain_slices(d->k, KD), plain_slices(d->v, KD),
                                              ns_attn, d->rope_cos, d->rope_sin, kc, vc, c.kv_dtype == 1, d->att,
                                              d->step, 1, (int)c.heads, (int)c.kv_heads, (int)c.head_dim,
                                              (int)c.max_seq, s));
        ro.gamma = L.ffn_norm;
        ro.ssp = d->ssp2;
        TRY(mth::launch_oil8_gemv_resid(mth::Oil8Seg{L.wo, L.cbo, nullptr, H}, d->att, QD, ro, &ns_ffn.nparts, s));
        if (gate_up_fused(d, L) && mth::oil4_swiglu_supported(L.wgate, L.cbgate, d->h, F, H) &&
            d->c.cb_block == 128 && mth::i2s_swiglu_supported(L.wdown, H, F)) {
            // the SwiGLU in the gate/up epilogue (act in gu[0, F), the
            // maxima of |act| per 8 in gu[F, F + F / 8)), the quantisation
            // inside the down projection
            TRY(mth::launch_oil4_swiglu(L.wgate, L.cbgate, d->h, ns_ffn, d->gu, d->gu + F, F, H, s));
            ro.ssp = d->ssp;
            if (!last) {
                ro.gamma = d->layers[(size_t)l + 1].attn_norm;
                TRY(mth::launch_i2s_act(d->gu, d->gu + F, L.wdown, L.down_scale, nullptr, H, F, ro,
                                        &ns_attn.nparts, s));
            } else {
                TRY(mth::launch_i2s_act(d->gu, d->gu + F, L.wdown, L.down_scale, d->t, H, F, mth::ResidOut{},
                                        nullptr, s));
            }
            continue;
        }
        if (gate_up_fused(d, L)) {
            TRY(oil4(d, L.wgate, L.cbgate, d->h, d->gu, 2 * F, H, s));
        } else {
            TRY(oil4(d, L.wgate, L.cbgate, d->h, d->gu, F, H, s));
            TRY(oil4(d, L.wup, L.cbup, d->h, d->gu + F, F, H, s));
        }
        ro.ssp = d->ssp;
        if (!last) ro.gamma = d->layers[(size_t)l + 1].attn_norm;
        if (mth::i2s_swiglu_supported(L.wdown, H, F)) {
            // SwiGLU + int8 quantisation inside the down projection
            if (!last)
                TRY(mth::launch_i2s_swiglu(d->gu, d->gu + F, ns_ffn, L.wdown, L.down_scale, nullptr, H, F, ro,
                                           &ns_attn.nparts, s));
            else
                TRY(mth::launch_i2s_swiglu(d->gu, d->gu + F, ns_ffn, L.wdown, L.down_scale, d->t, H, F,
                                           mth::ResidOut{}, nullptr, s));
            continue;
        }
        TRY(mth::launch_silu_mul_quant_slices(plain_slices(d->gu, F), plain_slices(d->gu + F, F), ns_ffn, d->aq,
                                              d->a_inv, nullptr, 1, F, s));
        if (!last)
            TRY(mth::launch_i2s_gemv_resid(L.wdown, L.down_scale, d->aq, d->a_inv, H, F, ro, &ns_attn.nparts, s));
        else
            TRY(mth::launch_i2s_gemv(L.wdown, L.down_scale, nullptr, d->aq, d->a_inv, d->t, H, F, 1, s));
    }
    TRY(mth::launch_rms_norm(d->x, d->t, d->g.final_norm, d->h, 1, H, c.eps, s));
    TRY(oil8(d, d->g.lm_idx, d->g.lm_cb, d->h, d->logits, c.vocab, H, s));
    TRY(mth::launch_argmax(d->logits, 1, c.vocab, d->ids, d->hist, d->step, (int)d->hist_stride, (int)d->prompt_len,
                           d->arg_v, d->arg_i, s));
#undef TRY
    return hipSuccess;
}

hipError_t enqueue_step(const mth_decoder* d, hipStream_t s) {
    const mth_decoder_config& c = d->c;
    const int64_t B = d->batch, H = c.hidden, F = c.ffn, QD = c.heads * c.head_dim, KD = c.kv_heads * c.head_dim;
    hipError_t e;
#define TRY(call)                        \
    do {                                 \
        if ((e = (call)) != hipSuccess) return e; \
    } while (0)
    using mth::Slices;
    using mth::plain_slices;
    // Batches of 2..16 leave the Q/K/V, O and down projections' outputs as
    // their split-K partial sums (one token group, in the workspace) and the
    // consumer (the attention, the next norm) adds them: no reduction
    // launches.
    // Each partial buffer is read by the launch right after its producer and
    // only then overwritten.  Taps copy whole outputs, so they take the
    // reduced path (same sums in the same order).
    const bool fold = B >= 2 && B <= 16 && !d->taps;
    // A single sequence splits each RMSNorm over the launches around it
    // (ResidOut / NormScale, common.h): the O and down projections finish
    // the residual stream and write x * gamma of the next norm with partial
    // sums of squares, the Q/K/V and gate/up GEMVs take x * gamma as is, and
    // the attention and the SwiGLU apply 1 / rms: no norm launches but the
    // final one.
    bool fold1 = B == 1 && !d->taps;
    for (int64_t l = 0; fold1 && l < c.layers; l++) {
        const mth_decoder_layer& L = d->layers[(size_t)l];
        const mth::Oil8Seg o_seg{L.wo, L.cbo, nullptr, H};
        fold1 = mth::oil8_segs_fusable(&o_seg, 1, QD) && ((uintptr_t)d->att & 15u) == 0 &&
                (l + 1 == c.layers || mth::i2s_resid_supported(L.wdown, d->aq, H, F));
    }
    if (fold1) return enqueue_step_split_norm(d, s);
    const Slices none{nullptr, 0, 0, 0, 1.0f, nullptr};
    // Batches split the RMSNorms too, but the O and down projections leave
    // split-K partial sums, so the residual add runs as its own wide launch
    // (resid_split: x += partials, x * gamma, partial sums of squares); the
    // Q/K/V and gate/up GEMVs take x * gamma and the attention and the SwiGLU
    // apply 1 / rms.  The embedding writes the first layer's.
    bool splitb = fold && mth::resid_split_parts(H) * B <= H / 4 + 2 &&
                  ((((uintptr_t)d->x | (uintptr_t)d->h) & 15u) == 0);
    for (int64_t l = 0; splitb && l < c.layers; l++) {
        const mth_decoder_layer& L = d->layers[(size_t)l];
        splitb = ((((uintptr_t)L.attn_norm | (uintptr_t)L.ffn_norm) & 15u) == 0) &&
                 mth::resid_split_supported(d->x, none, L.attn_norm, d->h, B, H);
    }
    mth::NormScale ns_attn{}, ns_ffn{};
    if (splitb) {
        ns_attn = mth::NormScale{d->ssp, 1, (float)H, c.eps};
        ns_ffn = mth::NormScale{d->ssp2, 0, (float)H, c.eps};
    }
    const int64_t tap_floats = mth_decoder_tap_floats(d);
    auto tap_copy = [&](float* dst, const void* src, size_t bytes) {
        return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s);
    };
    TRY(mth::launch_embed(d->g.emb, d->hist, d->step, (int)d->hist_stride, d->x, B, (int)H, (int)c.vocab, s,
                          splitb ? mth::ResidOut{d->x, d->layers[0].attn_norm, d->h, d->ssp} : mth::ResidOut{}));
    Slices resid = none;  // the previous layer's FFN output, added by the next norm
    for (int64_t l = 0; l < c.layers; l++) {
        const mth_decoder_layer& L = d->layers[(size_t)l];
        char* kc = d->kc + l * d->layer_kv * d->kv_elem;
        char* vc = d->vc + l * d->layer_kv * d->kv_elem;
        // taps of this layer (mth_decoder_set_taps): x_attn, gu, act, aq, a_inv, down
        float* tp = d->taps ? d->taps + l * tap_floats : nullptr;
        float* tp_gu = tp ? tp + B * H : nullptr;
        float* tp_act = tp ? tp_gu + B * 2 * F : nullptr;
        float* tp_aq = tp ? tp_act + B * F : nullptr;
        float* tp_inv = tp ? tp_aq + B * F / 4 : nullptr;
        float* tp_down = tp ? tp_inv + B : nullptr;
        // residual of the previous layer's FFN folded into this norm
        if (!splitb)
            TRY(mth::launch_rms_norm_slices(d->x, resid, L.attn_norm, d->h, B, H, c.eps, s));
        else if (l > 0)
            TRY(mth::launch_resid_split(d->x, resid, L.attn_norm, d->h, d->ssp, B, H, &ns_attn.nparts, s));
        // Q, K, V, then RoPE + KV append + attention
        Slices sq = plain_slices(d->q, QD), sk = plain_slices(d->k, KD), sv = plain_slices(d->v, KD);
        const mth::Oil8Seg qkv_seg[3] = {{L.wq, L.cbq, d->q, QD}, {L.wk, L.cbk, d->k, KD}, {L.wv, L.cbv, d->v, KD}};
        if (fold && mth::oil8_bt_segs_fusable(qkv_seg, 3, H, B) && mth::oil8_bt_slices(H) <= mth::kMaxSlices) {
            Slices o[3];
            TRY(mth::launch_oil8_gemv_bt_segs_slices(qkv_seg, 3, d->h, H, B, d->bt_partial, o, s));
            sq = o[0], sk = o[1], sv = o[2];
        } else {
            TRY(qkv(d, L, d->h, d->q, d->k, d->v, B, s));
        }
        TRY(mth::launch_rope_attention_slices(sq, sk, sv, ns_attn, d->rope_cos, d->rope_sin, kc, vc,
                                              c.kv_dtype == 1, d->att,
                                              d->step, B, (int)c.heads, (int)c.kv_heads, (int)c.head_dim,
                                              (int)c.max_seq, s));
        // O projection; its output is added to the residual by the FFN norm
        Slices so = plain_slices(d->t, H);
        const mth::Oil8Seg o_seg{L.wo, L.cbo, d->t, H};
        if (fold && mth::oil8_bt_segs_fusable(&o_seg, 1, QD, B) && mth::oil8_bt_slices(QD) <= mth::kMaxSlices &&
            ((uintptr_t)d->att & 15u) == 0) {
            TRY(mth::launch_oil8_gemv_bt_segs_slices(&o_seg, 1, d->att, QD, B, d->bt_partial, &so, s));
        } else {
            TRY(oil8(d, L.wo, L.cbo, d->att, d->t, H, QD, s));
        }
        if (splitb)
            TRY(mth::launch_resid_split(d->x, so, L.ffn_norm, d->h, d->ssp2, B, H, &ns_ffn.nparts, s));
        else
            TRY(mth::launch_rms_norm_slices(d->x, so, L.ffn_norm, d->h, B, H, c.eps, s));
        if (tp) TRY(tap_copy(tp, d->x, (size_t)(B * H) * 4));
        const bool fused = gate_up_fused(d, L);
        // Split norm: the SwiGLU in the gate/up projection's K-slice
        // reduction (act over gu's gate half, block maxima in amx) and the
        // per-token int8 quantisation inside the ternary GEMV: no SwiGLU launch
        if (fused && splitb && mth::oil4_bt_swiglu_parts(F) <= kAmxParts &&
            mth::oil4_bt_swiglu_supported(F, H, c.cb_block, B) && mth::i2s_bt_supported(H, F, B) &&
            ((((uintptr_t)L.wgate | (uintptr_t)L.cbgate | (uintptr_t)d->h | (uintptr_t)L.wdown) & 15u) == 0)) {
            TRY(mth::launch_oil4_gemv_bt_swiglu(L.wgate, L.cbgate, c.cb_block, d->h, ns_ffn, d->gu, d->amx, F, H, B,
                                                d->bt_partial, s));
            TRY(mth::launch_i2s_gemv_bt_f32act(L.wdown, L.down_scale, d->gu, 2 * F, d->amx,
                                               mth::oil4_bt_swiglu_parts(F), d->a_inv, d->t, H, F, B, d->bt_partial,
                                               &resid, s));
            continue;
        }
        // gate/up, then silu(gate)*up quantised to int8 per token (once, not
        // per workgroup of the down projection), then the ternary GEMV on the
        // int8 activations
        if (fused) {
            const Slices sg = plain_slices(d->gu, 2 * F), su = plain_slices(d->gu + F, 2 * F);
            // (reduced here: the SwiGLU has one workgroup per token, too few
            // to read the gate/up slices as fast as the reduction kernel)
            TRY(oil4(d, L.wgate, L.cbgate, d->h, d->gu, 2 * F, H, s));
            if (tp) TRY(tap_copy(tp_gu, d->gu, (size_t)(B * 2 * F) * 4));
            TRY(mth::launch_silu_mul_quant_slices(sg, su, ns_ffn, d->aq, d->a_inv, tp_act, B, F, s));
        } else {
            TRY(oil4(d, L.wgate, L.cbgate, d->h, d->gu, F, H, s));
            TRY(oil4(d, L.wup, L.cbup, d->h, d->gu + B * F, F, H, s));
            if (tp) {  // gate [B][F] and up [B][F] -> [B][gate, up]
                TRY(hipMemcpy2DAsync(tp_gu, (size_t)(2 * F) * 4, d->gu, (size_t)F * 4, (size_t)F * 4, (size_t)B,
                                     hipMemcpyDeviceToDevice, s));
                TRY(hipMemcpy2DAsync(tp_gu + F, (size_t)(2 * F) * 4, d->gu + B * F, (size_t)F * 4, (size_t)F * 4,
                                     (size_t)B, hipMemcpyDeviceToDevice, s));
            }
            if (splitb)
                TRY(mth::launch_silu_mul_quant_slices(plain_slices(d->gu, F), plain_slices(d->gu + B * F, F), ns_ffn,
                                                      d->aq, d->a_inv, tp_act, B, F, s));
            else
                TRY(mth::launch_silu_mul_quant(d->gu, d->gu + B * F, d->aq, d->a_inv, tp_act, B, F, F, F, s));
        }
        resid = plain_slices(d->t, H);
        if ((((uintptr_t)L.wdown | (uintptr_t)d->aq) & 15u) == 0 && mth::i2s_bt_supported(H, F, B)) {
            if (fold)
                TRY(mth::launch_i2s_gemv_bt_slices(L.wdown, L.down_scale, d->aq, d->a_inv, d->t, H, F, B,
                                                   d->bt_partial, &resid, s));
            else
                TRY(mth::launch_i2s_gemv_bt(L.wdown, L.down_scale, d->aq, d->a_inv, d->t, H, F, B, d->bt_partial, s));
        } else {
            TRY(mth::launch_i2s_gemv(L.wdown, L.down_scale, nullptr, d->aq, d->a_inv, d->t, H, F, B, s));
        }
        if (tp) {
            TRY(tap_copy(tp_aq, d->aq, (size_t)(B * F)));
            TRY(tap_copy(tp_inv, d->a_inv, (size_t)B * 4));
            TRY(tap_copy(tp_down, d->t, (size_t)(B * H) * 4));
        }
    }
    TRY(mth::launch_rms_norm_slices(d->x, resid, d->g.final_norm, d->h, B, H, c.eps, s));
    TRY(oil8(d, d->g.lm_idx, d->g.lm_cb, d->h, d->logits, c.vocab, H, s));
    TRY(mth::launch_argmax(d->logits, B, c.vocab, d->ids, d->hist, d->step, (int)d->hist_stride, (int)d->prompt_len,
                           d->arg_v, d->arg_i, s));
#undef TRY
    return hipSuccess;
}

}  // namespace

extern "C" {

int mth_decoder_create(const mth_decoder_config* cfg, mth_decoder** out) {
    if (!cfg || !out) return api_fail(MTH_EINVAL, "mth_decoder_create: null pointer");
    *out = nullptr;
    if (cfg->struct_size != (int64_t)sizeof(mth_decoder_config))
        return api_fail(MTH_EINVAL,
                        "mth_decoder_create: struct_size=%lld, this library's mth_decoder_config has %zu bytes "
                        "(caller built against another header version; ABI %d.%d)",
                        (long long)cfg->struct_size, sizeof(mth_decoder_config), mth_version() >> 16,
                        mth_version() & 0xffff);
    const mth_decoder_config& c = *cfg;
    if (c.vocab <= 0 || c.hidden <= 0 || c.layers <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.ffn <= 0 ||
        c.head_dim <= 0 || c.max_seq <= 0 || c.vocab >= (1ll << 31) || c.hidden >= (1ll << 24) ||
        c.ffn >= (1ll << 24) || c.layers > 4096)
        return api_fail(MTH_EINVAL, "mth_decoder_create: bad sizes");
    if (c.max_batch < 1 || c.max_batch > 16)
        return api_fail(MTH_EINVAL, "mth_decoder_create: max_batch=%lld outside 1..16", (long long)c.max_batch);
    if (c.hidden % 4 != 0 || c.ffn % 4 != 0)
        return api_fail(MTH_EINVAL, "mth_decoder_create: hidden and ffn must be multiples of 4");
    if (!mth::silu_mul_quant_supported(c.ffn))
        return api_fail(MTH_EUNSUPPORTED, "mth_decoder_create: ffn=%lld above 12288", (long long)c.ffn);
    if (c.heads % c.kv_heads != 0) return api_fail(MTH_EINVAL, "mth_decoder_create: heads %% kv_heads != 0");
    if (c.kv_dtype != 0 && c.kv_dtype != 1)
        return api_fail(MTH_EINVAL, "mth_decoder_create: kv_dtype=%lld (0 = FP32, 1 = bf16)", (long long)c.kv_dtype);
    if (c.cb_block < 0 || (c.cb_block > 0 && c.hidden % c.cb_block != 0))
        return api_fail(MTH_EINVAL, "mth_decoder_create: cb_block=%lld does not divide hidden", (long long)c.cb_block);
    if (!mth::attention_supported((int)c.head_dim, (int)c.max_seq))
        return api_fail(MTH_EUNSUPPORTED, "mth_decoder_create: head_dim=%lld / max_seq=%lld not supported "
                                          "(head_dim 64, 128 or 256; max_seq <= 16384)",
                        (long long)c.head_dim, (long long)c.max_seq);
    if (!(c.eps >= 0.0f) || !(c.theta > 0.0f)) return api_fail(MTH_EINVAL, "mth_decoder_create: bad eps/theta");

    mth_decoder* d = new mth_decoder;
    d->c = c;
    d->layers.assign((size_t)c.layers, mth_decoder_layer{});
    d->layer_set.assign((size_t)c.layers, false);
    hipError_t e = hipGetDevice(&d->device);
    const int64_t B = c.max_batch, H = c.hidden, F = c.ffn;
    const int64_t QD = c.heads * c.head_dim, KD = c.kv_heads * c.head_dim;
    d->hist_stride = c.max_seq + 1;
    d->layer_kv = B * KD * c.max_seq;
    d->kv_elem = c.kv_dtype == 1 ? 2 : 4;
    // prefill chunk: up to 1024 rows of (sequence, position)
    const int64_t PR = std::min<int64_t>(B * c.max_seq, 1024);
    d->pf_rows = PR;
    // workspace of the batched GEMVs: the largest of every projection's need
    const size_t partial = std::max({mth::oil4_bt_partial_bytes(2 * F, H), mth::oil8_bt_partial_bytes(QD + 2 * KD, H),
                                     mth::oil8_bt_partial_bytes(H, QD),
                                     mth::oil8_bt_partial_bytes(c.vocab, H), mth::i2s_bt_partial_bytes(H, F)});
    struct Slot {
        void** p;
        size_t bytes;
    } slots[] = {
        {(void**)&d->x, (size_t)(B * H) * 4},       {(void**)&d->h, (size_t)(B * H) * 4},
        {(void**)&d->t, (size_t)(B * H) * 4},       {(void**)&d->q, (size_t)(B * QD) * 4},
        {(void**)&d->k, (size_t)(B * KD) * 4},      {(void**)&d->v, (size_t)(B * KD) * 4},
        {(void**)&d->att, (size_t)(B * QD) * 4},    {(void**)&d->gu, (size_t)(B * 2 * F) * 4},
        {(void**)&d->aq, (size_t)(B * F)},          {(void**)&d->a_inv, (size_t)B * 4},
        {(void**)&d->logits, (size_t)(B * c.vocab) * 4},
        {(void**)&d->arg_v, (size_t)(B * mth::argmax_chunks(c.vocab)) * 4},
        {(void**)&d->arg_i, (size_t)(B * mth::argmax_chunks(c.vocab)) * 4},
        {(void**)&d->kc, (size_t)(c.layers * d->layer_kv) * d->kv_elem},
        {(void**)&d->vc, (size_t)(c.layers * d->layer_kv) * d->kv_elem},
        {(void**)&d->rope_cos, (size_t)(c.max_seq * (c.head_dim / 2)) * 4},
        {(void**)&d->rope_sin, (size_t)(c.max_seq * (c.head_dim / 2)) * 4},
        {(void**)&d->bt_partial, partial},
        {(void**)&d->hist, (size_t)(B * d->hist_stride) * 4},
        {(void**)&d->step, 4},                      {(void**)&d->ids, (size_t)B * 4},
        {(void**)&d->pf_x, (size_t)(PR * H) * 4},   {(void**)&d->pf_h, (size_t)(PR * H) * 4},
        {(void**)&d->pf_t, (size_t)(PR * H) * 4},   {(void**)&d->pf_q, (size_t)(PR * QD) * 4},
        {(void**)&d->pf_k, (size_t)(PR * KD) * 4},  {(void**)&d->pf_v, (size_t)(PR * KD) * 4},
        {(void**)&d->pf_att, (size_t)(PR * QD) * 4}, {(void**)&d->pf_gu, (size_t)(PR * 2 * F) * 4},
        {(void**)&d->pf_aq, (size_t)(PR * F)},      {(void**)&d->pf_inv, (size_t)PR * 4},
        {(void**)&d->ssp, (size_t)(H / 4 + 2) * 8},  {(void**)&d->ssp2, (size_t)(H / 4 + 2) * 8},
        {(void**)&d->amx, (size_t)(B * kAmxParts) * 4},
        {(void**)&d->pf_ws, PR >= kPfGemmRows ? std::max({mth::oil4_gemm_x32_workspace_bytes(PR, H),
                                                          mth::oil8_gemm_x32_workspace_bytes(PR, H),
                                                          mth::oil8_gemm_x32_workspace_bytes(PR, QD)})
                                              : (size_t)0},
    };
    size_t total = 0;
    for (const Slot& sl : slots) total += round_up(sl.bytes);
    if (e == hipSuccess) e = hipMalloc(&d->block, total);
    if (e != hipSuccess) {
        delete d;
        return api_fail(MTH_EDEVICE, "mth_decoder_create: allocating %zu bytes failed: %s", total,
                        hipGetErrorString(e));
    }
    size_t off = 0;
    for (const Slot& sl : slots) {
        *sl.p = sl.bytes ? (char*)d->block + off : nullptr;
        off += round_up(sl.bytes);
    }
    // RotaryEmbedding tables (src/transformer.cpp:102-117), float arithmetic
    // on the host, as the reference computes them
    const int64_t h2 = c.head_dim / 2;
    std::vector<float> cs((size_t)(c.max_seq * h2)), sn((size_t)(c.max_seq * h2));
    for (int64_t i = 0; i < c.max_seq; i++)
        for (int64_t j = 0; j < h2; j++) {
            const float inv_freq = 1.0f / std::pow(c.theta, (float)(2 * j) / (float)c.head_dim);
            const float val = (float)i * inv_freq;
            cs[(size_t)(i * h2 + j)] = std::cos(val);
            sn[(size_t)(i * h2 + j)] = std::sin(val);
        }
    e = hipMemcpy(d->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(d->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&d->cap_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        mth_decoder_destroy(d);
        return api_fail(MTH_EDEVICE, "mth_decoder_create: %s", hipGetErrorString(e));
    }
    *out = d;
    return api_ok();
}

void mth_decoder_destroy(mth_decoder* d) {
    if (!d) return;
    d->drop_graph();
    if (d->cap_stream) (void)hipStreamDestroy(d->cap_stream);
    if (d->block) (void)hipFree(d->block);
    delete d;
}

int mth_decoder_set_layer(mth_decoder* d, int64_t layer, const mth_decoder_layer* w) {
    if (!d || !w) return api_fail(MTH_EINVAL, "mth_decoder_set_layer: null pointer");
    if (layer < 0 || layer >= d->c.layers)
        return api_fail(MTH_EINVAL, "mth_decoder_set_layer: layer %lld outside 0..%lld", (long long)layer,
                        (long long)d->c.layers - 1);
    if (!w->attn_norm || !w->ffn_norm || !w->wq || !w->wk || !w->wv || !w->wo || !w->cbq || !w->cbk || !w->cbv ||
        !w->cbo || !w->wgate || !w->wup || !w->cbgate || !w->cbup || !w->wdown)
        return api_fail(MTH_EINVAL, "mth_decoder_set_layer: null weight pointer in layer %lld", (long long)layer);
    d->layers[(size_t)layer] = *w;
    d->layer_set[(size_t)layer] = true;
    d->drop_graph();
    return api_ok();
}

int mth_decoder_set_globals(mth_decoder* d, const mth_decoder_globals* g) {
    if (!d || !g || !g->emb || !g->final_norm || !g->lm_idx || !g->lm_cb)
        return api_fail(MTH_EINVAL, "mth_decoder_set_globals: null pointer");
    d->g = *g;
    d->globals_set = true;
    d->drop_graph();
    return api_ok();
}

int mth_decoder_start(mth_decoder* d, const int32_t* prompts, int64_t batch, int64_t prompt_len,
                      mth_stream_t stream) {
    if (!d || !prompts) return api_fail(MTH_EINVAL, "mth_decoder_start: null pointer");
    if (batch < 1 || batch > d->c.max_batch)
        return api_fail(MTH_EINVAL, "mth_decoder_start: batch=%lld outside 1..%lld", (long long)batch,
                        (long long)d->c.max_batch);
    if (prompt_len < 1 || prompt_len > d->c.max_seq)
        return api_fail(MTH_EINVAL, "mth_decoder_start: prompt_len=%lld outside 1..%lld", (long long)prompt_len,
                        (long long)d->c.max_seq);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipMemcpy2DAsync(d->hist, (size_t)d->hist_stride * 4, prompts, (size_t)prompt_len * 4,
                                    (size_t)prompt_len * 4, (size_t)batch, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipMemsetAsync(d->step, 0, 4, s);
    if (e != hipSuccess) return api_fail(MTH_EDEVICE, "mth_decoder_start: %s", hipGetErrorString(e));
    d->batch = batch;
    d->prompt_len = prompt_len;
    d->steps = 0;
    return api_ok();
}

int mth_decoder_step(mth_decoder* d, int64_t n, int use_graph, mth_stream_t stream) {
    if (!d) return api_fail(MTH_EINVAL, "mth_decoder_step: null decoder");
    if (d->batch == 0) return api_fail(MTH_EINVAL, "mth_decoder_step: no sequences started");
    for (int64_t l = 0; l < d->c.layers; l++)
        if (!d->layer_set[(size_t)l]) return api_fail(MTH_EINVAL, "mth_decoder_step: layer %lld has no weights",
                                                      (long long)l);
    if (!d->globals_set) return api_fail(MTH_EINVAL, "mth_decoder_step: embedding / lm_head not set");
    if (n < 0 || d->steps + n > d->c.max_seq)
        return api_fail(MTH_EINVAL, "mth_decoder_step: %lld steps after %lld exceed max_seq=%lld", (long long)n,
                        (long long)d->steps, (long long)d->c.max_seq);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipSuccess;
    if (use_graph && !d->taps) {
        if (d->exec && (d->graph_batch != d->batch || d->graph_prompt != d->prompt_len)) d->drop_graph();
        if (!d->exec) {
            e = hipStreamBeginCapture(d->cap_stream, hipStreamCaptureModeThreadLocal);
            if (e == hipSuccess) {
                const hipError_t le = enqueue_step(d, d->cap_stream);
                e = hipStreamEndCapture(d->cap_stream, &d->graph);
                if (le != hipSuccess) e = le;
            }
            if (e == hipSuccess) e = hipGraphGetNodes(d->graph, nullptr, &d->graph_nodes);
            if (e == hipSuccess) e = hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0);
            if (e != hipSuccess) {
                d->drop_graph();
                return api_fail(MTH_EDEVICE, "mth_decoder_step: graph capture failed: %s", hipGetErrorString(e));
            }
            d->graph_batch = d->batch;
            d->graph_prompt = d->prompt_len;
        }
        for (int64_t i = 0; i < n && e == hipSuccess; i++) e = hipGraphLaunch(d->exec, s);
    } else {
        for (int64_t i = 0; i < n && e == hipSuccess; i++) e = enqueue_step(d, s);
    }
    if (e != hipSuccess) return api_fail(MTH_EDEVICE, "mth_decoder_step: %s", hipGetErrorString(e));
    d->steps += n;
    return api_ok();
}

int mth_decoder_prefill(mth_decoder* d, mth_stream_t stream) {
    if (!d) return api_fail(MTH_EINVAL, "mth_decoder_prefill: null decoder");
    if (d->batch == 0) return api_fail(MTH_EINVAL, "mth_decoder_prefill: no sequences started");
    if (d->steps != 0)
        return api_fail(MTH_EINVAL, "mth_decoder_prefill: %lld steps already run since the start",
                        (long long)d->steps);
    for (int64_t l = 0; l < d->c.layers; l++)
        if (!d->layer_set[(size_t)l]) return api_fail(MTH_EINVAL, "mth_decoder_prefill: layer %lld has no weights",
                                                      (long long)l);
    if (!d->globals_set) return api_fail(MTH_EINVAL, "mth_decoder_prefill: embedding / lm_head not set");
    const hipError_t e = enqueue_prefill(d, (hipStream_t)stream);
    if (e != hipSuccess) return api_fail(MTH_EDEVICE, "mth_decoder_prefill: %s", hipGetErrorString(e));
    d->steps = d->prompt_len;
    return api_ok();
}

int mth_decoder_buffers(const mth_decoder* d, float** logits, int32_t** hist, int64_t* hist_stride) {
    if (!d) return api_fail(MTH_EINVAL, "mth_decoder_buffers: null decoder");
    if (logits) *logits = d->logits;
    if (hist) *hist = d->hist;
    if (hist_stride) *hist_stride = d->hist_stride;
    return api_ok();
}

int mth_decoder_read(const mth_decoder* d, float* logits, int32_t* hist, mth_stream_t stream) {
    if (!d) return api_fail(MTH_EINVAL, "mth_decoder_read: null decoder");
    if (d->batch == 0) return api_fail(MTH_EINVAL, "mth_decoder_read: no sequences started");
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipSuccess;
    if (logits) e = hipMemcpyAsync(logits, d->logits, (size_t)(d->batch * d->c.vocab) * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && hist)
        e = hipMemcpyAsync(hist, d->hist, (size_t)(d->batch * d->hist_stride) * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return api_fail(MTH_EDEVICE, "mth_decoder_read: %s", hipGetErrorString(e));
    return api_ok();
}

int64_t mth_decoder_steps_done(const mth_decoder* d) { return d ? d->steps : 0; }

int64_t mth_decoder_launches(const mth_decoder* d) { return d && d->exec ? (int64_t)d->graph_nodes : 0; }

int64_t mth_decoder_tap_floats(const mth_decoder* d) {
    if (!d) return 0;
    const int64_t B = d->batch, H = d->c.hidden, F = d->c.ffn;
    return B * (2 * H + 3 * F + F / 4 + 1);
}

int mth_decoder_read_kv(const mth_decoder* d, int64_t layer, void* k, void* v, mth_stream_t stream) {
    if (!d) return api_fail(MTH_EINVAL, "mth_decoder_read_kv: null decoder");
    if (d->batch == 0) return api_fail(MTH_EINVAL, "mth_decoder_read_kv: no sequences started");
    if (layer < 0 || layer >= d->c.layers)
        return api_fail(MTH_EINVAL, "mth_decoder_read_kv: layer %lld outside 0..%lld", (long long)layer,
                        (long long)d->c.layers - 1);
    hipStream_t s = (hipStream_t)stream;
    // rows of the started batch: the first batch * kv_heads * max_seq * head_dim elements of the layer
    const size_t bytes = (size_t)(d->batch * d->c.kv_heads * d->c.max_seq * d->c.head_dim) * d->kv_elem;
    const size_t off = (size_t)(layer * d->layer_kv) * d->kv_elem;
    hipError_t e = hipSuccess;
    if (k) e = hipMemcpyAsync(k, d->kc + off, bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && v) e = hipMemcpyAsync(v, d->vc + off, bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return api_fail(MTH_EDEVICE, "mth_decoder_read_kv: %s", hipGetErrorString(e));
    return api_ok();
}

int mth_decoder_set_taps(mth_decoder* d, float* taps) {
    if (!d) return api_fail(MTH_EINVAL, "mth_decoder_set_taps: null decoder");
    if (taps && d->batch == 0) return api_fail(MTH_EINVAL, "mth_decoder_set_taps: no sequences started");
    d->taps = taps;
    return api_ok();
}

}  // extern "C"
