/*
 * mythos_decoder.h — the mixed-format decoder stack on one MI355X
 * (libmythos_oil.so): Q/K/V/O and lm_head OIL8, FFN gate/up OIL4 with
 * per-block codebooks, FFN down ternary I2_S with per-token int8 activations,
 * RMSNorm, rotary embedding, attention over an FP32 or bf16 KV cache, greedy
 * argmax.
 *
 * Replaces, for this weight format mix, the reference's inference path
 * DenseModel::forward (src/model.cpp:45-75) -> TransformerBlock::forward
 * (src/transformer.cpp:396-406) -> Attention::forward inference branch
 * (:154-362) / FFN::forward (:373-387), driven token by token as
 * Generator::generate_tokens does (src/generator.cpp:14-64) with
 * Sampler::greedy (src/sampler.cpp:12-22).  Semantics that differ on purpose:
 * every layer rotates at the token's own position (the reference reads layer
 * 0's cache length, src/kv_cache.cpp:190-192); the softmax uses exp (not the
 * AVX2 build's Taylor polynomial, src/transformer.cpp:255-276); one KV cache
 * per sequence of the batch (the reference's is batch-1); weights are
 * [out][in] rows (the reference Linear holds them input-major).
 *
 * The caller owns the weights (device pointers, kernels' layouts as in
 * mythos_oil.h) and must keep them alive while the decoder runs.  The decoder
 * owns its KV cache, activations and token history, allocated on the current
 * device at create.  One step feeds one token per sequence: step s reads
 * token hist[b][s] (the prompt while s < prompt_len, then the previous step's
 * argmax), runs the stack at position s, and writes logits[b][vocab] and
 * hist[b][s + 1].  The step counter lives on the device, so a step is one
 * fixed launch sequence, replayed as a HIP graph.  Calls on one decoder must
 * be ordered on one stream.
 */
#ifndef MYTHOS_DECODER_H
#define MYTHOS_DECODER_H

#include <stdint.h>

#include "mythos_oil.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mth_decoder mth_decoder;

typedef struct {
    /* sizeof(mth_decoder_config) as the caller was compiled: mth_decoder_create
     * rejects any other value, so a caller built against another layout of
     * this struct fails cleanly instead of being misread (ABI major 2). */
    int64_t struct_size;
    int64_t vocab, hidden, layers, heads, kv_heads, head_dim, ffn;
    int64_t max_seq;   /* KV-cache positions per sequence (prompt + generated) */
    int64_t cb_block;  /* OIL4 codebook block length (0 = one codebook per tensor) */
    int64_t max_batch; /* sequences decoded together, 1..16 */
    float eps, theta;  /* RMSNorm epsilon, RoPE base */
    /* KV-cache element type: 0 = FP32 (KVCache's Tensor, src/kv_cache.cpp:61-62),
     * 1 = bf16: K (after RoPE) and V rounded to nearest even when appended,
     * attention reads them back exactly; half the cache bytes. */
    int64_t kv_dtype;
} mth_decoder_config;

typedef struct {
    const float* attn_norm;   /* [hidden] */
    const float* ffn_norm;    /* [hidden] */
    const uint8_t *wq, *wk, *wv, *wo; /* OIL8 [out][in] indices */
    const float *cbq, *cbk, *cbv, *cbo; /* 256-entry FP32 codebooks */
    /* OIL4 [ffn][hidden/2] nibbles and [ffn][hidden/cb_block][16] FP16
     * codebooks.  When wup directly follows wgate (and cbup cbgate) in memory,
     * both run as one launch over 2*ffn rows. */
    const uint8_t *wgate, *wup;
    const uint16_t *cbgate, *cbup;
    const uint8_t* wdown;     /* I2_S [hidden][ffn/4] */
    float down_scale;
} mth_decoder_layer;

typedef struct {
    const float* emb;         /* [vocab][hidden] FP32 */
    const float* final_norm;  /* [hidden] */
    const uint8_t* lm_idx;    /* OIL8 [vocab][hidden] */
    const float* lm_cb;
} mth_decoder_globals;

int mth_decoder_create(const mth_decoder_config* cfg, mth_decoder** out);
void mth_decoder_destroy(mth_decoder* d);
int mth_decoder_set_layer(mth_decoder* d, int64_t layer, const mth_decoder_layer* w);
int mth_decoder_set_globals(mth_decoder* d, const mth_decoder_globals* g);

/* Starts `batch` sequences: prompts [batch][prompt_len] int32 token ids
 * (device), 1 <= prompt_len <= max_seq.  Resets the step counter. */
int mth_decoder_start(mth_decoder* d, const int32_t* prompts, int64_t batch, int64_t prompt_len, mth_stream_t stream);

/* Runs n steps (n + steps already run <= max_seq).  use_graph: capture one
 * step into a HIP graph on first use and replay it. */
int mth_decoder_step(mth_decoder* d, int64_t n, int use_graph, mth_stream_t stream);

/* Device buffers: logits [batch][vocab] of the last step, and the token
 * history [batch][max_seq + 1] (row b: prompt, then generated ids). */
int mth_decoder_buffers(const mth_decoder* d, float** logits, int32_t** hist, int64_t* hist_stride);

/* Host copies (synchronous, after the stream's queued work): logits
 * [batch][vocab] and token history [batch][max_seq + 1]; either may be null. */
int mth_decoder_read(const mth_decoder* d, float* logits, int32_t* hist, mth_stream_t stream);

/* The whole prompt as one forward pass (src/generator.cpp:33-38: prefill,
 * then sampling of the last position): every prompt position of every
 * started sequence runs through the layer stack as a row of batched launches
 * (chunks of up to 1024 rows), filling the KV caches, then the last
 * positions' logits give the first generated token.  Afterwards the decoder
 * is where prompt_len mth_decoder_step calls would leave it (steps done =
 * prompt_len, logits and history likewise), so decoding continues with
 * mth_decoder_step.  Only right after mth_decoder_start (MTH_EINVAL
 * otherwise).  Runs its launches directly on the stream (no graph). */
int mth_decoder_prefill(mth_decoder* d, mth_stream_t stream);

/* Steps run since the last start (host-side count). */
int64_t mth_decoder_steps_done(const mth_decoder* d);

/* Kernel launches of one step: the nodes of the captured step graph (every
 * node is a kernel), 0 before the first graph step of the started batch.
 * For measurement (no reference counterpart). */
int64_t mth_decoder_launches(const mth_decoder* d);

/* Per-layer intermediate values, for parity tests and debugging (no
 * reference counterpart).  With taps non-null, every later step runs its
 * launches directly (no graph) and copies, for layer l, into
 * taps + l * mth_decoder_tap_floats(d), in this order, B = the started batch:
 *   x_attn [B][hidden]  residual stream after the attention half
 *   gu     [B][2*ffn]   gate outputs then up outputs, per token
 *   act    [B][ffn]     silu(gate) * up in FP32, before quantisation
 *   aq     [B][ffn]     its int8 quantisation (bytes: B*ffn/4 floats of storage)
 *   a_inv  [B]          per-token inverse scale of aq
 *   down   [B][hidden]  the ternary down projection (added to x_attn next)
 * taps: device memory of layers * mth_decoder_tap_floats(d) floats; null
 * turns the taps off.  Valid after mth_decoder_start (the batch sets the size). */
int mth_decoder_set_taps(mth_decoder* d, float* taps);
int64_t mth_decoder_tap_floats(const mth_decoder* d);

/* Host copy (synchronous) of layer `layer`'s K and V caches, each
 * [batch][kv_heads][max_seq][head_dim] of the cache's element type (FP32, or
 * bf16 bits as uint16 with kv_dtype 1) for the started batch; either pointer
 * may be null.  Positions not yet written hold zeros or older values.  For
 * parity tests and debugging (no reference counterpart). */
int mth_decoder_read_kv(const mth_decoder* d, int64_t layer, void* k, void* v, mth_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
