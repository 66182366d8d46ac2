/*
 * mythos_oil.h — C ABI of libmythos_oil.so: MI355X (gfx950) kernels for
 * MYTHOS.cpp's quantized-weight matvec/matmul path.
 *
 * Every entry point takes DEVICE pointers (memory the caller allocated with
 * hipMalloc or any HIP allocator), plain sizes and a HIP stream (hipStream_t
 * passed as void*; NULL = the default stream).  Calls are stream-ordered and
 * asynchronous: they validate, launch and return.  Outputs are overwritten,
 * never accumulated.
 *
 * Workspace.  The batched GEMVs (mth_oil8_gemv, mth_oil4_gemv, mth_i2s_gemv
 * with batch >= 2; for batches of >= 128 tokens mth_oil8_gemv and
 * mth_oil4_gemv run as MFMA GEMMs and keep each token row's FP16 hi / lo parts,
 * 4 * K bytes per token rounded up to 128 (OIL4) or 256 (OIL8) tokens,
 * plus 4 bytes per token),
 * mth_argmax, mth_oil4_gemm_prefill (per-row shifts of A,
 * 4 bytes per row, and an FP16 copy of A in MFMA fragment order,
 * ceil(M/16)*16*K*2 bytes, for K % 256 == 0, codebook blocks of a multiple
 * of 128 and N a multiple of 64, 96 or 112), mth_tl2_gemm (each activation
 * row quantised once: N * ceil(K/4) * 4 bytes plus 4 bytes per row, when
 * ceil(K/4) % 16 == 0) keep intermediate data in a device workspace
 * the library owns, one per (device, stream).  The first call that needs more
 * than the stream's workspace holds allocates a larger one (hipMalloc, at
 * least double the old size) and retires the old block WITHOUT freeing it, so
 * work queued earlier and HIP graphs captured earlier from that stream keep
 * valid addresses until the process ends.  No other entry point allocates.
 * Inside a stream capture a call never allocates: if the workspace is too
 * small it fails with MTH_EUNSUPPORTED, so reserve the size beforehand with
 * mth_workspace_reserve (or make one uncaptured call of the largest shape).
 * Calls on one stream share its workspace; a captured graph uses the
 * workspace of the stream it was captured on and must not be replayed
 * concurrently with other work that uses that stream's workspace.
 *
 * Return value: MTH_OK (0) or a negative MTH_E* code; the thread-local message
 * of the last failure is returned by mth_last_error().  Validation covers
 * NULL pointers, non-positive or inconsistent sizes, and the layout
 * constraints stated per function.  Unaligned or odd-sized inputs are not
 * errors: they run on the generic kernels.
 *
 * Each function names the reference interface it replaces
 * (path:line in the MYTHOS.cpp tree).  Host-pointer, synchronous drop-ins with
 * the reference's exact C++ signatures (namespace oil::kernel) are declared in
 * mythos.cpp_amd/host/include/oil/kernel.h and call these.
 */
#ifndef MYTHOS_OIL_H
#define MYTHOS_OIL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mth_stream_t; /* hipStream_t */

enum {
    MTH_OK = 0,
    MTH_EINVAL = -1,       /* bad pointer / size / layout argument          */
    MTH_EDEVICE = -2,      /* HIP runtime or launch failure                 */
    MTH_EUNSUPPORTED = -3, /* valid request this build does not implement    */
};

/* Message of the last failing call on this thread ("" if none). */
const char* mth_last_error(void);
/* ABI version: (major << 16) | minor. */
int mth_version(void);

/* Ensures the calling thread's current device holds at least `bytes` of
 * workspace for `stream` (see "Workspace" above); call it before capturing
 * batched GEMVs into a graph.  No reference counterpart: the reference's CPU
 * kernels keep no device state. */
int mth_workspace_reserve(int64_t bytes, mth_stream_t stream);

/* ---------------------------------------------------------------- OIL8 -- */

/* Reference semantics of oil::kernel::oil8_gemm (include/oil/kernel.h:33-35,
 * src/kernel_oil8.cpp:63-71): for every (m, n)
 *   out[m*N + n] = sum_k codebook[indices[(m*N + n)*K + k]] * act[n*K + k]
 * i.e. one weight row per (m, n) pair.  codebook: 256 floats. */
int mth_oil8_gemm(const uint8_t* indices, const float* codebook, const float* act, float* out,
                  int64_t M, int64_t N, int64_t K, mth_stream_t stream);

/* Decode GEMV over one OIL8 weight matrix shared by `batch` tokens (the
 * reference's oil8_gemm with N = 1, once per token, src/kernel_oil8.cpp:30-60):
 *   y[t*M + m] = sum_k codebook[indices[m*K + k]] * x[t*K + k],  t < batch.
 * Fast path: K % 16 == 0, K <= 4096, indices and x 16-byte aligned.  Batches
 * of >= 128 tokens with M % 64 == 0, K % 256 == 0 and 16-byte aligned y run
 * as the prompt prefill's MFMA GEMM (FP16 hi / lo parts of x and codebook,
 * FP32 sums: the FP32 bar; rows or codebooks holding Inf / NaN take FP32
 * products). */
int mth_oil8_gemv(const uint8_t* indices, const float* codebook, const float* x, float* y,
                  int64_t M, int64_t K, int64_t batch, mth_stream_t stream);

/* ---------------------------------------------------------------- OIL4 -- */

/* Reference semantics of oil::kernel::oil4_gemm (include/oil/kernel.h:39-41,
 * scalar path src/kernel_oil4.cpp:31-54): one 16-entry FP16 codebook,
 *   out[m*N + n] = sum_k f32(codebook[nib(r, k)]) * act[n*K + k],  r = m*N + n,
 * where the weight row r starts at byte (r*K)/2 and element k is the low
 * nibble of byte k/2 for even k, the high nibble for odd k.  The reference's
 * AVX2 build adds codebook[0]*sum(act[k<16*floor(K/16)]) on top (a load-width
 * bug); this entry point computes the scalar definition. */
int mth_oil4_gemm(const uint8_t* packed, const uint16_t* codebook, const float* act, float* out,
                  int64_t M, int64_t N, int64_t K, mth_stream_t stream);

/* Decode GEMV with per-block FP16 codebooks (the layout the BASELINE configs
 * use; the reference kernel takes one codebook per call):
 *   y[t*M + m] = sum_k f32(codebooks[(m*(K/cb_block) + k/cb_block)*16 + nib(m,k)]) * x[t*K + k]
 * packed: M rows of K/2 bytes, nibble order as above.  cb_block = 0 selects
 * a single shared 16-entry codebook.  Requires K even and, for cb_block > 0,
 * K % cb_block == 0.  Fast path: K % 32 == 0, K <= 4096, cb_block % 32 == 0,
 * 16-byte aligned packed / codebooks / x.  Batches of >= 128 tokens with
 * cb_block a multiple of 128, K % 256 == 0, M a multiple of 64, 96, 112 or
 * 128 and 16-byte aligned y run as the prompt prefill's MFMA GEMM (FP16 hi /
 * lo parts of x, FP32 sums). */
int mth_oil4_gemv(const uint8_t* packed, const uint16_t* codebooks, int64_t cb_block,
                  const float* x, float* y, int64_t M, int64_t K, int64_t batch,
                  mth_stream_t stream);

/* mth_oil4_gemv for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference (its CPU kernels need no scratch).  Same
 * arguments, results and kernels as mth_oil4_gemv; the batched path's K-slice
 * partial sums (16 tokens x M rows x K/1024 slices of FP32 for K >= 2048)
 * live in a fixed 8 MiB device array per GPU instead of the workspace, and
 * the call never allocates.  Shapes whose partial sums exceed 8 MiB (e.g.
 * K = 4096 with M > 32768) fail with MTH_EINVAL.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (several streams,
 * threads or concurrently replayed graphs) race; stream-ordered calls do not.
 * Nothing in the array needs clearing: every call writes what it reads. */
int mth_oil4_gemv_noalloc(const uint8_t* packed, const uint16_t* codebooks, int64_t cb_block,
                          const float* x, float* y, int64_t M, int64_t K, int64_t batch,
                          mth_stream_t stream);

/* Prefill GEMM (no reference counterpart beyond oil4_gemm's per-token
 * definition): C[m*N + n] = bf16( sum_k A[m*K + k] * W[n][k] ), A bf16
 * [M][K] row-major, W OIL4 [N][K] with per-block codebooks as in
 * mth_oil4_gemv, FP32 accumulation, C bf16 [M][N] (round to nearest even).
 * Weights are dequantised to FP16 (exact).  Each row of A is scaled by a
 * power of two that brings its maximum into [2^14, 2^15), converted
 * bf16 -> FP16 (exact for every value within 2^-31 of the row's maximum; a
 * row holding Inf or NaN is not scaled) and the row of C scaled back
 * exactly before its bf16 rounding, so activations of any magnitude keep
 * their bits.  K % 32 == 0, cb_block % 32 == 0, 16-byte aligned inputs
 * (MTH_EUNSUPPORTED otherwise).  Uses the stream's workspace (4 bytes per row
 * of A, plus an FP16 copy of A for the tile shapes above). */
int mth_oil4_gemm_prefill(const uint16_t* a_bf16, const uint8_t* packed, const uint16_t* codebooks,
                          int64_t cb_block, uint16_t* c_bf16, int64_t M, int64_t N, int64_t K,
                          mth_stream_t stream);

/* ---------------------------------------------------------- int8 / I2_S -- */

/* quantize_per_token (include/oil/int8_quant.h:17-20, src/int8_quant.cpp:8-31):
 * per row r: max_abs = max(max|src|, 1e-10), scale = 127/max_abs,
 * dst = (int8)round_half_away(src*scale), inv_scale = max_abs/127.
 * scale / inv_scale may be NULL. */
int mth_quantize_per_token(const float* src, int8_t* dst, float* scale, float* inv_scale,
                           int64_t rows, int64_t cols, mth_stream_t stream);

/* dequantize_per_tensor (include/oil/int8_quant.h:22-24, src/int8_quant.cpp:33-37):
 * dst[i] = (float)src[i] * inv_scale. */
int mth_dequantize_per_tensor(const int8_t* src, float* dst, int64_t n, float inv_scale,
                              mth_stream_t stream);

/* oil::kernel::i2s_gemv (include/oil/kernel.h:15-17, src/kernel_i2s.cpp:32-40)
 * applied to M rows and `batch` int8 tokens:
 *   y[t*M + m] = ((float)sum_k tern(packed[m*K/4 ..], k) * act[t*K + k] * w_scale) * act_scale[t]
 * with the LUT initialised (code 00 -> -1, 01 -> 0, 10/11 -> +1).
 * act_scale: device array of `batch` floats (the reference's act_scale).
 * Requires K % 4 == 0.  Bit-exact with the reference. */
int mth_i2s_gemv(const uint8_t* packed, float w_scale, const int8_t* act, const float* act_scale,
                 float* y, int64_t M, int64_t K, int64_t batch, mth_stream_t stream);

/* Fused decode op: quantize_per_token(x_t) then mth_i2s_gemv with
 * act_scale = inv_scale, in one launch.  Requires K % 4 == 0.  Bit-exact. */
int mth_i2s_gemv_f32(const uint8_t* packed, float w_scale, const float* x, float* y,
                     int64_t M, int64_t K, int64_t batch, mth_stream_t stream);

/* oil::kernel::i2s_gemm (include/oil/kernel.h:13-14, src/kernel_i2s.cpp:42-65):
 * out[m*N + n] = sum_k tern(w + m*(K/4), k) * act[n*K + k]  (FP32, no scales). */
int mth_i2s_gemm(const uint8_t* w, const float* act, float* out, int64_t M, int64_t N, int64_t K,
                 mth_stream_t stream);

/* oil::kernel::i2s_gemm_vnni (include/oil/kernel.h:63-65, body at
 * src/kernel_i2s.cpp:201-235): int8 activations, exact integer dot as FP32.
 * M >= 64, N >= 64, K % 256 == 0 with 16-byte aligned w / act run on int8
 * MFMA (bit-exact, no workspace); other shapes run one wave per output. */
int mth_i2s_gemm_vnni(const uint8_t* w, const int8_t* act, float* out, int64_t M, int64_t N, int64_t K,
                      mth_stream_t stream);

/* oil::kernel::tl1_gemm (include/oil/kernel.h:20-21, src/kernel_tl.cpp:33-74),
 * including its pair-LUT indexing by the first weight's code. */
int mth_tl1_gemm(const uint8_t* w, const float* act, float* out, int64_t M, int64_t N, int64_t K,
                 mth_stream_t stream);

/* oil::kernel::tl2_gemm (include/oil/kernel.h:26-27, src/kernel_tl.cpp:109-168).
 * Requires K % 3 == 0 (the reference reads past the activation row otherwise).
 * Rows of whole 16-byte segments (ceil(K/4) % 16 == 0) and a 16-byte aligned
 * w stream through a v_dot4 kernel after one quantisation per activation row
 * (workspace); other shapes run one wave per output.  Bit-exact either way. */
int mth_tl2_gemm(const uint8_t* w, const float* act, float* out, int64_t M, int64_t N, int64_t K,
                 mth_stream_t stream);

/* tl1_precompute_lut / tl2_precompute_lut (include/oil/kernel.h:22-23,28-29;
 * src/kernel_tl.cpp:13-31, 88-107): group = 2 writes K/2 tables of 9 entries,
 * group = 3 writes K/3 tables of 27 entries (requires K % 3 == 0); entry
 * (w0, w1[, w2]) in {-1,0,1}^group, row-major, = clamp_int8(sum a_i*w_i). */
int mth_tl_precompute_lut(const int8_t* act, int8_t* lut, int64_t K, int group, mth_stream_t stream);

/* ---- FP32 decode-step operators (config-5 decoder) ----------------------- */

/* oil::math::rms_norm (include/oil/math.h:24, src/math.cpp:182-205) over rows
 * of dim: double sum of squares, y = (float)(x / sqrt(ss/dim + eps)) * gamma.
 * y may equal x. */
int mth_rms_norm(const float* x, const float* gamma, float* y, int64_t rows, int64_t dim, float eps,
                 mth_stream_t stream);

/* TransformerBlock's residual add then the next RMSNorm (src/transformer.cpp:
 * 402-405, math::add + math::rms_norm in one pass): x <- t + x, y = rms_norm(x). */
int mth_add_rms_norm(float* x, const float* t, const float* gamma, float* y, int64_t rows, int64_t dim, float eps,
                     mth_stream_t stream);

/* oil::math::silu (src/math.cpp:119-128): y = x / (1 + exp(-x)). */
int mth_silu(const float* x, float* y, int64_t n, mth_stream_t stream);

/* FFN::forward's activation (src/transformer.cpp:377-386): silu(g) then
 * math::mul with u, over rows of n (row r of g at g + r*gstride, of u at
 * u + r*ustride); y is [rows][n]. */
int mth_silu_mul(const float* g, const float* u, float* y, int64_t rows, int64_t n, int64_t gstride,
                 int64_t ustride, mth_stream_t stream);

/* The same activation quantised per token for the ternary down projection
 * (quantize_per_token, src/int8_quant.cpp:24-31): q [rows][n] int8 and
 * inv_scale [rows] = max|a|/127, as mth_quantize_per_token of the
 * mth_silu_mul output.  n <= 12288. */
int mth_silu_mul_quant(const float* g, const float* u, int8_t* q, float* inv_scale, int64_t rows, int64_t n,
                       int64_t gstride, int64_t ustride, mth_stream_t stream);

/* The FFN of one token in two launches (the decoder's batch-1 path; no
 * single counterpart in the reference, which runs FFN::forward,
 * src/transformer.cpp:373-406, as separate GEMVs and elementwise ops):
 *
 * mth_oil4_gemv_swiglu: the gate and up projections of one OIL4 weight of
 * 2F rows (gate rows first, then up; per-128 codebooks as mth_oil4_gemv with
 * cb_block 128) and the SwiGLU in the same launch: act[F] = silu(g) * u,
 * bit-identical to mth_oil4_gemv over the 2F rows followed by mth_silu_mul,
 * and amax[F / 8] = max |act| over rows 8t..8t+7.  F % 8 == 0, K % 512 ==
 * 0, 512 <= K <= 4096, 16-byte aligned packed / codebooks / x.
 *
 * mth_i2s_gemv_act: y = the I2_S GEMV of quantize_per_token(act) (the
 * quantisation done inside the launch), bit-identical to
 * mth_quantize_per_token followed by mth_i2s_gemv; amax as written by
 * mth_oil4_gemv_swiglu (the maxima of |act| over groups of 8).  K % 64 ==
 * 0, K <= 12288, 16-byte aligned packed and act. */
int mth_oil4_gemv_swiglu(const uint8_t* packed, const uint16_t* codebooks, const float* x, float* act,
                         float* amax, int64_t F, int64_t K, mth_stream_t stream);
int mth_i2s_gemv_act(const uint8_t* packed, float w_scale, const float* act, const float* amax, float* y,
                     int64_t M, int64_t K, mth_stream_t stream);

/* The same pair for batches of 2..16 tokens (the decoder's batch path; the
 * reference runs FFN::forward per token as above):
 *
 * mth_oil4_gemv_swiglu_batch: x [batch][K]; gu [batch][2F]: act of token t
 * in gu[t*2F + i], i < F, = silu(g) * u, bit-identical to mth_oil4_gemv over
 * the 2F rows (same batch) followed by mth_silu_mul; gu[t*2F + F ..] is
 * overwritten.  amax [batch][mth_swiglu_batch_parts(F)] = max |act| over
 * columns 256j .. 256j + 255.  Per-128 codebooks (cb_block 128) or one
 * shared codebook (cb_block 0); K % 512 == 0, 512 <= K <= 8192, F % 4 ==
 * 0, 16-byte aligned packed / codebooks / x.
 *
 * mth_i2s_gemv_act_batch: y [batch][M] = the I2_S GEMV of
 * quantize_per_token(act[t*lda .. t*lda + K)) (src/int8_quant.cpp:24-31,
 * quantised inside the launch), bit-identical to mth_quantize_per_token
 * followed by mth_i2s_gemv; amax [batch][parts] the block maxima of |act|
 * over 256 columns as mth_oil4_gemv_swiglu_batch writes them (parts =
 * mth_swiglu_batch_parts(K)); inv_scale [batch] receives max|act| / 127.
 * K % 256 == 0, K <= 16384, lda % 4 == 0, 16-byte aligned packed and act.
 * Both use the stream's workspace (mth_workspace_reserve). */
int64_t mth_swiglu_batch_parts(int64_t F);
int mth_oil4_gemv_swiglu_batch(const uint8_t* packed, const uint16_t* codebooks, int64_t cb_block, const float* x,
                               float* gu, float* amax, int64_t F, int64_t K, int64_t batch, mth_stream_t stream);
int mth_i2s_gemv_act_batch(const uint8_t* packed, float w_scale, const float* act, int64_t lda, const float* amax,
                           float* inv_scale, float* y, int64_t M, int64_t K, int64_t batch, mth_stream_t stream);

/* oil::math::add / mul (src/math.cpp:251-258, :269-276). */
int mth_add(const float* a, const float* b, float* c, int64_t n, mth_stream_t stream);
int mth_mul(const float* a, const float* b, float* c, int64_t n, mth_stream_t stream);

/* oil::math::softmax over the last axis of [rows][dim] (src/math.cpp:207-249). */
int mth_softmax(const float* x, float* y, int64_t rows, int64_t dim, mth_stream_t stream);

/* ---- the rest of the ComputeBackend vtable's dense operators ------------
 * (include/oil/backend.h:55-71; the reference's CPU backend calls math::*,
 * src/backend.cpp:40-58).  Used by the HIP ComputeBackend of
 * libmythos_host.so; x and y may be the same array in the elementwise ones. */

/* oil::math::softmax along any axis (src/math.cpp:207-249): x, y viewed as
 * [outer][dim][inner], softmax over dim for every (outer, inner). */
int mth_softmax_axis(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner, mth_stream_t stream);

/* y = alpha * x + beta * y, each product and the sum rounded to FP32 (no
 * fused multiply-add), y always read: the epilogue of math::gemm / gemv
 * (src/math.cpp:70, :94), so NaN or Inf in y reaches the result as there. */
int mth_axpby(float alpha, const float* x, float beta, float* y, int64_t n, mth_stream_t stream);

/* oil::math::gemv (src/math.cpp:52-72): y[i] = alpha * sum_j A[i][j] x[j] +
 * beta * y[i], A [M][N] row-major. */
int mth_gemv_f32(float alpha, const float* A, const float* x, float beta, float* y, int64_t M, int64_t N,
                 mth_stream_t stream);

/* oil::math::relu, gelu (erf form), scale (src/math.cpp:99-117, :278-284). */
int mth_relu(const float* x, float* y, int64_t n, mth_stream_t stream);
int mth_gelu(const float* x, float* y, int64_t n, mth_stream_t stream);
int mth_scale(float s, const float* x, float* y, int64_t n, mth_stream_t stream);

/* oil::math::layer_norm over rows of dim (src/math.cpp:148-180): double mean
 * and variance, y = (float)((x - mean) / sqrt(var + eps)) * gamma + beta. */
int mth_layer_norm(const float* x, const float* gamma, const float* beta, float* y, int64_t rows, int64_t dim,
                   float eps, mth_stream_t stream);

/* RotaryEmbedding tables (src/transformer.cpp:102-117), computed on the host
 * in float: cos/sin [max_seq][head_dim/2] (host buffers). */
int mth_rope_tables(int64_t head_dim, int64_t max_seq, float theta, float* cos_t, float* sin_t);

/* RotaryEmbedding::apply (src/transformer.cpp:119-139) for one token per
 * sequence at position pos, plus KVCache::append (src/kv_cache.cpp:78-137):
 * q [batch][heads][head_dim] rotated in place; k rotated and v copied to
 * kcache/vcache [batch][kv_heads][max_seq][head_dim] at row pos.  cos_t/sin_t
 * are device copies of mth_rope_tables. */
int mth_rope_kv(float* q, const float* k, const float* v, const float* cos_t, const float* sin_t, float* kcache,
                float* vcache, int64_t pos, int64_t batch, int64_t heads, int64_t kv_heads, int64_t head_dim,
                int64_t max_seq, mth_stream_t stream);

/* Attention::forward's inference branch for one query token per sequence
 * (src/transformer.cpp:188-348 with S = 1, scalar softmax): head h attends to
 * cached positions 0..ctx-1 of kv head h % kv_heads, scale 1/sqrt(head_dim);
 * out [batch][heads][head_dim].  head_dim 64, 128 or 256; ctx <= max_seq <= 16384. */
int mth_attention_decode(const float* q, const float* kcache, const float* vcache, float* out, int64_t batch,
                         int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t ctx, int64_t max_seq,
                         mth_stream_t stream);

/* Sampler::greedy (src/sampler.cpp:12-22) per row of logits [rows][n]: the
 * first index of the maximum (NaN never wins). */
int mth_argmax(const float* logits, int32_t* ids, int64_t rows, int64_t n, mth_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MYTHOS_OIL_H */
