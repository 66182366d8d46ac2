// launch.h — internal launcher interface between the C ABI (capi.hip) and the
// kernel translation units.  Launchers assume validated arguments: the C ABI
// checks sizes, pointers and alignment before calling them, and each launcher
// only picks a kernel variant and a grid.  They return the hipError_t of the
// launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace mth {

// ---- errors of the C ABI (capi.hip): set the calling thread's message ----
int api_fail(int code, const char* fmt, ...);
int api_ok();

// ---- OIL8 (gemv.hip) ----------------------------------------------------
// y[t*M + m] = sum_k cb[idx[m*K + k]] * x[t*K + k]          (t < batch)
hipError_t launch_oil8_gemv(const uint8_t* idx, const float* cb, const float* x, float* y,
                            int64_t M, int64_t K, int64_t batch, hipStream_t s);
// Up to three OIL8 matrices with the same K and input, each with its own
// codebook and output (the Q, K and V projections), in one launch:
// seg[i].y[t*rows + m] = sum_k seg[i].cb[seg[i].idx[m*K + k]] * x[t*K + k].
// (Oil8Seg: common.h)
// Segments fused into one launch: K % 16 == 0, K <= 4096, 16-byte aligned
// weights and x (each workgroup stays inside one segment).
bool oil8_segs_fusable(const Oil8Seg* seg, int nseg, int64_t K);
hipError_t launch_oil8_gemv_segs(const Oil8Seg* seg, int nseg, const float* x, int64_t K, int64_t batch,
                                 hipStream_t s);
// Batch 1 with the residual epilogue (ResidOut, common.h) in place of y
// (seg.y unused; oil8_segs_fusable(&seg, 1, K)); *nparts: partials per token.
hipError_t launch_oil8_gemv_resid(const Oil8Seg& seg, const float* x, int64_t K, const ResidOut& ro, int* nparts,
                                  hipStream_t s);
// Reference per-(m,n) indexing (src/kernel_oil8.cpp:20-24):
// out[r] = sum_k cb[idx[r*K + k]] * act[(r % N)*K + k],  r < M*N
hipError_t launch_oil8_gemm_mn(const uint8_t* idx, const float* cb, const float* act, float* out,
                               int64_t M, int64_t N, int64_t K, hipStream_t s);

// ---- OIL4 (gemv.hip) ----------------------------------------------------
// cb_block > 0: codebooks[(m*(K/cb_block) + k/cb_block)*16 + i] (fp16 bits);
// cb_block == 0: one shared 16-entry codebook.
// Batch 1, per-128 codebooks: the fused gate/up projection (rows [0, F) the
// gate, [F, 2F) the up projection of one weight) with the SwiGLU in its
// epilogue: act[F] = silu(g * ni) * (u * ni) (ni from ns; ns.ssp null: 1)
// and amax[F / 8] = max |act| over rows 8t..8t+7.  K % 512 == 0, 512 <= K <=
// 4096 (the shapes launch_oil4_gemv runs on oil4_gemv_v2).
bool oil4_swiglu_supported(const uint8_t* nib, const uint16_t* cbs, const float* x, int64_t F, int64_t K);
hipError_t launch_oil4_swiglu(const uint8_t* nib, const uint16_t* cbs, const float* x, const NormScale& ns,
                              float* act, float* amax, int64_t F, int64_t K, hipStream_t s);
hipError_t launch_oil4_gemv(const uint8_t* nib, const uint16_t* cbs, int64_t cb_block,
                            const float* x, float* y, int64_t M, int64_t K, int64_t batch,
                            hipStream_t s);
// Batches of 2 and more (gemv_batched.hip), groups of 16 tokens per launch.
// partial: oil4_bt_partial_bytes(M, K) bytes of device scratch (null when
// that is 0); calls that share it must be stream-ordered.
bool oil4_bt_supported(int64_t M, int64_t K, int64_t cb_block, int64_t batch);
// Batches of 2..16: the gate/up projection of one OIL4 weight of 2F rows
// (gate first) and the SwiGLU after its K-slice reduction: gu[t][i] (i < F,
// row stride 2F) = silu(g * ni) * (u * ni) (ni from ns; ns.ssp null: 1) and
// amax[t][parts] the maxima of |act| over blocks of 256 columns
// (oil4_bt_swiglu_parts(F) per token).  gu: 2F floats per token.
bool oil4_bt_swiglu_supported(int64_t F, int64_t K, int64_t cb_block, int64_t batch);
int oil4_bt_swiglu_parts(int64_t F);
hipError_t launch_oil4_gemv_bt_swiglu(const uint8_t* nib, const uint16_t* cbs, int64_t cb_block, const float* x,
                                      const NormScale& ns, float* gu, float* amax, int64_t F, int64_t K,
                                      int64_t batch, float* partial, hipStream_t s);
size_t oil4_bt_partial_bytes(int64_t M, int64_t K);
hipError_t launch_oil4_gemv_bt(const uint8_t* nib, const uint16_t* cbs, int64_t cb_block, const float* x, float* y,
                               int64_t M, int64_t K, int64_t batch, float* partial, hipStream_t s);
// OIL8 for batches of 2 and more (gemv_batched.hip, FP16 MFMA with
// three products per block); same workspace contract as the OIL4 batched
// kernel.  The segmented form takes up to kOil8MaxSegs matrices; its
// workspace is oil8_bt_partial_bytes(total rows, K).
bool oil8_bt_supported(int64_t M, int64_t K, int64_t batch);
size_t oil8_bt_partial_bytes(int64_t M, int64_t K);
hipError_t launch_oil8_gemv_bt(const uint8_t* idx, const float* cb, const float* x, float* y, int64_t M, int64_t K,
                               int64_t batch, float* partial, hipStream_t s);
bool oil8_bt_segs_fusable(const Oil8Seg* seg, int nseg, int64_t K, int64_t batch);
// Batches of at most 16 without the slice reduction: the outputs as Slices
// (common.h), one per segment, valid until the workspace is reused.
int oil8_bt_slices(int64_t K);
hipError_t launch_oil8_gemv_bt_segs_slices(const Oil8Seg* seg, int nseg, const float* x, int64_t K, int64_t batch,
                                           float* partial, Slices* out, hipStream_t s);
hipError_t launch_oil8_gemv_bt_segs(const Oil8Seg* seg, int nseg, const float* x, int64_t K, int64_t batch,
                                    float* partial, hipStream_t s);
// Reference per-(m,n) indexing with one codebook (src/kernel_oil4.cpp:41-52).
hipError_t launch_oil4_gemm_mn(const uint8_t* nib, const uint16_t* cb, const float* act, float* out,
                               int64_t M, int64_t N, int64_t K, hipStream_t s);

// ---- int8 / ternary (ternary.hip) ----------------------------------------
hipError_t launch_quantize_per_token(const float* src, int8_t* dst, float* scale, float* inv_scale,
                                     int64_t rows, int64_t cols, hipStream_t s);
hipError_t launch_dequantize(const int8_t* src, float* dst, int64_t n, float inv_scale, hipStream_t s);
hipError_t launch_tl_precompute_lut(const int8_t* act, int8_t* lut, int64_t K, int group, hipStream_t s);
// y[t*M + m] = ((float)dot(t(w_m), q_t) * w_scale) * inv_t
//   fused:   q_t, inv_t from quantize_per_token(x_t) inside the kernel
//   unfused: q_t = act[t*K..], inv_t = act_scale[t]
hipError_t launch_i2s_gemv(const uint8_t* packed, float w_scale, const float* x,
                           const int8_t* act, const float* act_scale, float* y,
                           int64_t M, int64_t K, int64_t batch, hipStream_t s);
// Unfused (int8 activations) batches of 2..16 per launch group on int8 MFMA;
// workspace contract as the batched OIL4/OIL8 kernels.
bool i2s_bt_supported(int64_t M, int64_t K, int64_t batch);
size_t i2s_bt_partial_bytes(int64_t M, int64_t K);
hipError_t launch_i2s_gemv_bt(const uint8_t* packed, float w_scale, const int8_t* act, const float* act_scale, float* y,
                              int64_t M, int64_t K, int64_t batch, float* partial, hipStream_t s);
// Batches of at most 16 without the slice reduction (Slices with the I2_S
// epilogue, common.h).
// Batches of 2..16 with FP32 activations quantised inside the launch (the
// decode step): act[t * lda + k] and amax[t][nmx] as
// launch_oil4_gemv_bt_swiglu writes them; inv[t] = max|act| / 127 is
// written (the output's act scale).  out: the output as Slices (split-K
// partials or y itself).
hipError_t launch_i2s_gemv_bt_f32act(const uint8_t* packed, float w_scale, const float* act, int64_t lda,
                                     const float* amax, int nmx, float* inv, float* y, int64_t M, int64_t K,
                                     int64_t batch, float* partial, Slices* out, hipStream_t s);
// launch_i2s_gemv_bt_f32act with the slices reduced into y [batch][M].
hipError_t launch_i2s_gemv_bt_f32act_y(const uint8_t* packed, float w_scale, const float* act, int64_t lda,
                                       const float* amax, int nmx, float* inv, float* y, int64_t M, int64_t K,
                                       int64_t batch, float* partial, hipStream_t s);
hipError_t launch_i2s_gemv_bt_slices(const uint8_t* packed, float w_scale, const int8_t* act, const float* act_scale,
                                    float* y, int64_t M, int64_t K, int64_t batch, float* partial, Slices* out,
                                    hipStream_t s);
// Batch 1, int8 activations, with the residual epilogue (ResidOut,
// common.h) in place of y; *nparts: partials per token.
bool i2s_resid_supported(const uint8_t* packed, const int8_t* act, int64_t M, int64_t K);
hipError_t launch_i2s_gemv_resid(const uint8_t* packed, float w_scale, const int8_t* act, const float* act_scale,
                                 int64_t M, int64_t K, const ResidOut& ro, int* nparts, hipStream_t s);
// Batch 1: the SwiGLU and the per-token int8 quantisation of g, u (with the
// RMSNorm's 1 / rms from ns) fused into the I2_S down projection; ro
// (ResidOut) or y; ro.ssp must differ from ns.ssp.  *nparts: partials.
bool i2s_swiglu_supported(const uint8_t* packed, int64_t M, int64_t K);
hipError_t launch_i2s_swiglu(const float* g, const float* u, const NormScale& ns, const uint8_t* packed, float w_scale,
                             float* y, int64_t M, int64_t K, const ResidOut& ro, int* nparts, hipStream_t s);
// Batch 1: as launch_i2s_swiglu with the SwiGLU already applied: act[K] =
// silu(g * ni) * (u * ni) and amax[K / 8] the maxima of |act| over groups of
// 8 (launch_oil4_swiglu's outputs); quantisation and product as there.
hipError_t launch_i2s_act(const float* act, const float* amax, const uint8_t* packed, float w_scale, float* y,
                          int64_t M, int64_t K, const ResidOut& ro, int* nparts, hipStream_t s);
hipError_t launch_i2s_gemm(const uint8_t* w, const float* a, float* o,
                           int64_t M, int64_t N, int64_t K, hipStream_t s);
// Shapes the int8-MFMA kernel covers (M, N >= 64, K % 256 == 0, 32-bit
// offsets); launch_i2s_gemm_vnni takes it for them when w and a are 16-byte
// aligned, else one wave per output.
bool i2s_gemm_mfma_ok(int64_t M, int64_t N, int64_t K);
hipError_t launch_i2s_gemm_vnni(const uint8_t* w, const int8_t* a, float* o,
                                int64_t M, int64_t N, int64_t K, hipStream_t s);
// The prompt prefill's down projection on int8 MFMA: y [N][M] = the I2_S
// GEMV of every token row n of the int8 activations a [N][K] with act scale
// inv[n] (bit-identical to launch_i2s_gemv per row); i2s_gemm_mfma_ok(M, N, K)
// and 16-byte aligned w, a (else hipErrorInvalidValue).
hipError_t launch_i2s_gemm_rows(const uint8_t* w, float w_scale, const int8_t* a, const float* inv, float* y, int64_t M,
                                int64_t N, int64_t K, hipStream_t s);
hipError_t launch_tl1_gemm(const uint8_t* w, const float* a, float* o,
                           int64_t M, int64_t N, int64_t K, hipStream_t s);
hipError_t launch_tl2_gemm(const uint8_t* w, const float* a, float* o,
                           int64_t M, int64_t N, int64_t K, hipStream_t s);
// Whole 16-byte segments per weight row (ceil(K/4) % 16 == 0, aligned w):
// the activations quantised once per row into ws (tl2_workspace_bytes, 0 when
// the shape takes launch_tl2_gemm), then a streaming v_dot4 kernel.
size_t tl2_workspace_bytes(const uint8_t* w, int64_t M, int64_t N, int64_t K);
hipError_t launch_tl2_gemm_ws(const uint8_t* w, const float* a, float* o, int64_t M, int64_t N, int64_t K, void* ws,
                              hipStream_t s);

// ---- OIL4 prefill GEMM (gemm_oil4.hip) -----------------------------------
// Each row of A is scaled by a power of two into FP16's range and the output
// row scaled back (per-row shifts: oil4_prefill_shift_bytes(M) of workspace,
// rsh, filled by the launch).
size_t oil4_prefill_shift_bytes(int64_t M);
hipError_t launch_oil4_gemm_prefill(const uint16_t* a_bf16, const uint8_t* nib, const uint16_t* cbs,
                                    int64_t cb_block, uint16_t* c_bf16,
                                    int64_t M, int64_t N, int64_t K, int* rsh, hipStream_t s);
bool oil4_gemm_prefill_supported(int64_t M, int64_t N, int64_t K, int64_t cb_block);
// The FP16-A kernels (oil4_prefill_a16 + oil4_prefill_ws) for K % 256 == 0, cb_block % 64 == 0
// and N a multiple of 64, 96, 112 or 128: needs a workspace of
// oil4_prefill_shift_bytes(M) + oil4_prefill_workspace_bytes (the row shifts,
// then A converted to FP16; 0 = shape not covered).
size_t oil4_prefill_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t cb_block);
hipError_t launch_oil4_gemm_prefill_a16(const uint16_t* a_bf16, const uint8_t* nib, const uint16_t* cbs,
                                       int64_t cb_block, uint16_t* c_bf16, int64_t M, int64_t N, int64_t K,
                                       void* ws, hipStream_t s);

// The prompt prefill's OIL4 projection with FP32 rows (FP32 accurate, the
// decode GEMVs' arithmetic on MFMA): c [Mr][N] = a [Mr][K] W^T, each row of a
// split into FP16 hi + lo after a power-of-two scale (two products per
// weight, sums FP32).  ws: oil4_gemm_x32_workspace_bytes(Mr, K).
bool oil4_gemm_x32_supported(int64_t Mr, int64_t N, int64_t K, int64_t cb_block);
size_t oil4_gemm_x32_workspace_bytes(int64_t Mr, int64_t K);
hipError_t launch_oil4_gemm_x32(const float* a, const uint8_t* nib, const uint16_t* cbs, int64_t cb_block, float* c,
                                int64_t Mr, int64_t N, int64_t K, void* ws, hipStream_t s);
// The FP32 rows' FP16 hi / lo fragments both x32 GEMMs read: ws holds the
// row shifts (oil4_prefill_shift_bytes(Mr)), then 256 virtual rows per 128
// real rows of K FP16 values, for `cover` real rows (a multiple of 128, >= Mr;
// 0: Mr rounded up to 128; rows past Mr are zeros).  A row holding Inf or NaN
// gets the shift kRowNonFinite.
constexpr int kRowNonFinite = 1 << 20;
hipError_t launch_prefill_a16x(const float* a, int64_t Mr, int64_t K, void* ws, hipStream_t s, int64_t cover = 0);

// The prompt prefill's OIL8 projections (gemm_oil8.hip): y_s [Mr][rows_s] =
// a [Mr][K] W_s^T for up to three weights in one launch (Q, K, V), FP32
// accurate (FP16 hi / lo parts of rows and codebook entries, three products
// per weight, FP32 sums); segments of a multiple of 64 rows, K % 256 == 0,
// 16-byte aligned indices and outputs.  ws: oil8_gemm_x32_workspace_bytes.
bool oil8_gemm_x32_supported(const Oil8Seg* seg, int nseg, int64_t Mr, int64_t K);
size_t oil8_gemm_x32_workspace_bytes(int64_t Mr, int64_t K);
hipError_t launch_oil8_gemm_x32(const float* a, const Oil8Seg* seg, int nseg, int64_t Mr, int64_t K, void* ws,
                                hipStream_t s);

// ---- FP32 decode-step operators (dense.hip) ---------------------------------
// x <- t + x (when t), then y = rms_norm(x) * gamma per row of dim.
hipError_t launch_rms_norm(float* x, const float* t, const float* gamma, float* y, int64_t rows, int64_t dim,
                           float eps, hipStream_t s);
// The residual add of the split RMSNorm for a batch (resid_split_k): x <-
// t + x, xg = x * gamma, partial sums of x^2 in ssp[row][*nparts]
// (resid_split_parts(dim) per row); the consumers apply 1 / rms (NormScale).
bool resid_split_supported(const float* x, const Slices& t, const float* gamma, const float* xg, int64_t rows,
                           int64_t dim);
int resid_split_parts(int64_t dim);
hipError_t launch_resid_split(float* x, const Slices& t, const float* gamma, float* xg, double* ssp, int64_t rows,
                              int64_t dim, int* nparts, hipStream_t s);
// launch_rms_norm with t read as Slices (t.n == 0: no residual add).
hipError_t launch_rms_norm_slices(float* x, const Slices& t, const float* gamma, float* y, int64_t rows, int64_t dim,
                                  float eps, hipStream_t s);
// y[r][i] = silu(g[r*gstride + i]) * u[r*ustride + i], i < n
hipError_t launch_silu_mul(const float* g, const float* u, float* y, int64_t rows, int64_t n, int64_t gstride,
                           int64_t ustride, hipStream_t s);
hipError_t launch_silu(const float* x, float* y, int64_t n, hipStream_t s);
hipError_t launch_add(const float* a, const float* b, float* c, int64_t n, hipStream_t s);
hipError_t launch_mul(const float* a, const float* b, float* c, int64_t n, hipStream_t s);
hipError_t launch_softmax(const float* x, float* y, int64_t rows, int64_t dim, hipStream_t s);
// The ComputeBackend vtable's remaining dense operators (dense.hip).
hipError_t launch_softmax_axis(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner, hipStream_t s);
hipError_t launch_axpby(float alpha, const float* x, float beta, float* y, int64_t n, hipStream_t s);
hipError_t launch_gemv_f32(float alpha, const float* A, const float* x, float beta, float* y, int64_t M, int64_t N,
                           hipStream_t s);
hipError_t launch_relu(const float* x, float* y, int64_t n, hipStream_t s);
hipError_t launch_gelu(const float* x, float* y, int64_t n, hipStream_t s);
hipError_t launch_scale(float a, const float* x, float* y, int64_t n, hipStream_t s);
hipError_t launch_layer_norm(const float* x, const float* gamma, const float* beta, float* y, int64_t rows,
                             int64_t dim, float eps, hipStream_t s);
// Position pos = (step ? *step : 0) + pos0; caches [batch][kv_heads][max_seq][head_dim].
hipError_t launch_rope_kv(float* q, const float* k, const float* v, const float* cos_t, const float* sin_t,
                          float* kc, float* vc, const int* step, int pos0, int64_t batch, int heads, int kv_heads,
                          int head_dim, int max_seq, hipStream_t s);
// ctx = (step ? *step : 0) + ctx0 + 1 <= max_seq positions.
bool attention_supported(int head_dim, int max_seq);
hipError_t launch_attention(const float* q, const float* kc, const float* vc, float* out, const int* step, int ctx0,
                            int64_t batch, int heads, int kv_heads, int head_dim, int max_seq, hipStream_t s);
// RoPE of the current token's q/k at pos = *step, KV append, then attention
// over pos + 1 positions (one launch).  Caches FP32, or bf16 bits (kv_bf16).
hipError_t launch_rope_attention(const float* q, const float* k, const float* v, const float* cos_t,
                                 const float* sin_t, void* kc, void* vc, bool kv_bf16, float* out, const int* step,
                                 int64_t batch, int heads, int kv_heads, int head_dim, int max_seq, hipStream_t s);
// q/k/v as Slices (common.h): rows of heads*head_dim / kv_heads*head_dim.
// ns (common.h): q/k/v projected from x * gamma, scaled by the norm here.
hipError_t launch_rope_attention_slices(const Slices& q, const Slices& k, const Slices& v, const NormScale& ns,
                                        const float* cos_t, const float* sin_t, void* kc, void* vc, bool kv_bf16,
                                        float* out, const int* step, int64_t batch, int heads, int kv_heads,
                                        int head_dim, int max_seq, hipStream_t s);
// Prefill rows: row r is position p0 + r % np of sequence r / np.
// Attention of each row over the cache positions 0 .. its own (q rotated).
hipError_t launch_attention_rows(const float* q, const void* kc, const void* vc, bool kv_bf16, float* out,
                                 int64_t rows, int np, int p0, int heads, int kv_heads, int head_dim, int max_seq,
                                 hipStream_t s);
// RoPE of each row's q (in place) and k; k, v appended to the caches.
hipError_t launch_rope_kv_rows(float* q, const float* k, const float* v, const float* cos_t, const float* sin_t,
                               void* kc, void* vc, bool kv_bf16, int64_t rows, int np, int p0, int heads, int kv_heads,
                               int head_dim, int max_seq, hipStream_t s);
// x[r] = emb[hist[r / np][p0 + r % np]]
hipError_t launch_embed_rows(const float* emb, const int* hist, int hist_stride, float* x, int64_t rows, int np, int p0,
                             int dim, int vocab, hipStream_t s);
// silu(g) * u then quantize_per_token: q [rows][n] int8, inv_scale [rows];
// act (nullable) receives the FP32 activations [rows][n].
bool silu_mul_quant_supported(int64_t n);
// g/u as Slices (common.h)
hipError_t launch_silu_mul_quant_slices(const Slices& g, const Slices& u, const NormScale& ns, int8_t* q,
                                        float* inv_scale, float* act, int64_t rows, int64_t n, hipStream_t s);
hipError_t launch_silu_mul_quant(const float* g, const float* u, int8_t* q, float* inv_scale, float* act,
                                 int64_t rows, int64_t n, int64_t gstride, int64_t ustride, hipStream_t s);
// Greedy argmax in two launches; pv/pi: rows * argmax_chunks(n) partials.
// With hist: writes the next input token; with step: advances it last.
int argmax_chunks(int64_t n);
hipError_t launch_argmax(const float* logits, int64_t rows, int64_t n, int* ids, int* hist, int* step,
                         int hist_stride, int prompt_len, float* pv, int* pi, hipStream_t s);
hipError_t launch_embed(const float* emb, const int* hist, const int* step, int hist_stride, float* x, int64_t batch,
                        int dim, int vocab, hipStream_t s, const ResidOut& ro = ResidOut{});

}  // namespace mth
