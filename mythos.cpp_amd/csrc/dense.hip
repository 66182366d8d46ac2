// dense.hip — the FP32 decode-step operators around the quantized GEMVs
// (gfx950): RMSNorm (optionally fused with the residual add before it),
// SwiGLU, softmax, elementwise add/mul, rotary embedding + KV-cache append,
// decode attention over the KV cache, greedy argmax and the embedding gather.
//
// Reference semantics (each kernel cites its source):
//   math::rms_norm   src/math.cpp:182-205   double sum of squares, double inverse
//                                           root, (float)(x * inv) * gamma
//   math::silu/mul   src/math.cpp:119-128, :269-276 (FFN: src/transformer.cpp:377-386)
//   math::softmax    src/math.cpp:207-249   float max, float exp, double sum
//   math::add        src/math.cpp:251-258
//   RotaryEmbedding  src/transformer.cpp:119-139  rotate-half pairs (d, d + D/2)
//   Attention        src/transformer.cpp:188-348  inference branch with S = 1
//                                           (scalar softmax: exp, float sum, * 1/sum)
//   Sampler::greedy  src/sampler.cpp:12-22  first index of the maximum
//   Embedding        src/transformer.cpp:29-46    ids outside [0, vocab) read row 0
//
// All of these are bandwidth- or latency-bound at decode sizes (a few KB to a
// few MB per launch); they use float4 accesses where rows allow and keep
// every reduction inside one workgroup (no global atomics, no fences).
#include <hip/hip_runtime.h>

#include "common.h"
#include "launch.h"

// The reference's operators are plain float expressions; they stay plain and
// uncontracted here so that products and sums round as they do there
// (explicit fmaf calls stay fused).  Division and sqrt are correctly rounded
// (HIP's default).
#pragma clang fp contract(off)

namespace mth {
namespace {

constexpr int kT = 256;  // threads per workgroup (4 waves)

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, MTH_WAVE);
    return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, MTH_WAVE);
    return v;
}

// Sum over the workgroup; every thread gets the total.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if constexpr (sizeof(T) == 8)
        v = wave_sum_d(v);
    else
        v = wave_sum_f(v);
    __syncthreads();  // red may still be read by a previous reduction
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float block_max(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// ---- RMSNorm, optionally after the residual add ---------------------------
// One workgroup per row.  With t: x <- t + x first (math::add of the block's
// residual, src/transformer.cpp:402,405), written back.  dim % 4 == 0.
// x and y may be the same array (in-place normalisation): each thread reads
// its own elements before it writes them.
__global__ __launch_bounds__(kT) void rms_norm_k(float* x, const float* __restrict__ t,
                                                 const float* __restrict__ gamma, float* y, int dim, float eps) {
    __shared__ double red[4];
    float* xr = x + (int64_t)blockIdx.x * dim;
    const float* tr = t ? t + (int64_t)blockIdx.x * dim : nullptr;
    float* yr = y + (int64_t)blockIdx.x * dim;
    double ss = 0.0;
    for (int i = threadIdx.x * 4; i < dim; i += kT * 4) {
        float4 v = ldf4(xr + i);
        if (tr) {
            const float4 a = ldf4(tr + i);
            v = make_float4((a.x + v.x), (a.y + v.y), (a.z + v.z), (a.w + v.w));
            *(float4*)(xr + i) = v;
        }
        ss += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    ss = block_sum(ss, red);
    const double inv = 1.0 / sqrt(ss / (double)dim + (double)eps);
    for (int i = threadIdx.x * 4; i < dim; i += kT * 4) {
        const float4 v = ldf4(xr + i);  // this thread's own elements (written above)
        const float4 g = ldf4(gamma + i);
        float4 o;
        o.x = ((float)((double)v.x * inv) * g.x);
        o.y = ((float)((double)v.y * inv) * g.y);
        o.z = ((float)((double)v.z * inv) * g.z);
        o.w = ((float)((double)v.w * inv) * g.w);
        *(float4*)(yr + i) = o;
    }
}

// Generic-width variant (dim % 4 != 0 or unaligned rows).
__global__ __launch_bounds__(kT) void rms_norm_any_k(float* x, const float* __restrict__ t,
                                                     const float* __restrict__ gamma, float* y, int64_t dim,
                                                     float eps) {
    __shared__ double red[4];
    float* xr = x + (int64_t)blockIdx.x * dim;
    const float* tr = t ? t + (int64_t)blockIdx.x * dim : nullptr;
    float* yr = y + (int64_t)blockIdx.x * dim;
    double ss = 0.0;
    for (int64_t i = threadIdx.x; i < dim; i += kT) {
        float v = xr[i];
        if (tr) {
            v = (tr[i] + v);
            xr[i] = v;
        }
        ss += (double)v * v;
    }
    ss = block_sum(ss, red);
    const double inv = 1.0 / sqrt(ss / (double)dim + (double)eps);
    for (int64_t i = threadIdx.x; i < dim; i += kT) yr[i] = ((float)((double)xr[i] * inv) * gamma[i]);
}

// ---- SwiGLU and elementwise ------------------------------------------------
__device__ __forceinline__ float silu1(float g) { return (g / (1.0f + expf(-g))); }

// y[r][i] = silu(g) * u with g = gu[r][i], u = gu[r][n + i] (the gate and up
// outputs of one fused GEMV, rows of 2n), or g/u from separate arrays.
__global__ __launch_bounds__(kT) void silu_mul_k(const float* __restrict__ g, const float* __restrict__ u,
                                                 float* __restrict__ y, int64_t n, int64_t gstride, int64_t ustride) {
    const int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x;
    const int64_t r = blockIdx.y;
    if (i < n) y[r * n + i] = (silu1(g[r * gstride + i]) * u[r * ustride + i]);
}

__global__ __launch_bounds__(kT) void silu_k(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x;
    if (i < n) y[i] = silu1(x[i]);
}

__global__ __launch_bounds__(kT) void add_k(const float* __restrict__ a, const float* __restrict__ b,
                                            float* __restrict__ c, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x;
    if (i < n) c[i] = (a[i] + b[i]);
}

__global__ __launch_bounds__(kT) void mul_k(const float* __restrict__ a, const float* __restrict__ b,
                                            float* __restrict__ c, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x;
    if (i < n) c[i] = (a[i] * b[i]);
}

// ---- softmax over rows (math::softmax, last axis) --------------------------
__global__ __launch_bounds__(kT) void softmax_k(const float* __restrict__ x, float* __restrict__ y, int64_t dim) {
    __shared__ double redd[4];
    __shared__ float redf[4];
    const float* xr = x + (int64_t)blockIdx.x * dim;
    float* yr = y + (int64_t)blockIdx.x * dim;
    float mx = -INFINITY;
    for (int64_t i = threadIdx.x; i < dim; i += kT) mx = fmaxf(mx, xr[i]);
    mx = block_max(mx, redf);
    double sum = 0.0;
    for (int64_t i = threadIdx.x; i < dim; i += kT) {
        const float e = expf((xr[i] - mx));
        yr[i] = e;
        sum += (double)e;
    }
    sum = block_sum(sum, redd);
    const double inv = 1.0 / sum;
    for (int64_t i = threadIdx.x; i < dim; i += kT) yr[i] = (float)((double)yr[i] * inv);
}

// ---- rotary embedding + KV-cache append ------------------------------------
// One workgroup per token b.  q [B][heads*D] rotated in place; k rotated and,
// with v, written to the caches at position pos = *step (+ pos0):
// cache[(b*kv_heads + h)*max_seq + pos][D].  cos/sin: [max_seq][D/2].
__global__ __launch_bounds__(kT) void rope_kv_k(float* __restrict__ q, const float* __restrict__ k,
                                                const float* __restrict__ v, const float* __restrict__ cos_t,
                                                const float* __restrict__ sin_t, float* __restrict__ kc,
                                                float* __restrict__ vc, const int* __restrict__ step, int pos0,
                                                int heads, int kv_heads, int D, int max_seq) {
    const int b = blockIdx.x;
    const int pos = (step ? *step : 0) + pos0;
    const int h2 = D / 2;
    const float* cr = cos_t + (int64_t)pos * h2;
    const float* sr = sin_t + (int64_t)pos * h2;
    const int nq = heads * h2, nk = kv_heads * h2;
    float* qb = q + (int64_t)b * heads * D;
    for (int i = threadIdx.x; i < nq; i += kT) {
        const int h = i / h2, d = i % h2;
        float* p = qb + h * D;
        const float x1 = p[d], x2 = p[d + h2], c = cr[d], s = sr[d];
        p[d] = ((x1 * c) - (x2 * s));
        p[d + h2] = ((x1 * s) + (x2 * c));
    }
    const float* kb = k + (int64_t)b * kv_heads * D;
    const float* vb = v + (int64_t)b * kv_heads * D;
    for (int i = threadIdx.x; i < nk; i += kT) {
        const int h = i / h2, d = i % h2;
        const float* p = kb + h * D;
        const float x1 = p[d], x2 = p[d + h2], c = cr[d], s = sr[d];
        const int64_t row = (((int64_t)b * kv_heads + h) * max_seq + pos) * D;
        kc[row + d] = ((x1 * c) - (x2 * s));
        kc[row + d + h2] = ((x1 * s) + (x2 * c));
        vc[row + d] = vb[h * D + d];
        vc[row + d + h2] = vb[h * D + d + h2];
    }
}

// ---- decode attention --------------------------------------------------------
// Workgroup (head h, token b): ctx = *step + ctx0 + 1 cached positions of kv
// head h % kv_heads.  D = 64 * HPL; each lane holds HPL elements of q.
// Scores: one position per wave iteration (coalesced K row, wave sum);
// softmax in LDS; P*V: waves split positions, lanes own HPL columns.
template <int HPL>
__global__ __launch_bounds__(kT) void attention_k(const float* __restrict__ q, const float* __restrict__ kc,
                                                  const float* __restrict__ vc, float* __restrict__ out,
                                                  const int* __restrict__ step, int ctx0, int heads, int kv_heads,
                                                  int max_seq, float scale) {
    constexpr int D = 64 * HPL;
    extern __shared__ float sc[];           // [ctx] scores, then probabilities
    __shared__ float redf[4];
    __shared__ float part[4][D];
    const int h = blockIdx.x, b = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ctx = (step ? *step : 0) + ctx0 + 1;
    const int kh = h % kv_heads;
    const float* qh = q + ((int64_t)b * heads + h) * D;
    const float* kb = kc + ((int64_t)b * kv_heads + kh) * max_seq * D;
    const float* vb = vc + ((int64_t)b * kv_heads + kh) * max_seq * D;
    float qv[HPL];
#pragma unroll
    for (int j = 0; j < HPL; ++j) qv[j] = qh[lane + 64 * j];
    for (int t = wave; t < ctx; t += 4) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < HPL; ++j) s = fmaf(qv[j], kb[(int64_t)t * D + lane + 64 * j], s);
        s = wave_sum_f(s);
        if (lane == 0) sc[t] = (s * scale);
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < ctx; t += kT) mx = fmaxf(mx, sc[t]);
    mx = block_max(mx, redf);
    float sum = 0.0f;
    for (int t = threadIdx.x; t < ctx; t += kT) {
        const float e = expf((sc[t] - mx));
        sc[t] = e;
        sum += e;
    }
    sum = block_sum(sum, redf);
    const float inv = (1.0f / sum);
    __syncthreads();
    float acc[HPL];
#pragma unroll
    for (int j = 0; j < HPL; ++j) acc[j] = 0.0f;
    for (int t = wave; t < ctx; t += 4) {
        const float p = (sc[t] * inv);
#pragma unroll
        for (int j = 0; j < HPL; ++j) acc[j] = fmaf(p, vb[(int64_t)t * D + lane + 64 * j], acc[j]);
    }
#pragma unroll
    for (int j = 0; j < HPL; ++j) part[wave][lane + 64 * j] = acc[j];
    __syncthreads();
    float* ob = out + ((int64_t)b * heads + h) * D;
    for (int d = threadIdx.x; d < D; d += kT) ob[d] = (part[0][d] + part[1][d]) + (part[2][d] + part[3][d]);
}

// ---- greedy argmax + token bookkeeping ---------------------------------------
// Row b of logits [B][n]: first index of the maximum (NaN never wins; all-NaN
// or all -inf rows give 0).  Writes ids[b]; with hist, also the next input
// token hist[b][s + 1] once the prompt is consumed (s + 1 >= prompt_len).
__global__ __launch_bounds__(kT) void argmax_k(const float* __restrict__ logits, int64_t n, int* __restrict__ ids,
                                               int* __restrict__ hist, const int* __restrict__ step, int hist_stride,
                                               int prompt_len) {
    __shared__ float bv[kT];
    __shared__ int bi[kT];
    const float* r = logits + (int64_t)blockIdx.x * n;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int64_t i = threadIdx.x; i < n; i += kT) {
        const float x = r[i];
        if (x > v) {
            v = x;
            idx = (int)i;
        }
    }
    bv[threadIdx.x] = v;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (int o = kT / 2; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            const float v2 = bv[threadIdx.x + o];
            const int i2 = bi[threadIdx.x + o];
            if (v2 > bv[threadIdx.x] || (v2 == bv[threadIdx.x] && i2 < bi[threadIdx.x])) {
                bv[threadIdx.x] = v2;
                bi[threadIdx.x] = i2;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int best = bi[0] == 0x7fffffff ? 0 : bi[0];
        if (ids) ids[blockIdx.x] = best;
        if (hist) {
            const int s = *step;
            if (s + 1 >= prompt_len && s + 1 < hist_stride) hist[(int64_t)blockIdx.x * hist_stride + s + 1] = best;
        }
    }
}

// x[b] = emb[id] with id = hist[b][*step] (ids outside [0, vocab) -> 0).
__global__ __launch_bounds__(kT) void embed_k(const float* __restrict__ emb, const int* __restrict__ hist,
                                              const int* __restrict__ step, int hist_stride, float* __restrict__ x,
                                              int dim, int vocab) {
    const int b = blockIdx.x;
    int id = hist[(int64_t)b * hist_stride + *step];
    if (id < 0 || id >= vocab) id = 0;
    const float* src = emb + (int64_t)id * dim;
    float* dst = x + (int64_t)b * dim;
    for (int i = threadIdx.x * 4; i < dim; i += kT * 4) *(float4*)(dst + i) = ldf4(src + i);
}

__global__ void advance_k(int* step) {
    if (threadIdx.x == 0) *step += 1;
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + kT - 1) / kT); }
inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

hipError_t launch_rms_norm(float* x, const float* t, const float* gamma, float* y, int64_t rows, int64_t dim,
                           float eps, hipStream_t s) {
    if (dim % 4 == 0 && dim < (1ll << 31) && al16(x) && al16(y) && al16(gamma) && (!t || al16(t)))
        rms_norm_k<<<(unsigned)rows, kT, 0, s>>>(x, t, gamma, y, (int)dim, eps);
    else
        rms_norm_any_k<<<(unsigned)rows, kT, 0, s>>>(x, t, gamma, y, dim, eps);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* g, const float* u, float* y, int64_t rows, int64_t n, int64_t gstride,
                           int64_t ustride, hipStream_t s) {
    silu_mul_k<<<dim3(blocks_for(n), (unsigned)rows), kT, 0, s>>>(g, u, y, n, gstride, ustride);
    return hipGetLastError();
}

hipError_t launch_silu(const float* x, float* y, int64_t n, hipStream_t s) {
    silu_k<<<blocks_for(n), kT, 0, s>>>(x, y, n);
    return hipGetLastError();
}

hipError_t launch_add(const float* a, const float* b, float* c, int64_t n, hipStream_t s) {
    add_k<<<blocks_for(n), kT, 0, s>>>(a, b, c, n);
    return hipGetLastError();
}

hipError_t launch_mul(const float* a, const float* b, float* c, int64_t n, hipStream_t s) {
    mul_k<<<blocks_for(n), kT, 0, s>>>(a, b, c, n);
    return hipGetLastError();
}

hipError_t launch_softmax(const float* x, float* y, int64_t rows, int64_t dim, hipStream_t s) {
    softmax_k<<<(unsigned)rows, kT, 0, s>>>(x, y, dim);
    return hipGetLastError();
}

hipError_t launch_rope_kv(float* q, const float* k, const float* v, const float* cos_t, const float* sin_t,
                          float* kc, float* vc, const int* step, int pos0, int64_t batch, int heads, int kv_heads,
                          int head_dim, int max_seq, hipStream_t s) {
    rope_kv_k<<<(unsigned)batch, kT, 0, s>>>(q, k, v, cos_t, sin_t, kc, vc, step, pos0, heads, kv_heads, head_dim,
                                             max_seq);
    return hipGetLastError();
}

bool attention_supported(int head_dim, int max_seq) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && max_seq > 0 && max_seq <= 16384;
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc, float* out, const int* step, int ctx0,
                            int64_t batch, int heads, int kv_heads, int head_dim, int max_seq, hipStream_t s) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    const size_t lds = (size_t)max_seq * sizeof(float);
    const dim3 grid((unsigned)heads, (unsigned)batch);
    if (head_dim == 64)
        attention_k<1><<<grid, kT, lds, s>>>(q, kc, vc, out, step, ctx0, heads, kv_heads, max_seq, scale);
    else if (head_dim == 128)
        attention_k<2><<<grid, kT, lds, s>>>(q, kc, vc, out, step, ctx0, heads, kv_heads, max_seq, scale);
    else
        attention_k<4><<<grid, kT, lds, s>>>(q, kc, vc, out, step, ctx0, heads, kv_heads, max_seq, scale);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int64_t rows, int64_t n, int* ids, int* hist, const int* step,
                         int hist_stride, int prompt_len, hipStream_t s) {
    argmax_k<<<(unsigned)rows, kT, 0, s>>>(logits, n, ids, hist, step, hist_stride, prompt_len);
    return hipGetLastError();
}

hipError_t launch_embed(const float* emb, const int* hist, const int* step, int hist_stride, float* x, int64_t batch,
                        int dim, int vocab, hipStream_t s) {
    embed_k<<<(unsigned)batch, kT, 0, s>>>(emb, hist, step, hist_stride, x, dim, vocab);
    return hipGetLastError();
}

hipError_t launch_advance(int* step, hipStream_t s) {
    advance_k<<<1, 64, 0, s>>>(step);
    return hipGetLastError();
}

}  // namespace mth
