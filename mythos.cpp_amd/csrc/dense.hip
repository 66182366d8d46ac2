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
constexpr int kArgChunk = 2048;  // argmax columns per stage-1 workgroup

__device__ __forceinline__ double wave_sum_d(double v) { return wave_sum_dbl(v); }
__device__ __forceinline__ float wave_sum_f(float v) { return group_sum<64>(v); }

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
// The same over NW waves (pairwise over the waves in order: for NW == 4 the
// sums of block_sum and the maximum of block_max).
template <int NW, typename T>
__device__ __forceinline__ T block_sum_w(T v, T* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if constexpr (sizeof(T) == 8)
        v = wave_sum_d(v);
    else
        v = wave_sum_f(v);
    __syncthreads();  // red may still be read by a previous reduction
    if (lane == 0) red[wave] = v;
    __syncthreads();
    T t[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) t[w] = red[w];
#pragma unroll
    for (int st = 1; st < NW; st *= 2)
#pragma unroll
        for (int i = 0; i + st < NW; i += 2 * st) t[i] = t[i] + t[i + st];
    return t[0];
}
template <int NW>
__device__ __forceinline__ float block_max_w(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, red[w]);
    return m;
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
constexpr int kRN = 1024;  // threads of the float4 RMSNorm (one float4 each at dim 4096)
// t: the residual as Slices (common.h; t.n == 0: none), so the split-K
// partial sums of the GEMV that produced it are added here.
__global__ __launch_bounds__(kRN) void rms_norm_k(float* x, Slices t, const float* __restrict__ gamma, float* y,
                                                  int dim, float eps) {
    __shared__ double red[kRN / 64];
    float* xr = x + (int64_t)blockIdx.x * dim;
    float* yr = y + (int64_t)blockIdx.x * dim;
    double ss = 0.0;
    for (int i = threadIdx.x * 4; i < dim; i += kRN * 4) {
        float4 v = ldf4(xr + i);
        if (t.n) {
            const float4 a = slice_value4(t, blockIdx.x, i);
            v = make_float4((a.x + v.x), (a.y + v.y), (a.z + v.z), (a.w + v.w));
            *(float4*)(xr + i) = v;
        }
        ss += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    ss = wave_sum_d(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = 0.0;
#pragma unroll
    for (int w = 0; w < kRN / 64; ++w) ss += red[w];
    const double inv = 1.0 / sqrt(ss / (double)dim + (double)eps);
    for (int i = threadIdx.x * 4; i < dim; i += kRN * 4) {
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

// The residual add of the split RMSNorm for a batch of rows (ResidOut,
// common.h), as a launch of its own since the producers of t leave split-K
// partial sums: x <- t + x (the sum of rms_norm_k), xg = x * gamma, and per
// workgroup the sum of x^2 over its 4 * kRS columns (double, in rms_norm_k's
// per-element order) in ssp[row][blockIdx.x].  The consumers apply the
// 1 / rms (NormScale).  grid (ceil(dim / (4 kRS)), rows); dim % 4 == 0.
constexpr int kRS = 64;
__global__ __launch_bounds__(kRS) void resid_split_k(float* x, Slices t, const float* __restrict__ gamma, float* xg,
                                                     double* ssp, int dim) {
    __shared__ double red[kRS / 64];
    const int r = blockIdx.y, i = (blockIdx.x * kRS + threadIdx.x) * 4;
    double ss = 0.0;
    if (i < dim) {
        float* xr = x + (int64_t)r * dim + i;
        float4 v = ldf4(xr);
        const float4 g = ldf4(gamma + i);
        if (t.n) {
            const float4 a = slice_value4(t, r, i);
            v = make_float4((a.x + v.x), (a.y + v.y), (a.z + v.z), (a.w + v.w));
            *(float4*)xr = v;
        }
        *(float4*)(xg + (int64_t)r * dim + i) = make_float4(v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w);
        ss = (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    ss = wave_sum_dbl(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    if (threadIdx.x == 0) {
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < kRS / 64; ++w) tot += red[w];
        ssp[(int64_t)r * gridDim.x + blockIdx.x] = tot;
    }
}

// Generic-width variant (dim % 4 != 0 or unaligned rows).
__global__ __launch_bounds__(kT) void rms_norm_any_k(float* x, Slices t, const float* __restrict__ gamma, float* y,
                                                     int64_t dim, float eps) {
    __shared__ double red[4];
    float* xr = x + (int64_t)blockIdx.x * dim;
    float* yr = y + (int64_t)blockIdx.x * dim;
    double ss = 0.0;
    for (int64_t i = threadIdx.x; i < dim; i += kT) {
        float v = xr[i];
        if (t.n) {
            v = (slice_value(t, blockIdx.x, i) + v);
            xr[i] = v;
        }
        ss += (double)v * v;
    }
    ss = block_sum(ss, red);
    const double inv = 1.0 / sqrt(ss / (double)dim + (double)eps);
    for (int64_t i = threadIdx.x; i < dim; i += kT) yr[i] = ((float)((double)xr[i] * inv) * gamma[i]);
}

// ---- SwiGLU and elementwise ------------------------------------------------

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

// ---- the remaining dense operators of the ComputeBackend vtable ------------
// (include/oil/backend.h:55-71, dispatched to math:: by the reference's CPU
// backend, src/backend.cpp:40-58)
//   math::gemv            src/math.cpp:52-72    s = sum_j A[i][j] x[j]; y = alpha*s + beta*y
//   gemm's epilogue       src/math.cpp:74-97    C = alpha*(A B) + beta*C, C always read
//   math::relu            src/math.cpp:99-105
//   math::gelu            src/math.cpp:107-117  0.5f * v * (1 + erf(v * 1/sqrt 2))
//   math::layer_norm      src/math.cpp:148-180  double mean, double variance of the
//                                               deviations, (float)(d * inv) * gamma + beta
//   math::softmax, axis   src/math.cpp:207-249  as softmax_k, along a strided axis
//   math::scale           src/math.cpp:278-284
__global__ __launch_bounds__(kT) void axpby_k(float alpha, const float* __restrict__ x, float beta,
                                              float* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x;
    if (i < n) y[i] = alpha * x[i] + beta * y[i];
}

// One wave per row; the row's products summed in FP32 per lane, then across
// the wave.
__global__ __launch_bounds__(kT) void gemv_f32_k(float alpha, const float* __restrict__ A,
                                                 const float* __restrict__ x, float beta, float* __restrict__ y,
                                                 int64_t M, int64_t N) {
    const int64_t row = (int64_t)blockIdx.x * (kT / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const float* a = A + row * N;
    float s = 0.0f;
    for (int64_t j = lane; j < N; j += 64) s += a[j] * x[j];
    s = group_sum<64>(s);
    if (lane == 0) y[row] = alpha * s + beta * y[row];
}

__global__ __launch_bounds__(kT) void relu_k(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x;
    if (i < n) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

__global__ __launch_bounds__(kT) void gelu_k(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x;
    if (i < n) {
        const float v = x[i];
        y[i] = 0.5f * v * (1.0f + erff(v * 0.7071067811865475f));
    }
}

__global__ __launch_bounds__(kT) void scale_k(float s, const float* __restrict__ x, float* __restrict__ y,
                                              int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x;
    if (i < n) y[i] = s * x[i];
}

// One workgroup per row.
__global__ __launch_bounds__(kT) void layer_norm_k(const float* __restrict__ x, const float* __restrict__ gamma,
                                                   const float* __restrict__ beta, float* __restrict__ y,
                                                   int64_t dim, float eps) {
    __shared__ double red[4];
    const float* xr = x + (int64_t)blockIdx.x * dim;
    float* yr = y + (int64_t)blockIdx.x * dim;
    double s = 0.0;
    for (int64_t j = threadIdx.x; j < dim; j += kT) s += xr[j];
    const double mu = block_sum(s, red) / (double)dim;
    double v = 0.0;
    for (int64_t j = threadIdx.x; j < dim; j += kT) {
        const double d = (double)xr[j] - mu;
        v += d * d;
    }
    const double var = block_sum(v, red) / (double)dim;
    const double inv = 1.0 / sqrt(var + (double)eps);
    for (int64_t j = threadIdx.x; j < dim; j += kT) yr[j] = (float)(((double)xr[j] - mu) * inv) * gamma[j] + beta[j];
}

// Softmax along a strided axis: thread = (outer o, inner i), the dim values
// x[o][d][i] at stride inner.
__global__ __launch_bounds__(kT) void softmax_strided_k(const float* __restrict__ x, float* __restrict__ y,
                                                        int64_t outer, int64_t dim, int64_t inner) {
    const int64_t t = (int64_t)blockIdx.x * kT + threadIdx.x;
    if (t >= outer * inner) return;
    const int64_t o = t / inner, i = t - o * inner;
    const float* src = x + o * dim * inner + i;
    float* dst = y + o * dim * inner + i;
    float mx = -INFINITY;
    for (int64_t d = 0; d < dim; ++d) mx = fmaxf(mx, src[d * inner]);
    double sum = 0.0;
    for (int64_t d = 0; d < dim; ++d) {
        const float e = expf(src[d * inner] - mx);
        dst[d * inner] = e;
        sum += (double)e;
    }
    const double inv = 1.0 / sum;
    for (int64_t d = 0; d < dim; ++d) dst[d * inner] = (float)((double)dst[d * inner] * inv);
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

// ---- KV-cache element types -----------------------------------------------------
// FP32, or bf16 (round to nearest even on store, exact widening on load).
__device__ __forceinline__ float kv_store_value(float v, float) { return v; }
__device__ __forceinline__ uint16_t bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);  // NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint16_t kv_store_value(float v, uint16_t) { return bf16_rne(v); }
// the value an element reads back as after a store
__device__ __forceinline__ float kv_rounded(float v, float) { return v; }
__device__ __forceinline__ float kv_rounded(float v, uint16_t) { return __uint_as_float((uint32_t)bf16_rne(v) << 16); }
__device__ __forceinline__ float4 kv_load4(const float* p) { return *(const float4*)p; }
__device__ __forceinline__ float4 kv_widen(const uint2& w) {
    return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                       __uint_as_float(w.y & 0xffff0000u));
}
__device__ __forceinline__ float4 kv_widen(const float4& v) { return v; }
__device__ __forceinline__ float4 kv_load4(const uint16_t* p) { return kv_widen(*(const uint2*)p); }
// four elements as loaded (bf16 stays packed until used)
template <typename KV> struct KvRaw4 { typedef float4 type; };
template <> struct KvRaw4<uint16_t> { typedef uint2 type; };
__device__ __forceinline__ float4 kv_raw4(const float* p) { return *(const float4*)p; }
__device__ __forceinline__ uint2 kv_raw4(const uint16_t* p) { return *(const uint2*)p; }

// ---- decode attention --------------------------------------------------------
// Workgroup (head h, token b) over ctx = *step + ctx0 + 1 positions of kv
// head kh = h % kv_heads, cache rows [b][kh][t][D].
// Latency, not bandwidth, bounds this kernel at decode sizes, so the cache
// rows are loaded as early as their order of use allows (the CU returns
// loads in issue order): first each thread's K rows of the first 192
// positions, then (after the q/k/v staging, so that the K rows of the
// other workgroups on the CU come first) the V rows it accumulates in P*V
// (up to VP of them, positions sl + SL j, kept packed), so the scores wait
// only for K and the V rows arrive during the softmax.  Scores: one position per thread, the
// dot product over d in four interleaved FP32 partial sums (d mod 4) added
// pairwise, q broadcast from LDS.  Softmax in LDS.  P*V: thread = (float4
// column group g, position slice sl), four accumulators; slices are summed
// through LDS in a fixed order.
// ROPE: the current token's q/k/v (pre-rotation, the Q/K/V projection
// outputs read as Slices, common.h: [B][heads*D] and [B][kv_heads*D] or
// their split-K partial sums) are rotated here (RotaryEmbedding::apply), the
// current position's k/v come from LDS, and the workgroup with h < kv_heads
// writes them to the cache row pos (KVCache::append) -- no workgroup reads
// that row from memory in this launch.  Without ROPE, q is already rotated
// and all ctx rows come from the cache.
// KV: the cache element type (float, or uint16_t holding bf16 bits); with
// bf16, the current position's k/v are rounded in LDS as the cache stores them.
// Rows: grid.y = rows of q/out; row r is position (step ? *step : 0) + ctx0 +
// r % np of sequence r / np (np = 1: one position per sequence, decode; np
// > 1: the prompt rows of a prefill chunk, each attending causally).
// ns (ROPE, NormScale in common.h): q/k/v are projections of x * gamma and
// get the RMSNorm's 1 / rms here.
// NT: threads per workgroup (256, or 512 for a decode step of few heads:
// the same work in 8 waves, each phase half as long).
template <int D, bool ROPE, typename KV, int NT = kT>
__global__ __launch_bounds__(NT) void attention_k(Slices q, Slices kin, Slices vin, NormScale ns,
                                                  const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                  KV* kc, KV* vc, float* __restrict__ out, const int* __restrict__ step,
                                                  int ctx0, int np, int heads, int kv_heads, int max_seq,
                                                  float scale) {
    typedef typename KvRaw4<KV>::type Raw;
    constexpr int G = D / 4;        // float4 column groups
    constexpr int NW = NT / 64;
    constexpr int SL = NT / G;      // position slices in P*V
    constexpr int VP = (sizeof(KV) == 2 ? 16 : 8) * 128 / D * kT / NT;  // V rows per thread held in registers
    static_assert(VP >= 1, "V rows per thread");
    extern __shared__ float sc[];   // [max_seq] scores, then probabilities
    __shared__ __align__(16) float qs[D], ks[D], vs[D];
    __shared__ float4 part[SL][G];
    __shared__ float redf[NW];
    const int h = blockIdx.x, row = blockIdx.y, b = row / np, tid = threadIdx.x;
    const int pos = (step ? *step : 0) + ctx0 + row % np;  // the last position attended to
    const int ctx = pos + 1;
    const int kh = h % kv_heads;
    const int64_t crow = ((int64_t)b * kv_heads + kh) * max_seq;  // cache row of position 0
    const int nmem = ROPE ? pos : ctx;  // positions read from the cache
    const int g = tid % G, sl = tid / G;

    // Every load issued before the first wait, in order of use: the norm's
    // partial sums and the current token's q/k/v partials (and RoPE angles),
    // then this thread's K row of the first tile, then its V rows; the sums
    // of both come after.
    // Plain q/k/v (one slice, no epilogue: the decode GEMVs' own outputs)
    // are six loads; split-K partials are loaded without branches
    // (slice_issue_all) and added after the cache loads are issued.
    double npart[kNormBatch];
    if (ROPE && ns.ssp) norm_issue(ns, row, tid, NT, npart);
    const bool plain = q.n == 1 && !q.tscale && (!ROPE || (kin.n == 1 && vin.n == 1 && !kin.tscale && !vin.tscale));
    // (more than 4 waves: split-K q/k/v summed on the spot, the registers are short)
    constexpr bool RAW = NT <= kT;
    float raw[RAW ? (ROPE ? 6 : 1) : 1][kMaxSlices];
    float q1 = 0.0f, q2 = 0.0f, k1 = 0.0f, k2 = 0.0f, v1 = 0.0f, v2 = 0.0f, c = 0.0f, sn = 0.0f;
    if (ROPE) {
        if (tid < D / 2) {
            const int64_t qm = h * D + tid, km = kh * D + tid;
            if (!RAW && !plain) {
                q1 = slice_value(q, row, qm);
                q2 = slice_value(q, row, qm + D / 2);
                k1 = slice_value(kin, row, km);
                k2 = slice_value(kin, row, km + D / 2);
                v1 = slice_value(vin, row, km);
                v2 = slice_value(vin, row, km + D / 2);
            } else if (plain) {
                q1 = q.p[row * q.ts + qm];
                q2 = q.p[row * q.ts + qm + D / 2];
                k1 = kin.p[row * kin.ts + km];
                k2 = kin.p[row * kin.ts + km + D / 2];
                v1 = vin.p[row * vin.ts + km];
                v2 = vin.p[row * vin.ts + km + D / 2];
            } else if constexpr (RAW) {
                slice_issue_all(q, row, qm, raw[0]);
                slice_issue_all(q, row, qm + D / 2, raw[1]);
                slice_issue_all(kin, row, km, raw[2]);
                slice_issue_all(kin, row, km + D / 2, raw[3]);
                slice_issue_all(vin, row, km, raw[4]);
                slice_issue_all(vin, row, km + D / 2, raw[5]);
            }
            c = cos_t[(int64_t)pos * (D / 2) + tid];
            sn = sin_t[(int64_t)pos * (D / 2) + tid];
        }
    } else if (tid < D) {
        if (plain)
            q1 = q.p[row * q.ts + h * D + tid];
        else if constexpr (RAW)
            slice_issue_all(q, row, h * D + tid, raw[0]);
        else
            q1 = slice_value(q, row, h * D + tid);
    }
    // cache rows: K of the first KPRE rounds, then this thread's V rows.  A
    // K row is read by KL lanes, 16 bytes each (row kr of a round of KRR
    // rows, chunk kl), so that a load instruction covers whole rows.
    constexpr int KE = 16 / (int)sizeof(KV);  // cache elements per 16-byte chunk
    constexpr int KL = D / KE;                // lanes per K row
    constexpr int KRR = NT / KL;              // K rows per round
    constexpr int KPRE = 192 / KRR < 12 ? 192 / KRR : 12;  // rounds loaded up front (<= 192 rows)
    const int kl = tid % KL, kr = tid / KL;
    const KV* kchunk = kc + crow * D + kl * KE;
    uint4 kpre[KPRE];
#pragma unroll
    for (int i = 0; i < KPRE; ++i) {
        const int t = i * KRR + kr;
        kpre[i] = *(const uint4*)(kchunk + (int64_t)(t < nmem ? t : 0) * D);
    }
    // every wave's K rows issued before any wave goes on (the V rows follow
    // the staging below)
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const KV* vcol = vc + crow * D + 4 * g;
    Raw vpre[VP];
    if (RAW && !plain) {
        if (ROPE) {
            if (tid < D / 2) {
                q1 = slice_sum(q, row, raw[0]);
                q2 = slice_sum(q, row, raw[1]);
                k1 = slice_sum(kin, row, raw[2]);
                k2 = slice_sum(kin, row, raw[3]);
                v1 = slice_sum(vin, row, raw[4]);
                v2 = slice_sum(vin, row, raw[5]);
            }
        } else if (tid < D) {
            q1 = slice_sum(q, row, raw[0]);
        }
    }
    if (ROPE) {
        __shared__ double nred[NW];
        float ni = 1.0f;
        if (ns.ssp) {  // the RMSNorm's 1 / rms (NormScale): same sum as norm_scale
            const double sum = wave_sum_dbl(norm_finish(ns, row, tid, NT, npart));
            if ((tid & 63) == 0) nred[tid >> 6] = sum;
            __syncthreads();
            double t = 0.0;
#pragma unroll
            for (int w = 0; w < NW; ++w) t += nred[w];
            ni = (float)(1.0 / sqrt(t / (double)ns.dim + (double)ns.eps));
            q1 *= ni, q2 *= ni, k1 *= ni, k2 *= ni, v1 *= ni, v2 *= ni;
        }
        if (tid < D / 2) {
            qs[tid] = q1 * c - q2 * sn;
            qs[tid + D / 2] = q1 * sn + q2 * c;
            ks[tid] = kv_rounded(k1 * c - k2 * sn, KV{});
            ks[tid + D / 2] = kv_rounded(k1 * sn + k2 * c, KV{});
            vs[tid] = kv_rounded(v1, KV{});
            vs[tid + D / 2] = kv_rounded(v2, KV{});
        }
    } else if (tid < D) {
        qs[tid] = q1;
    }
    __syncthreads();  // qs, ks, vs
    // this thread's V rows, issued only now: the K rows of the other workgroups on the CU, issued meanwhile,
    // come back before them (batch 16, two workgroups per CU: decode +1.7 %; batch 1 unchanged)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < VP; ++j) {
        const int t = sl + SL * j;
        vpre[j] = kv_raw4(vcol + (int64_t)(t < nmem ? t : 0) * D);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (ROPE && h < kv_heads && tid < D) {
        kc[(crow + pos) * D + tid] = kv_store_value(ks[tid], KV{});
        vc[(crow + pos) * D + tid] = kv_store_value(vs[tid], KV{});
    }
    // scores: each lane's chunk against the same columns of q, summed over
    // the row's KL lanes (butterfly: every lane of the group gets the sum)
    float qv[KE];
#pragma unroll
    for (int e = 0; e < KE; ++e) qv[e] = qs[kl * KE + e];
    auto score = [&](const uint4& w) {
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int e = 0; e < KE; e += 2) {
            float k0, k1;
            if (sizeof(KV) == 2) {
                k0 = __uint_as_float(u[e / 2] << 16);
                k1 = __uint_as_float(u[e / 2] & 0xffff0000u);
            } else {
                k0 = __uint_as_float(u[e]);
                k1 = __uint_as_float(u[e + 1]);
            }
            s0 = s0 + qv[e] * k0;
            s1 = s1 + qv[e + 1] * k1;
        }
        return lanes_sum<KL>(s0 + s1) * scale;
    };
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < KPRE; ++i) {
        if (i * KRR >= nmem) break;  // uniform: rounds past the context
        const int t = i * KRR + kr;
        const float s = score(kpre[i]);
        if (t < nmem) {
            if (kl == 0) sc[t] = s;
            mx = fmaxf(mx, s);
        }
    }
    // rows past the preloaded rounds (contexts beyond KPRE * KRR rows): KB rounds' loads in flight together
    // (one round trip per KB rounds, not per round)
    constexpr int KB = 4;
    for (int t0 = KPRE * KRR; t0 < nmem; t0 += KB * KRR) {
        uint4 kb[KB];
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            const int t = t0 + b * KRR + kr;
            kb[b] = *(const uint4*)(kchunk + (int64_t)(t < nmem ? t : 0) * D);
        }
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            const int t = t0 + b * KRR + kr;
            const float s = score(kb[b]);
            if (t < nmem) {
                if (kl == 0) sc[t] = s;
                mx = fmaxf(mx, s);
            }
        }
    }
    if (ROPE && tid == (pos % NT)) {  // the current position, from LDS
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int d = 0; d < D; d += 4) {
            const float4 k4 = *(const float4*)(ks + d);
            const float4 q4 = *(const float4*)(qs + d);
            s0 = s0 + q4.x * k4.x;
            s1 = s1 + q4.y * k4.y;
            s2 = s2 + q4.z * k4.z;
            s3 = s3 + q4.w * k4.w;
        }
        const float s = ((s0 + s1) + (s2 + s3)) * scale;
        sc[pos] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max_w<NW>(mx, redf);
    float sum = 0.0f;
    for (int t = tid; t < ctx; t += NT) {
        const float e = expf(sc[t] - mx);
        sc[t] = e;
        sum += e;
    }
    sum = block_sum_w<NW>(sum, redf);   // its barriers also publish sc[]
    const float inv = 1.0f / sum;
    float4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto axpy = [](float4& a, float p, const float4& v) {
        a.x = fmaf(p, v.x, a.x);
        a.y = fmaf(p, v.y, a.y);
        a.z = fmaf(p, v.z, a.z);
        a.w = fmaf(p, v.w, a.w);
    };
#pragma unroll
    for (int j = 0; j < VP; ++j) {
        const int t = sl + SL * j;
        if (t < nmem) axpy(acc[j & 3], sc[t] * inv, kv_widen(vpre[j]));
    }
    // rows past the preloaded ones: 8 rows' loads in flight together (rows past the context read row 0 and
    // are not added)
    for (int t = sl + SL * VP; t < nmem; t += 8 * SL) {
        float4 v4[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int tj = t + j * SL;
            v4[j] = kv_load4(vcol + (int64_t)(tj < nmem ? tj : 0) * D);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int tj = t + j * SL;
            if (tj < nmem) axpy(acc[j & 3], sc[tj] * inv, v4[j]);
        }
    }
    if (ROPE && sl == (pos % SL)) axpy(acc[1], sc[pos] * inv, *(const float4*)(vs + 4 * g));
    acc[0].x += acc[1].x; acc[0].y += acc[1].y; acc[0].z += acc[1].z; acc[0].w += acc[1].w;
    acc[2].x += acc[3].x; acc[2].y += acc[3].y; acc[2].z += acc[3].z; acc[2].w += acc[3].w;
    acc[0].x += acc[2].x; acc[0].y += acc[2].y; acc[0].z += acc[2].z; acc[0].w += acc[2].w;
    part[sl][g] = acc[0];
    __syncthreads();
    if (tid < G) {
        float4 r = part[0][tid];
#pragma unroll
        for (int j = 1; j < SL; ++j) {
            const float4 o = part[j][tid];
            r.x += o.x;
            r.y += o.y;
            r.z += o.z;
            r.w += o.w;
        }
        *(float4*)(out + ((int64_t)row * heads + h) * D + 4 * tid) = r;
    }
}

// ---- SwiGLU fused with the per-token int8 quantisation ----------------------
// One workgroup of 1024 threads per token: a = silu(g) * u kept in registers
// (kSQ per thread, all loads issued before any use), then quantize_per_token
// (src/int8_quant.cpp:8-31): max|a| (floor 1e-10), scale = 127/max,
// q = (int8)round_half_away(a * scale), inv = max/127.  n <= kSQT * kSQ.
constexpr int kSQT = 1024, kSQ = 12;
// act (optional): the FP32 activations, [rows][n].
// g, u: the gate and up outputs as Slices (common.h), so the split-K
// partial sums of the GEMV are added here.
// ns (NormScale, common.h): g/u are projections of x * gamma and get the
// RMSNorm's 1 / rms here.
__global__ __launch_bounds__(kSQT) void silu_mul_quant_k(Slices g, Slices u, NormScale ns, int8_t* __restrict__ q,
                                                         float* __restrict__ inv_scale, float* __restrict__ act,
                                                         int n) {
    __shared__ float red[kSQT / 64];
    __shared__ double nred[kSQT / 64];
    const int r = blockIdx.x, tid = threadIdx.x;
    double npart[kNormBatch];  // the norm's partial sums, loaded first
    if (ns.ssp) norm_issue(ns, r, tid, kSQT, npart);
    float gv[kSQ], uv[kSQ];
    if (g.n == 1 && u.n == 1) {
        const float* gr = g.p + r * g.ts;
        const float* ur = u.p + r * u.ts;
#pragma unroll
        for (int j = 0; j < kSQ; ++j) {
            const int i = tid + j * kSQT;
            gv[j] = i < n ? gr[i] : 0.0f;
            uv[j] = i < n ? ur[i] : 0.0f;
        }
    } else {
#pragma unroll
        for (int j = 0; j < kSQ; ++j) {
            const int i = tid + j * kSQT;
            gv[j] = i < n ? slice_value(g, r, i) : 0.0f;
            uv[j] = i < n ? slice_value(u, r, i) : 0.0f;
        }
    }
    if (ns.ssp) {
        const float ni = norm_scale_issued<kSQT / 64>(ns, r, npart, nred);
#pragma unroll
        for (int j = 0; j < kSQ; ++j) {
            gv[j] *= ni;
            uv[j] *= ni;
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < kSQ; ++j) {
        gv[j] = silu1(gv[j]) * uv[j];
        m = fmaxf(m, fabsf(gv[j]));
    }
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < kSQT / 64; ++w) m = fmaxf(m, red[w]);
    if (m < 1e-10f) m = 1e-10f;
    const float sc = __fdiv_rn(127.0f, m);
    int8_t* qr = q + (int64_t)r * n;
#pragma unroll
    for (int j = 0; j < kSQ; ++j) {
        const int i = tid + j * kSQT;
        if (i < n) qr[i] = (int8_t)quant_i8(gv[j], sc);
    }
    if (act) {
        float* ar = act + (int64_t)r * n;
#pragma unroll
        for (int j = 0; j < kSQ; ++j) {
            const int i = tid + j * kSQT;
            if (i < n) ar[i] = gv[j];
        }
    }
    if (tid == 0) inv_scale[r] = __fdiv_rn(m, 127.0f);
}

// ---- greedy argmax + token bookkeeping ---------------------------------------
// Sampler::greedy: first index of the maximum of a row; NaN never wins,
// all-NaN / all -inf rows give 0.  (value, index) pairs combine by larger
// value, then smaller index.
__device__ __forceinline__ void amax_merge(float& v, int& i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}
__device__ __forceinline__ void block_amax(float& v, int& i, float* bv, int* bi) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax_merge(v, i, __shfl_xor(v, o, MTH_WAVE), __shfl_xor(i, o, MTH_WAVE));
    if (lane == 0) {
        bv[wave] = v;
        bi[wave] = i;
    }
    __syncthreads();
    v = bv[0];
    i = bi[0];
#pragma unroll
    for (int w = 1; w < kT / 64; ++w) amax_merge(v, i, bv[w], bi[w]);
}

// Stage 1: workgroup (chunk c, row b) scans columns [c*chunk, (c+1)*chunk)
// with float4 loads and writes its (value, index) pair.  chunk % 4 == 0.
__global__ __launch_bounds__(kT) void argmax_part_k(const float* __restrict__ logits, int64_t n, int chunk,
                                                    float* __restrict__ pv, int* __restrict__ pi) {
    __shared__ float bv[kT / 64];
    __shared__ int bi[kT / 64];
    const float* r = logits + (int64_t)blockIdx.y * n;
    const int64_t c0 = (int64_t)blockIdx.x * chunk;
    const int64_t c1 = c0 + chunk < n ? c0 + chunk : n;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    const bool vec = (n % 4) == 0;
    for (int64_t i = c0 + 4 * threadIdx.x; i < c1; i += 4 * kT) {
        if (vec && i + 3 < c1) {
            const float4 x = ldf4(r + i);
            if (x.x > v) { v = x.x; idx = (int)i; }
            if (x.y > v) { v = x.y; idx = (int)i + 1; }
            if (x.z > v) { v = x.z; idx = (int)i + 2; }
            if (x.w > v) { v = x.w; idx = (int)i + 3; }
        } else {
            for (int64_t j = i; j < i + 4 && j < c1; ++j)
                if (r[j] > v) { v = r[j]; idx = (int)j; }
        }
    }
    block_amax(v, idx, bv, bi);
    if (threadIdx.x == 0) {
        pv[blockIdx.y * gridDim.x + blockIdx.x] = v;
        pi[blockIdx.y * gridDim.x + blockIdx.x] = idx;
    }
}

// Stage 2 (one workgroup): row b's result from its nc partials -> ids[b];
// with hist, the next input token hist[b][s + 1] once the prompt is consumed
// (s + 1 >= prompt_len); with step, then advances *step (the last launch of a
// decode step: every earlier kernel of the step has read it).
__global__ __launch_bounds__(kT) void argmax_final_k(const float* __restrict__ pv, const int* __restrict__ pi, int nc,
                                                     int rows, int* __restrict__ ids, int* __restrict__ hist,
                                                     int* step, int hist_stride, int prompt_len) {
    __shared__ float bv[kT / 64];
    __shared__ int bi[kT / 64];
    const int s = step ? *step : 0;
    for (int b = 0; b < rows; ++b) {
        float v = -INFINITY;
        int idx = 0x7fffffff;
        for (int c = threadIdx.x; c < nc; c += kT) amax_merge(v, idx, pv[b * nc + c], pi[b * nc + c]);
        block_amax(v, idx, bv, bi);
        if (threadIdx.x == 0) {
            const int best = idx == 0x7fffffff ? 0 : idx;
            if (ids) ids[b] = best;
            if (hist && s + 1 >= prompt_len && s + 1 < hist_stride) hist[(int64_t)b * hist_stride + s + 1] = best;
        }
        __syncthreads();
    }
    if (step && threadIdx.x == 0) *step = s + 1;
}

// x[b] = emb[id] with id = hist[b][*step] (ids outside [0, vocab) -> 0).
// ro.x set: also xg = x * ro.gamma and ro.ssp[b] = sum x^2 (ResidOut,
// common.h; one partial per token).
__global__ __launch_bounds__(kT) void embed_k(const float* __restrict__ emb, const int* __restrict__ hist,
                                              const int* __restrict__ step, int hist_stride, float* __restrict__ x,
                                              int dim, int vocab, ResidOut ro) {
    __shared__ double red[kT / 64];
    const int b = blockIdx.x;
    int id = hist[(int64_t)b * hist_stride + *step];
    if (id < 0 || id >= vocab) id = 0;
    const float* src = emb + (int64_t)id * dim;
    float* dst = x + (int64_t)b * dim;
    double sq = 0.0;
    for (int i = threadIdx.x * 4; i < dim; i += kT * 4) {
        const float4 v = ldf4(src + i);
        *(float4*)(dst + i) = v;
        if (ro.x) {
            const float4 g = ldf4(ro.gamma + i);
            *(float4*)(ro.xg + (int64_t)b * dim + i) = make_float4(v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w);
            sq += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
        }
    }
    if (ro.x) {
        sq = block_sum(sq, red);
        if (threadIdx.x == 0) ro.ssp[b] = sq;
    }
}

// Prefill rows: row r is position p0 + r % np of sequence r / np.
// x[r] = emb[id], id = hist[r / np][p0 + r % np] (ids outside [0, vocab) -> 0).
__global__ __launch_bounds__(kT) void embed_rows_k(const float* __restrict__ emb, const int* __restrict__ hist,
                                                   int hist_stride, float* __restrict__ x, int dim, int vocab, int np,
                                                   int p0) {
    const int r = blockIdx.x;
    int id = hist[(int64_t)(r / np) * hist_stride + p0 + r % np];
    if (id < 0 || id >= vocab) id = 0;
    const float* src = emb + (int64_t)id * dim;
    float* dst = x + (int64_t)r * dim;
    for (int i = threadIdx.x * 4; i < dim; i += kT * 4) *(float4*)(dst + i) = ldf4(src + i);
}

// RoPE of row r's q (in place) and k at its position, k and v appended to
// the caches at that position (rope_kv_k per row; KV: cache element type,
// values stored as the decode attention stores them).
template <typename KV>
__global__ __launch_bounds__(kT) void rope_kv_rows_k(float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v, const float* __restrict__ cos_t,
                                                     const float* __restrict__ sin_t, KV* __restrict__ kc,
                                                     KV* __restrict__ vc, int np, int p0, int heads, int kv_heads,
                                                     int D, int max_seq) {
    const int r = blockIdx.x, b = r / np, pos = p0 + r % np;
    const int h2 = D / 2;
    const float* cr = cos_t + (int64_t)pos * h2;
    const float* sr = sin_t + (int64_t)pos * h2;
    float* qb = q + (int64_t)r * heads * D;
    for (int i = threadIdx.x; i < heads * h2; i += kT) {
        const int h = i / h2, d = i % h2;
        float* p = qb + h * D;
        const float x1 = p[d], x2 = p[d + h2], c = cr[d], s = sr[d];
        p[d] = x1 * c - x2 * s;
        p[d + h2] = x1 * s + x2 * c;
    }
    const float* kb = k + (int64_t)r * kv_heads * D;
    const float* vb = v + (int64_t)r * kv_heads * D;
    for (int i = threadIdx.x; i < kv_heads * h2; i += kT) {
        const int h = i / h2, d = i % h2;
        const float* p = kb + h * D;
        const float x1 = p[d], x2 = p[d + h2], c = cr[d], s = sr[d];
        const int64_t row = (((int64_t)b * kv_heads + h) * max_seq + pos) * D;
        kc[row + d] = kv_store_value(x1 * c - x2 * s, KV{});
        kc[row + d + h2] = kv_store_value(x1 * s + x2 * c, KV{});
        vc[row + d] = kv_store_value(vb[h * D + d], KV{});
        vc[row + d + h2] = kv_store_value(vb[h * D + d + h2], KV{});
    }
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + kT - 1) / kT); }
inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

hipError_t launch_rms_norm_slices(float* x, const Slices& t, const float* gamma, float* y, int64_t rows, int64_t dim,
                                  float eps, hipStream_t s) {
    const bool t_al = t.n == 0 || (al16(t.p) && t.ts % 4 == 0 && t.zs % 4 == 0);
    if (dim % 4 == 0 && dim < (1ll << 31) && al16(x) && al16(y) && al16(gamma) && t_al)
        rms_norm_k<<<(unsigned)rows, kRN, 0, s>>>(x, t, gamma, y, (int)dim, eps);
    else
        rms_norm_any_k<<<(unsigned)rows, kT, 0, s>>>(x, t, gamma, y, dim, eps);
    return hipGetLastError();
}

bool resid_split_supported(const float* x, const Slices& t, const float* gamma, const float* xg, int64_t rows,
                           int64_t dim) {
    const bool t_al = t.n == 0 || (al16(t.p) && t.ts % 4 == 0 && t.zs % 4 == 0);
    return dim % 4 == 0 && dim < (1ll << 31) && rows >= 1 && rows <= 65535 && al16(x) && al16(gamma) && al16(xg) &&
           t_al && t.n <= kMaxSlices;
}

int resid_split_parts(int64_t dim) { return (int)((dim + 4 * kRS - 1) / (4 * kRS)); }

hipError_t launch_resid_split(float* x, const Slices& t, const float* gamma, float* xg, double* ssp, int64_t rows,
                              int64_t dim, int* nparts, hipStream_t s) {
    if (!resid_split_supported(x, t, gamma, xg, rows, dim)) return hipErrorInvalidValue;
    const int np = resid_split_parts(dim);
    resid_split_k<<<dim3((unsigned)np, (unsigned)rows), kRS, 0, s>>>(x, t, gamma, xg, ssp, (int)dim);
    if (nparts) *nparts = np;
    return hipGetLastError();
}

hipError_t launch_rms_norm(float* x, const float* t, const float* gamma, float* y, int64_t rows, int64_t dim,
                           float eps, hipStream_t s) {
    const Slices ts = t ? plain_slices(t, dim) : Slices{nullptr, 0, 0, 0, 1.0f, nullptr};
    return launch_rms_norm_slices(x, ts, gamma, y, rows, dim, eps, s);
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

hipError_t launch_softmax_axis(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner, hipStream_t s) {
    if (inner == 1) return launch_softmax(x, y, outer, dim, s);
    softmax_strided_k<<<blocks_for(outer * inner), kT, 0, s>>>(x, y, outer, dim, inner);
    return hipGetLastError();
}

hipError_t launch_axpby(float alpha, const float* x, float beta, float* y, int64_t n, hipStream_t s) {
    axpby_k<<<blocks_for(n), kT, 0, s>>>(alpha, x, beta, y, n);
    return hipGetLastError();
}

hipError_t launch_gemv_f32(float alpha, const float* A, const float* x, float beta, float* y, int64_t M, int64_t N,
                           hipStream_t s) {
    gemv_f32_k<<<(unsigned)((M + kT / 64 - 1) / (kT / 64)), kT, 0, s>>>(alpha, A, x, beta, y, M, N);
    return hipGetLastError();
}

hipError_t launch_relu(const float* x, float* y, int64_t n, hipStream_t s) {
    relu_k<<<blocks_for(n), kT, 0, s>>>(x, y, n);
    return hipGetLastError();
}

hipError_t launch_gelu(const float* x, float* y, int64_t n, hipStream_t s) {
    gelu_k<<<blocks_for(n), kT, 0, s>>>(x, y, n);
    return hipGetLastError();
}

hipError_t launch_scale(float a, const float* x, float* y, int64_t n, hipStream_t s) {
    scale_k<<<blocks_for(n), kT, 0, s>>>(a, x, y, n);
    return hipGetLastError();
}

hipError_t launch_layer_norm(const float* x, const float* gamma, const float* beta, float* y, int64_t rows,
                             int64_t dim, float eps, hipStream_t s) {
    layer_norm_k<<<(unsigned)rows, kT, 0, s>>>(x, gamma, beta, y, dim, eps);
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

// ---- prompt attention --------------------------------------------------------
// Workgroup (head h, sequence b, tile of up to 64 query rows): rows
// b np + i (i in [64 z, 64 z + 64) and < np) of q / out, at positions
// p0 + i, each attending causally to cache rows 0 .. p0 + i of kv head
// h % kv_heads (the decode kernel's semantics, one workgroup per row, for a
// whole tile of rows at once, so each K / V row is read once per 64 query
// rows).  The context streams through LDS in tiles of 64 positions; per
// tile: scores (FP32, dot products over d in order, times 1 / sqrt(D)) of a
// 4 x 4 block per thread (rows 4 (t / 16) + a, positions t % 16 + 16 c),
// the causal mask, a running maximum per row with the earlier tiles' sums
// and outputs rescaled by exp(m_old - m_new), exp(s - m) into LDS, and
// P V accumulated per thread for its 4 rows x D / 16 columns; at the end
// the rows are divided by their sums.  The same softmax and weighted sum as
// the decode kernel up to FP32 rounding order.
namespace {
template <int D, typename KV>
__global__ __launch_bounds__(256) void attn_prefill_k(const float* __restrict__ q, const KV* __restrict__ kc,
                                                      const KV* __restrict__ vc, float* __restrict__ out, int np,
                                                      int p0, int heads, int kv_heads, int max_seq, float scale) {
    constexpr int QT = 64, KT = 64, DP = D + 4, PP = KT + 4, NC = D / 64;
    __shared__ __align__(16) float Qs[QT * DP];
    __shared__ __align__(16) float Ks[KT * DP];
    __shared__ __align__(16) float Vs[KT * DP];
    __shared__ __align__(16) float Ps[QT * PP];
    const int h = blockIdx.x, b = blockIdx.y, i0 = blockIdx.z * QT, tid = threadIdx.x;
    const int nq = min(QT, np - i0);
    const int kh = h % kv_heads;
    const int64_t crow = ((int64_t)b * kv_heads + kh) * max_seq;  // cache row of position 0
    const int64_t qstride = (int64_t)heads * D;
    const int ctx = p0 + i0 + nq;  // positions the tile's last row attends to
    const int qg = tid >> 4, kg = tid & 15;
    for (int c = tid; c < QT * (D / 4); c += 256) {
        const int r = c / (D / 4), d = 4 * (c % (D / 4));
        *(float4*)(Qs + r * DP + d) = r < nq ? *(const float4*)(q + (int64_t)(b * np + i0 + r) * qstride + h * D + d)
                                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float m[4], l[4];
    float4 o[4][NC];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        m[a] = -INFINITY;
        l[a] = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) o[a][c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    for (int t0 = 0; t0 < ctx; t0 += KT) {
        __syncthreads();  // the previous tile's K, V and P are consumed
        for (int c = tid; c < KT * (D / 4); c += 256) {
            const int r = c / (D / 4), d = 4 * (c % (D / 4)), t = t0 + r;
            const bool in = t < ctx;
            const int64_t off = (crow + (in ? t : 0)) * D + d;
            *(float4*)(Ks + r * DP + d) = in ? kv_load4(kc + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            *(float4*)(Vs + r * DP + d) = in ? kv_load4(vc + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        __syncthreads();
        float s[4][4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int c = 0; c < 4; ++c) s[a][c] = 0.0f;
        for (int d = 0; d < D; d += 4) {
            float4 qv[4], kv[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) qv[a] = *(const float4*)(Qs + (4 * qg + a) * DP + d);
#pragma unroll
            for (int c = 0; c < 4; ++c) kv[c] = *(const float4*)(Ks + (kg + 16 * c) * DP + d);
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float t = s[a][c];
                    t = fmaf(qv[a].x, kv[c].x, t);
                    t = fmaf(qv[a].y, kv[c].y, t);
                    t = fmaf(qv[a].z, kv[c].z, t);
                    s[a][c] = fmaf(qv[a].w, kv[c].w, t);
                }
        }
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const int qp = p0 + i0 + 4 * qg + a;  // position of row a (rows past nq: masked like any row)
            float tm = -INFINITY;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int kp = t0 + kg + 16 * c;
                s[a][c] = kp <= qp ? s[a][c] * scale : -INFINITY;
                tm = fmaxf(tm, s[a][c]);
            }
            tm = group_reduce<16>(tm, MaxOp{});
            const float mn = fmaxf(m[a], tm);  // finite: position 0 is in the first tile of every row
            const float alpha = expf(m[a] - mn);
            float rs = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float p = expf(s[a][c] - mn);
                Ps[(4 * qg + a) * PP + kg + 16 * c] = p;
                rs += p;
            }
            rs = group_reduce<16>(rs, AddOp{});
            l[a] = fmaf(l[a], alpha, rs);
            m[a] = mn;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                o[a][c].x *= alpha;
                o[a][c].y *= alpha;
                o[a][c].z *= alpha;
                o[a][c].w *= alpha;
            }
        }
        __syncthreads();
        const int jn = min(KT, ctx - t0);
        for (int j = 0; j < jn; ++j) {
            float4 vv[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) vv[c] = *(const float4*)(Vs + j * DP + 4 * kg + 64 * c);
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const float p = Ps[(4 * qg + a) * PP + j];
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    o[a][c].x = fmaf(p, vv[c].x, o[a][c].x);
                    o[a][c].y = fmaf(p, vv[c].y, o[a][c].y);
                    o[a][c].z = fmaf(p, vv[c].z, o[a][c].z);
                    o[a][c].w = fmaf(p, vv[c].w, o[a][c].w);
                }
            }
        }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        const int r = 4 * qg + a;
        if (r >= nq) continue;
        const float inv = 1.0f / l[a];
        float* dst = out + (int64_t)(b * np + i0 + r) * qstride + h * D + 4 * kg;
#pragma unroll
        for (int c = 0; c < NC; ++c)
            *(float4*)(dst + 64 * c) = make_float4(o[a][c].x * inv, o[a][c].y * inv, o[a][c].z * inv, o[a][c].w * inv);
    }
}

}  // namespace

template <bool ROPE, typename KV>
static hipError_t run_attention(const Slices& q, const Slices& k, const Slices& v, const NormScale& ns,
                                const float* cos_t, const float* sin_t, KV* kc, KV* vc, float* out, const int* step,
                                int ctx0, int64_t rows, int np, int heads, int kv_heads, int head_dim, int max_seq,
                                hipStream_t s) {
    // the kernel reads 1..kMaxSlices partials of q (and of k, v with RoPE)
    auto bad = [](const Slices& x) { return x.n < 1 || x.n > kMaxSlices; };
    if (bad(q) || (ROPE && (bad(k) || bad(v)))) return hipErrorInvalidValue;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const size_t lds = (size_t)max_seq * sizeof(float);
    const dim3 grid((unsigned)heads, (unsigned)rows);
    // few workgroups (a decode step of a handful of sequences): 8 waves each (16 measured 0.9 % slower for a
    // batch-1 decode step once the V rows were issued after the staging, 4 waves 1.3 % slower)
    const bool wide = ROPE && np == 1 && rows * heads <= 128;
    // long contexts (more than 1024 positions) of a few rows x heads: 16 waves, twice the cache loads in flight
    const bool wider = np == 1 && rows * heads <= 128 && max_seq > 1024;
    if (wider) {
        if (head_dim == 64)
            attention_k<64, ROPE, KV, 1024><<<grid, 1024, lds, s>>>(q, k, v, ns, cos_t, sin_t, kc, vc, out, step,
                                                                      ctx0, np, heads, kv_heads, max_seq, scale);
        else if (head_dim == 128)
            attention_k<128, ROPE, KV, 1024><<<grid, 1024, lds, s>>>(q, k, v, ns, cos_t, sin_t, kc, vc, out, step,
                                                                       ctx0, np, heads, kv_heads, max_seq, scale);
        else
            attention_k<256, ROPE, KV, 1024><<<grid, 1024, lds, s>>>(q, k, v, ns, cos_t, sin_t, kc, vc, out, step,
                                                                       ctx0, np, heads, kv_heads, max_seq, scale);
        return hipGetLastError();
    }
    if (head_dim == 64) {
        if (wide)
            attention_k<64, ROPE, KV, 512><<<grid, 512, lds, s>>>(q, k, v, ns, cos_t, sin_t, kc, vc, out, step,
                                                                    ctx0, np, heads, kv_heads, max_seq, scale);
        else
            attention_k<64, ROPE, KV><<<grid, kT, lds, s>>>(q, k, v, ns, cos_t, sin_t, kc, vc, out, step, ctx0, np,
                                                            heads, kv_heads, max_seq, scale);
    } else if (head_dim == 128) {
        if (wide)
            attention_k<128, ROPE, KV, 512><<<grid, 512, lds, s>>>(q, k, v, ns, cos_t, sin_t, kc, vc, out, step,
                                                                     ctx0, np, heads, kv_heads, max_seq, scale);
        else
            attention_k<128, ROPE, KV><<<grid, kT, lds, s>>>(q, k, v, ns, cos_t, sin_t, kc, vc, out, step, ctx0,
                                                             np, heads, kv_heads, max_seq, scale);
    } else {
        if (wide)
            attention_k<256, ROPE, KV, 512><<<grid, 512, lds, s>>>(q, k, v, ns, cos_t, sin_t, kc, vc, out, step,
                                                                     ctx0, np, heads, kv_heads, max_seq, scale);
        else
            attention_k<256, ROPE, KV><<<grid, kT, lds, s>>>(q, k, v, ns, cos_t, sin_t, kc, vc, out, step, ctx0,
                                                             np, heads, kv_heads, max_seq, scale);
    }
    return hipGetLastError();
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc, float* out, const int* step, int ctx0,
                            int64_t batch, int heads, int kv_heads, int head_dim, int max_seq, hipStream_t s) {
    const Slices qs = plain_slices(q, (int64_t)heads * head_dim), none{nullptr, 0, 0, 0, 1.0f, nullptr};
    return run_attention<false, float>(qs, none, none, NormScale{}, nullptr, nullptr, (float*)kc, (float*)vc, out,
                                       step, ctx0, batch, 1, heads, kv_heads, head_dim, max_seq, s);
}

hipError_t launch_attention_rows(const float* q, const void* kc, const void* vc, bool kv_bf16, float* out,
                                 int64_t rows, int np, int p0, int heads, int kv_heads, int head_dim, int max_seq,
                                 hipStream_t s) {
    const Slices qs = plain_slices(q, (int64_t)heads * head_dim), none{nullptr, 0, 0, 0, 1.0f, nullptr};
    // tiles of query rows (a prompt chunk of 16 positions or more per sequence)
    const bool aligned = (((uintptr_t)q | (uintptr_t)out | (uintptr_t)kc | (uintptr_t)vc) & 15u) == 0;
    if (np >= 16 && aligned && (head_dim == 64 || head_dim == 128) && rows % np == 0 && rows / np <= 65535 &&
        heads <= 65535) {
        const dim3 grid((unsigned)heads, (unsigned)(rows / np), (unsigned)((np + 63) / 64));
        const float scale = 1.0f / sqrtf((float)head_dim);
        if (head_dim == 64) {
            if (kv_bf16)
                attn_prefill_k<64, uint16_t><<<grid, 256, 0, s>>>(q, (const uint16_t*)kc, (const uint16_t*)vc, out, np,
                                                                   p0, heads, kv_heads, max_seq, scale);
            else
                attn_prefill_k<64, float><<<grid, 256, 0, s>>>(q, (const float*)kc, (const float*)vc, out, np, p0,
                                                                heads, kv_heads, max_seq, scale);
        } else {
            if (kv_bf16)
                attn_prefill_k<128, uint16_t><<<grid, 256, 0, s>>>(q, (const uint16_t*)kc, (const uint16_t*)vc, out,
                                                                    np, p0, heads, kv_heads, max_seq, scale);
            else
                attn_prefill_k<128, float><<<grid, 256, 0, s>>>(q, (const float*)kc, (const float*)vc, out, np, p0,
                                                                 heads, kv_heads, max_seq, scale);
        }
        return hipGetLastError();
    }
    if (kv_bf16)
        return run_attention<false, uint16_t>(qs, none, none, NormScale{}, nullptr, nullptr, (uint16_t*)kc,
                                              (uint16_t*)vc, out, nullptr, p0, rows, np, heads, kv_heads, head_dim,
                                              max_seq, s);
    return run_attention<false, float>(qs, none, none, NormScale{}, nullptr, nullptr, (float*)kc, (float*)vc, out,
                                       nullptr, p0, rows, np, heads, kv_heads, head_dim, max_seq, s);
}

hipError_t launch_rope_attention(const float* q, const float* k, const float* v, const float* cos_t,
                                 const float* sin_t, void* kc, void* vc, bool kv_bf16, float* out, const int* step,
                                 int64_t batch, int heads, int kv_heads, int head_dim, int max_seq, hipStream_t s) {
    return launch_rope_attention_slices(plain_slices(q, (int64_t)heads * head_dim),
                                        plain_slices(k, (int64_t)kv_heads * head_dim),
                                        plain_slices(v, (int64_t)kv_heads * head_dim), NormScale{}, cos_t, sin_t, kc,
                                        vc, kv_bf16, out, step, batch, heads, kv_heads, head_dim, max_seq, s);
}

hipError_t launch_rope_attention_slices(const Slices& q, const Slices& k, const Slices& v, const NormScale& ns,
                                        const float* cos_t, const float* sin_t, void* kc, void* vc, bool kv_bf16,
                                        float* out, const int* step, int64_t batch, int heads, int kv_heads,
                                        int head_dim, int max_seq, hipStream_t s) {
    if (kv_bf16)
        return run_attention<true, uint16_t>(q, k, v, ns, cos_t, sin_t, (uint16_t*)kc, (uint16_t*)vc, out, step, 0,
                                             batch, 1, heads, kv_heads, head_dim, max_seq, s);
    return run_attention<true, float>(q, k, v, ns, cos_t, sin_t, (float*)kc, (float*)vc, out, step, 0, batch, 1,
                                      heads, kv_heads, head_dim, max_seq, s);
}

bool silu_mul_quant_supported(int64_t n) { return n > 0 && n <= (int64_t)kSQT * kSQ; }

hipError_t launch_silu_mul_quant_slices(const Slices& g, const Slices& u, const NormScale& ns, int8_t* q,
                                        float* inv_scale, float* act, int64_t rows, int64_t n, hipStream_t s) {
    silu_mul_quant_k<<<(unsigned)rows, kSQT, 0, s>>>(g, u, ns, q, inv_scale, act, (int)n);
    return hipGetLastError();
}

hipError_t launch_silu_mul_quant(const float* g, const float* u, int8_t* q, float* inv_scale, float* act,
                                 int64_t rows, int64_t n, int64_t gstride, int64_t ustride, hipStream_t s) {
    return launch_silu_mul_quant_slices(plain_slices(g, gstride), plain_slices(u, ustride), NormScale{}, q, inv_scale,
                                        act, rows, n, s);
}

int argmax_chunks(int64_t n) { return (int)((n + kArgChunk - 1) / kArgChunk); }

hipError_t launch_argmax(const float* logits, int64_t rows, int64_t n, int* ids, int* hist, int* step,
                         int hist_stride, int prompt_len, float* pv, int* pi, hipStream_t s) {
    const int nc = argmax_chunks(n);
    argmax_part_k<<<dim3((unsigned)nc, (unsigned)rows), kT, 0, s>>>(logits, n, kArgChunk, pv, pi);
    argmax_final_k<<<1, kT, 0, s>>>(pv, pi, nc, (int)rows, ids, hist, step, hist_stride, prompt_len);
    return hipGetLastError();
}

hipError_t launch_embed_rows(const float* emb, const int* hist, int hist_stride, float* x, int64_t rows, int np, int p0,
                             int dim, int vocab, hipStream_t s) {
    embed_rows_k<<<(unsigned)rows, kT, 0, s>>>(emb, hist, hist_stride, x, dim, vocab, np, p0);
    return hipGetLastError();
}

hipError_t launch_rope_kv_rows(float* q, const float* k, const float* v, const float* cos_t, const float* sin_t,
                               void* kc, void* vc, bool kv_bf16, int64_t rows, int np, int p0, int heads, int kv_heads,
                               int head_dim, int max_seq, hipStream_t s) {
    if (kv_bf16)
        rope_kv_rows_k<uint16_t><<<(unsigned)rows, kT, 0, s>>>(q, k, v, cos_t, sin_t, (uint16_t*)kc, (uint16_t*)vc, np,
                                                               p0, heads, kv_heads, head_dim, max_seq);
    else
        rope_kv_rows_k<float><<<(unsigned)rows, kT, 0, s>>>(q, k, v, cos_t, sin_t, (float*)kc, (float*)vc, np, p0,
                                                            heads, kv_heads, head_dim, max_seq);
    return hipGetLastError();
}

hipError_t launch_embed(const float* emb, const int* hist, const int* step, int hist_stride, float* x, int64_t batch,
                        int dim, int vocab, hipStream_t s, const ResidOut& ro) {
    embed_k<<<(unsigned)batch, kT, 0, s>>>(emb, hist, step, hist_stride, x, dim, vocab, ro);
    return hipGetLastError();
}

}  // namespace mth
