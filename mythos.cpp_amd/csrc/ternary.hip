// ternary.hip — int8 activation quantisation and the ternary (I2_S / TL)
// kernels on gfx950.
//
// Replaces src/int8_quant.cpp:8-41 and src/kernel_i2s.cpp:32-65,201-235,
// src/kernel_tl.cpp:13-168.  Every ternary result is an exact integer dot
// product followed by the reference's FP32 epilogue, so outputs are bit-exact
// against the reference (not merely close).
//
// I2_S packing (src/kernel_i2s.cpp:13-30): element 4i+j of a row is bits
// 2j..2j+1 of byte i, code 00 -> -1, 01 -> 0, 10 -> +1, 11 -> +1.
//
// Fast I2_S GEMV (decode):
//   * the workgroup quantises the token's activations once into LDS
//     (max|x| block reduction, IEEE 127/max, round-half-away, int8);
//   * LPR lanes share a row; lane li owns 16-byte weight segments
//     seg = li + LPR*s (64 weights each) and keeps the matching 64 int8
//     activations in VGPRs, byte-transposed so that one dword of packed
//     weights feeds four v_dot4_i32_i8 without moving weight bits around;
//   * codes are mapped to u = t+1 in {0,1,2} in place (code 3 -> 2 by one
//     subtract), so sum(t*a) = sum(u*a) - sum(a), with sum(a) per lane
//     computed once;
//   * the int32 row sum is reduced across the LPR lanes and the epilogue is
//     ((float)sum * w_scale) * inv_scale, exactly the reference's order.
#include "common.h"
#include "launch.h"

namespace mth {
namespace {

constexpr int kWG = 256;
constexpr int kWaves = kWG / MTH_WAVE;

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Block-wide max of |x[0..K)| with the reference's floor (int8_quant.cpp:10-15).
// Returns max_abs in every thread.  Uses red[kWaves].
__device__ __forceinline__ float block_absmax(const float* __restrict__ x, int64_t K, float* red) {
    float m = 0.0f;
    for (int64_t k = threadIdx.x; k < K; k += kWG) m = fmaxf(m, fabsf(x[k]));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) r = fmaxf(r, red[w]);
    if (r < 1e-10f) r = 1e-10f;
    return r;
}

// ---------------------------------------------------------------------------
// quantize_per_token: one workgroup per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kWG) void quantize_rows(const float* __restrict__ src, int8_t* __restrict__ dst,
                                                     float* __restrict__ scale, float* __restrict__ inv,
                                                     int64_t cols) {
    __shared__ float red[kWaves];
    const int64_t row = blockIdx.x;
    const float* x = src + row * cols;
    const float mx = block_absmax(x, cols, red);
    const float sc = __fdiv_rn(127.0f, mx);
    for (int64_t k = threadIdx.x; k < cols; k += kWG) dst[row * cols + k] = (int8_t)quant_i8(x[k], sc);
    if (threadIdx.x == 0) {
        if (scale) scale[row] = sc;
        if (inv) inv[row] = __fdiv_rn(mx, 127.0f);
    }
}

// u-code dword: codes 3 -> 2 (t = u - 1 with u in {0,1,2}), field-wise.
__device__ __forceinline__ uint32_t ucode(uint32_t w) { return w - ((w >> 1) & w & 0x55555555u); }

// dot of 16 ternary weights (one dword of codes) with 16 transposed acts.
__device__ __forceinline__ int tdot16(uint32_t w, const uint32_t (&A)[4], int acc) {
    const uint32_t u = ucode(w);
    acc = dot4(u & 0x03030303u, A[0], acc);
    acc = dot4((u >> 2) & 0x03030303u, A[1], acc);
    acc = dot4((u >> 4) & 0x03030303u, A[2], acc);
    acc = dot4((u >> 6) & 0x03030303u, A[3], acc);
    return acc;
}

// ---------------------------------------------------------------------------
// Fast I2_S GEMV.  Requires K % 64 == 0, K <= 64*LPR*NSEG, 16-byte aligned
// packed weights.  Dynamic LDS: K bytes of quantised activations.
// ---------------------------------------------------------------------------
// Workgroup = 4 waves x (64/LPR) rows; the weight loads are released once
// the activations are in (see below) and stay in registers over the tokens
// of a batch.
template <int LPR, int NSEG, bool FUSED>
__global__ __launch_bounds__(kWG, 2) void i2s_gemv_fast(
    const uint8_t* packed, float w_scale, const float* __restrict__ x,
    const int8_t* __restrict__ act, const float* __restrict__ act_scale, float* __restrict__ y,
    int M, int K, int batch) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    int8_t* q = (int8_t*)lds_raw;
    __shared__ float red[kWaves];
    constexpr int RPP = MTH_WAVE / LPR;          // rows per wave
    constexpr int XQ = (64 * LPR * NSEG) / 1024;  // float4 of x per thread (K <= 64*LPR*NSEG)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane % LPR, ro = lane / LPR;
    const int bpr = K >> 2;        // bytes per row
    const int nseg = bpr >> 4;     // 16-byte segments per row
    const int row = (blockIdx.x * kWaves + wave) * RPP + ro;
    const bool rv = row < M;

    // The token's activations are fetched (and reduced) before the weight
    // stream is released: a load issued after other waves' weight loads waits
    // behind them in the CU's in-order memory pipeline.  Weight loads are
    // unconditional (clamped addresses); out-of-row segments get the padding
    // code at use.  packed is not __restrict__, so the loads stay below the
    // first barrier.
    float4 xr[XQ];
    if (FUSED) {
#pragma unroll
        for (int j = 0; j < XQ; ++j) {
            const int k = (tid + j * kWG) * 4;
            xr[j] = ldf4(x + (k < K ? k : 0));
        }
    }
    uint4 w[NSEG];
    auto issue_w = [&]() {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < NSEG; ++s) {
            const int seg = li + LPR * s;
            w[s] = ld_stream(packed + (int64_t)min(row, M - 1) * bpr + (int64_t)min(seg, nseg - 1) * 16);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    for (int t = 0; t < batch; ++t) {
        float inv;
        if (FUSED) {
            const float* xt = x + (int64_t)t * K;
            float m = 0.0f;
#pragma unroll
            for (int j = 0; j < XQ; ++j) {
                const int k = (tid + j * kWG) * 4;
                if (t > 0) xr[j] = ldf4(xt + (k < K ? k : 0));
                if (k >= K) xr[j] = make_float4(0, 0, 0, 0);
                m = fmaxf(m, fmaxf(fmaxf(fabsf(xr[j].x), fabsf(xr[j].y)), fmaxf(fabsf(xr[j].z), fabsf(xr[j].w))));
            }
            m = wave_max(m);
            if (lane == 0) red[wave] = m;
            __syncthreads();
            if (t == 0) issue_w();
            float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
            if (mx < 1e-10f) mx = 1e-10f;
            const float sc = __fdiv_rn(127.0f, mx);
            inv = __fdiv_rn(mx, 127.0f);
#pragma unroll
            for (int j = 0; j < XQ; ++j) {
                const int k = (tid + j * kWG) * 4;
                if (k < K) {
                    const uint32_t b0 = (uint32_t)quant_i8(xr[j].x, sc) & 0xffu, b1 = (uint32_t)quant_i8(xr[j].y, sc) & 0xffu;
                    const uint32_t b2 = (uint32_t)quant_i8(xr[j].z, sc) & 0xffu, b3 = (uint32_t)quant_i8(xr[j].w, sc) & 0xffu;
                    *(uint32_t*)(q + k) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
                }
            }
        } else {
            inv = act_scale[t];
            const int8_t* at = act + (int64_t)t * K;
            for (int k = tid * 16; k < K; k += kWG * 16) *(uint4*)(q + k) = ld16(at + k);
        }
        __syncthreads();
        if (!FUSED && t == 0) issue_w();

        // lane's activations, transposed: A[s][d][j] byte b = a[seg*64 + 16d + 4b + j]
        uint32_t A[NSEG][4][4];
        int asum = 0;
#pragma unroll
        for (int s = 0; s < NSEG; ++s) {
            const int seg = li + LPR * s;
            if (seg < nseg) {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint4 n = *(const uint4*)(q + seg * 64 + 16 * d);
                    const uint32_t N[4] = {n.x, n.y, n.z, n.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        A[s][d][j] = ((N[0] >> (8 * j)) & 0xffu) | (((N[1] >> (8 * j)) & 0xffu) << 8) |
                                     (((N[2] >> (8 * j)) & 0xffu) << 16) | (((N[3] >> (8 * j)) & 0xffu) << 24);
#pragma unroll
                    for (int j = 0; j < 4; ++j) asum = dot4(N[j], 0x01010101u, asum);
                }
            } else {
#pragma unroll
                for (int d = 0; d < 4; ++d)
#pragma unroll
                    for (int j = 0; j < 4; ++j) A[s][d][j] = 0;
            }
        }
        __syncthreads();  // q may be overwritten by the next token

        {
            int acc = 0;
#pragma unroll
            for (int s = 0; s < NSEG; ++s) {
                // segments past the row (and clamped rows) use the padding code
                // 01 (t = 0, u = 1), which meets A = 0: they contribute nothing
                const bool sv = li + LPR * s < nseg;
                const uint32_t pad = 0x55555555u;
                acc = tdot16(sv ? w[s].x : pad, A[s][0], acc);
                acc = tdot16(sv ? w[s].y : pad, A[s][1], acc);
                acc = tdot16(sv ? w[s].z : pad, A[s][2], acc);
                acc = tdot16(sv ? w[s].w : pad, A[s][3], acc);
            }
            acc = group_sum_i<LPR>(acc - asum);
            if (li == 0 && rv) y[(int64_t)t * M + row] = __fmul_rn(__fmul_rn((float)acc, w_scale), inv);
        }
    }
}

// Generic I2_S GEMV: one wave per (row, token); any K % 4 == 0.
template <bool FUSED>
__global__ __launch_bounds__(kWG) void i2s_gemv_generic(
    const uint8_t* __restrict__ packed, float w_scale, const float* __restrict__ x,
    const int8_t* __restrict__ act, const float* __restrict__ act_scale, float* __restrict__ y,
    int64_t M, int64_t K, int64_t batch) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= M) return;
    const uint8_t* w = packed + row * (K / 4);
    for (int64_t t = 0; t < batch; ++t) {
        float sc = 0.0f, inv;
        const float* xt = x + t * K;
        if (FUSED) {
            float m = 0.0f;
            for (int64_t k = lane; k < K; k += 64) m = fmaxf(m, fabsf(xt[k]));
            m = wave_max(m);
            if (m < 1e-10f) m = 1e-10f;
            sc = __fdiv_rn(127.0f, m);
            inv = __fdiv_rn(m, 127.0f);
        } else {
            inv = act_scale[t];
        }
        int acc = 0;
        for (int64_t k = lane; k < K; k += 64) {
            const int code = (w[k >> 2] >> (2 * (k & 3))) & 3;
            const int tv = code == 0 ? -1 : (code == 1 ? 0 : 1);
            const int a = FUSED ? quant_i8(xt[k], sc) : (int)act[t * K + k];
            acc += tv * a;
        }
        acc = group_sum_i<64>(acc);
        if (lane == 0) y[t * M + row] = __fmul_rn(__fmul_rn((float)acc, w_scale), inv);
    }
}

__device__ __forceinline__ int tern(const uint8_t* w, int64_t e) {
    const int code = (w[e >> 2] >> (2 * (e & 3))) & 3;
    return code == 0 ? -1 : (code == 1 ? 0 : 1);
}

// i2s_gemm (src/kernel_i2s.cpp:42-65): float activations, weights shared over
// n (row m at w + m*(K/4)); one wave per (m, n); out[m*N + n].
__global__ __launch_bounds__(kWG) void i2s_gemm_k(const uint8_t* __restrict__ w, const float* __restrict__ a,
                                                  float* __restrict__ o, int64_t M, int64_t N, int64_t K) {
    const int lane = threadIdx.x & 63;
    const int64_t id = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (id >= M * N) return;
    const int64_t m = id / N, n = id % N;
    const uint8_t* wr = w + m * (K / 4);
    const float* ar = a + n * K;
    float s = 0.0f;
    for (int64_t k = lane; k < K; k += 64) {
        const int tv = tern(wr, k);
        s += tv == 0 ? 0.0f : (tv > 0 ? ar[k] : -ar[k]);
    }
    s = group_sum<64>(s);
    if (lane == 0) o[id] = s;
}

// i2s_gemm_vnni (src/kernel_i2s.cpp:201-235): int8 activations; the exact
// integer dot converted to FP32.
__global__ __launch_bounds__(kWG) void i2s_gemm_vnni_k(const uint8_t* __restrict__ w, const int8_t* __restrict__ a,
                                                       float* __restrict__ o, int64_t M, int64_t N, int64_t K) {
    const int lane = threadIdx.x & 63;
    const int64_t id = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (id >= M * N) return;
    const int64_t m = id / N, n = id % N;
    const uint8_t* wr = w + m * (K / 4);
    const int8_t* ar = a + n * K;
    int acc = 0;
    for (int64_t k = lane; k < K; k += 64) acc += tern(wr, k) * (int)ar[k];
    acc = group_sum_i<64>(acc);
    if (lane == 0) o[id] = (float)acc;
}

// Per-(m,n) activation quantisation of src/kernel_tl.cpp:42-52 done in the
// wave: returns scale = 127/max_abs of act row n.
__device__ __forceinline__ float row_scale(const float* __restrict__ ar, int64_t K) {
    float m = 0.0f;
    for (int64_t k = threadIdx.x & 63; k < K; k += 64) m = fmaxf(m, fabsf(ar[k]));
    m = wave_max(m);
    if (m < 1e-10f) m = 1e-10f;
    return __fdiv_rn(127.0f, m);
}

__device__ __forceinline__ int clamp8(int v) { return v < -128 ? -128 : (v > 127 ? 127 : v); }

// tl1_gemm (src/kernel_tl.cpp:33-74): weight row (m,n) at w + ((m*N+n)*K)/4;
// pair i (even, i < K-1) adds LUT entry `code(i)` of the 9-entry pair table:
// 0 -> -a0-a1, 1 -> -a0, 2 -> -a0+a1, 3 -> -a1 (each clamped to int8).
__global__ __launch_bounds__(kWG) void tl1_gemm_k(const uint8_t* __restrict__ w, const float* __restrict__ a,
                                                  float* __restrict__ o, int64_t M, int64_t N, int64_t K) {
    const int lane = threadIdx.x & 63;
    const int64_t id = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (id >= M * N) return;
    const int64_t n = id % N;
    const float* ar = a + n * K;
    const float sc = row_scale(ar, K);
    const uint8_t* wr = w + (id * K) / 4;
    int acc = 0;
    for (int64_t p = lane; p < K / 2; p += 64) {
        const int64_t i = 2 * p;
        if (i >= K - 1) break;
        const int code = (wr[i >> 2] >> (2 * (i & 3))) & 3;
        const int a0 = quant_i8(ar[i], sc), a1 = quant_i8(ar[i + 1], sc);
        const int v = code == 0 ? -a0 - a1 : (code == 1 ? -a0 : (code == 2 ? -a0 + a1 : -a1));
        acc += clamp8(v);
    }
    acc = group_sum_i<64>(acc);
    if (lane == 0) o[id] = __fdiv_rn((float)acc, sc);
}

// tl2_gemm (src/kernel_tl.cpp:109-168) for K % 3 == 0: weight row (m,n) at
// w + (m*N+n)*ceil(K/4); exact sum_k q[k]*t(k); out = (float)total / scale.
__global__ __launch_bounds__(kWG) void tl2_gemm_k(const uint8_t* __restrict__ w, const float* __restrict__ a,
                                                  float* __restrict__ o, int64_t M, int64_t N, int64_t K) {
    const int lane = threadIdx.x & 63;
    const int64_t id = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (id >= M * N) return;
    const int64_t n = id % N;
    const float* ar = a + n * K;
    const float sc = row_scale(ar, K);
    const uint8_t* wr = w + id * ((K * 2 + 7) / 8);
    int acc = 0;
    for (int64_t k = lane; k < K; k += 64) acc += quant_i8(ar[k], sc) * tern(wr, k);
    acc = group_sum_i<64>(acc);
    if (lane == 0) o[id] = __fdiv_rn((float)acc, sc);
}

__global__ __launch_bounds__(kWG) void dequantize_k(const int8_t* __restrict__ src, float* __restrict__ dst,
                                                    int64_t n, float inv) {
    const int64_t i = (int64_t)blockIdx.x * kWG + threadIdx.x;
    if (i < n) dst[i] = __fmul_rn((float)src[i], inv);
}

// Pair / triple LUTs of src/kernel_tl.cpp:13-31 and :88-107; one thread per
// group, entries in (w0, w1[, w2]) row-major order over {-1, 0, 1}.
__global__ __launch_bounds__(kWG) void tl_lut_k(const int8_t* __restrict__ act, int8_t* __restrict__ lut,
                                                int64_t groups, int group) {
    const int64_t g = (int64_t)blockIdx.x * kWG + threadIdx.x;
    if (g >= groups) return;
    const int a0 = act[g * group], a1 = act[g * group + 1], a2 = group == 3 ? act[g * group + 2] : 0;
    const int ntab = group == 3 ? 27 : 9;
    for (int e = 0; e < ntab; ++e) {
        int w0, w1, w2;
        if (group == 3) { w0 = e / 9 - 1; w1 = (e / 3) % 3 - 1; w2 = e % 3 - 1; }
        else { w0 = e / 3 - 1; w1 = e % 3 - 1; w2 = 0; }
        lut[g * ntab + e] = (int8_t)clamp8(a0 * w0 + a1 * w1 + a2 * w2);
    }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ---------------------------------------------------------------------------
// I2_S GEMV for batches of 2..16 on int8 MFMA (v_mfma_i32_16x16x64_i8).
// ---------------------------------------------------------------------------
// y[t][m] = ((float)sum_k t(m,k) * q[t][k] * w_scale) * act_scale[t], the
// sum exact in int32, as src/kernel_i2s.cpp:32-40 per row and token.
// Workgroup = 4 waves x 16 rows and a K slice of whole 256-column
// super-chunks; grid = (ceil(M / 64), S).  Per super-chunk, lane l (row
// r = l % 16, group g = l / 16) loads the 16 code bytes of its row at
// columns 64g .. 64g + 63 and feeds 4 MFMAs; in MFMA j its A operand is the
// u-codes (t + 1, code 3 read as 2) of columns 64g + 16j .. +15 in the byte
// order (col 4i + s at byte i of dword s), and its B operand the activations
// of token r at the same columns in the same order (transposed once per
// workgroup while staging into LDS).  So D = sum (t + 1) q, and the kernel
// subtracts sum q (accumulated while staging) to get sum t q.  With S > 1
// every slice writes its exact integer partial (|sum| < 2^24, exact in
// FP32) and i2s_bt_reduce adds them in order and applies the epilogue.
typedef int i32x4 __attribute__((ext_vector_type(4)));
constexpr int kIbRows = 64, kIbTok = 16;

__device__ __forceinline__ uint32_t byte_t4x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, int s) {
    // byte i of the result = byte s of the i-th input
    return ((a >> (8 * s)) & 0xffu) | (((b >> (8 * s)) & 0xffu) << 8) | (((c >> (8 * s)) & 0xffu) << 16) |
           (((d >> (8 * s)) & 0xffu) << 24);
}

__global__ __launch_bounds__(kWG) void i2s_gemv_bt(const uint8_t* packed, float w_scale, const int8_t* act,
                                                   const float* __restrict__ act_scale, float* __restrict__ y,
                                                   float* __restrict__ partial, int M, int K, int batch) {
    __shared__ __align__(16) uint32_t qs[2][kIbTok * 16 * 4];  // [token][16-col group][4 dwords]
    __shared__ int asum_p[kIbTok][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.x * kIbRows + wave * 16;
    const int nsc = K / 256, S = gridDim.y;
    const int sc0 = (int)((int64_t)blockIdx.y * nsc / S), sc1 = (int)((int64_t)(blockIdx.y + 1) * nsc / S);
    const int bpr = K / 4;
    const uint8_t* wrow = packed + (int64_t)min(m0 + r, M - 1) * bpr + 16 * g;  // clamped rows
    // staging: thread = (token st, 16-column group sg)
    const int st = tid >> 4, sg = tid & 15;
    const bool sv = st < batch;
    const int8_t* arow = act + (int64_t)(sv ? st : 0) * K + 16 * sg;
    uint4 an = sv ? ld16(arow + sc0 * 256) : make_uint4(0, 0, 0, 0);
    uint4 wn = ld_stream(wrow + sc0 * 64);
    int asum = 0;
    i32x4 acc = {0, 0, 0, 0};
    for (int c = sc0; c < sc1; ++c) {
        uint32_t* qb = qs[c & 1];
        {
            const uint32_t a4[4] = {an.x, an.y, an.z, an.w};  // columns 16sg + 4i + s at byte s of a4[i]
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) qb[(st * 16 + sg) * 4 + s2] = byte_t4x4(a4[0], a4[1], a4[2], a4[3], s2);
#pragma unroll
            for (int i = 0; i < 4; ++i) asum = dot4(a4[i], 0x01010101u, asum);
        }
        __syncthreads();
        const uint4 w = wn;
        if (c + 1 < sc1) {
            wn = ld_stream(wrow + (c + 1) * 64);
            if (sv) an = ld16(arow + (c + 1) * 256);
        }
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t u = ucode(wd[j]);
            const i32x4 a = {(int)(u & 0x03030303u), (int)((u >> 2) & 0x03030303u), (int)((u >> 4) & 0x03030303u),
                             (int)((u >> 6) & 0x03030303u)};
            const i32x4 b = *(const i32x4*)(qb + (r * 16 + 4 * g + j) * 4);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
        }
    }
    asum_p[st][sg] = asum;
    __syncthreads();
    // D: lane l holds rows 4g + i for token r
    const int t = r;
    if (t >= batch) return;
    int as = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) as += asum_p[t][j];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * g + i;
        if (m >= M) continue;
        const int v = acc[i] - as;
        if (S == 1)
            y[(int64_t)t * M + m] = __fmul_rn(__fmul_rn((float)v, w_scale), act_scale[t]);
        else
            partial[((int64_t)blockIdx.y * kIbTok + t) * M + m] = (float)v;
    }
}

__global__ __launch_bounds__(kWG) void i2s_bt_reduce(const float* __restrict__ partial, float w_scale,
                                                     const float* __restrict__ act_scale, float* __restrict__ y, int M,
                                                     int batch, int nslice) {
    const int64_t i = (int64_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= (int64_t)batch * M) return;
    const int64_t t = i / M, m = i - t * M;
    const float* p = partial + t * M + m;
    float s = 0.0f;  // integers below 2^24: exact in any order
    for (int z = 0; z < nslice; ++z) s += p[(int64_t)z * kIbTok * M];
    y[i] = __fmul_rn(__fmul_rn(s, w_scale), act_scale[t]);
}

inline int ib_slices(int64_t M, int64_t K) {
    const int64_t groups = (M + kIbRows - 1) / kIbRows, nsc = K / 256;
    int S = 1;
    while (S < 16 && groups * S < 256 && 2 * S <= nsc) S *= 2;
    return S;
}

template <int LPR, int NSEG>
hipError_t run_i2s_fast(const uint8_t* packed, float w_scale, const float* x, const int8_t* act,
                        const float* act_scale, float* y, int64_t M, int64_t K, int64_t batch, hipStream_t s) {
    constexpr int RPP = MTH_WAVE / LPR;
    const int grid = ceil_div(M, RPP * kWaves);
    const size_t lds = (size_t)((K + 15) / 16) * 16;
    if (x)
        i2s_gemv_fast<LPR, NSEG, true><<<grid, kWG, lds, s>>>(packed, w_scale, x, act, act_scale, y, (int)M,
                                                               (int)K, (int)batch);
    else
        i2s_gemv_fast<LPR, NSEG, false><<<grid, kWG, lds, s>>>(packed, w_scale, x, act, act_scale, y, (int)M,
                                                                (int)K, (int)batch);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_quantize_per_token(const float* src, int8_t* dst, float* scale, float* inv_scale,
                                     int64_t rows, int64_t cols, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    quantize_rows<<<(unsigned)rows, kWG, 0, s>>>(src, dst, scale, inv_scale, cols);
    return hipGetLastError();
}

hipError_t launch_dequantize(const int8_t* src, float* dst, int64_t n, float inv_scale, hipStream_t s) {
    dequantize_k<<<ceil_div(n, kWG), kWG, 0, s>>>(src, dst, n, inv_scale);
    return hipGetLastError();
}

hipError_t launch_tl_precompute_lut(const int8_t* act, int8_t* lut, int64_t K, int group, hipStream_t s) {
    const int64_t groups = K / group;
    if (groups == 0) return hipSuccess;
    tl_lut_k<<<ceil_div(groups, kWG), kWG, 0, s>>>(act, lut, groups, group);
    return hipGetLastError();
}

hipError_t launch_i2s_gemv(const uint8_t* packed, float w_scale, const float* x, const int8_t* act,
                           const float* act_scale, float* y, int64_t M, int64_t K, int64_t batch,
                           hipStream_t s) {
    const int64_t nseg = K / 64;
    const bool fast = K % 64 == 0 && nseg <= 256 && M < (1ll << 31) && aligned16(packed) &&
                      (x ? aligned16(x) : aligned16(act));
    if (fast) {
        if (nseg <= 16) return run_i2s_fast<16, 1>(packed, w_scale, x, act, act_scale, y, M, K, batch, s);
        if (nseg <= 32) return run_i2s_fast<16, 2>(packed, w_scale, x, act, act_scale, y, M, K, batch, s);
        if (nseg <= 64) return run_i2s_fast<32, 2>(packed, w_scale, x, act, act_scale, y, M, K, batch, s);
        if (nseg <= 128) return run_i2s_fast<32, 4>(packed, w_scale, x, act, act_scale, y, M, K, batch, s);
        if (nseg <= 192) return run_i2s_fast<64, 3>(packed, w_scale, x, act, act_scale, y, M, K, batch, s);
        return run_i2s_fast<64, 4>(packed, w_scale, x, act, act_scale, y, M, K, batch, s);
    }
    if (x)
        i2s_gemv_generic<true><<<ceil_div(M, kWaves), kWG, 0, s>>>(packed, w_scale, x, act, act_scale, y, M, K, batch);
    else
        i2s_gemv_generic<false><<<ceil_div(M, kWaves), kWG, 0, s>>>(packed, w_scale, x, act, act_scale, y, M, K, batch);
    return hipGetLastError();
}

bool i2s_bt_supported(int64_t M, int64_t K, int64_t batch) {
    return batch >= 2 && K >= 256 && K % 256 == 0 && K < (1 << 24) / 128 && M < (1ll << 31);
}

size_t i2s_bt_partial_bytes(int64_t M, int64_t K) {
    const int S = ib_slices(M, K);
    return S > 1 ? (size_t)(S * kIbTok * M * 4) : 0;
}

hipError_t launch_i2s_gemv_bt(const uint8_t* packed, float w_scale, const int8_t* act, const float* act_scale, float* y,
                              int64_t M, int64_t K, int64_t batch, float* partial, hipStream_t s) {
    const int S = ib_slices(M, K);
    const dim3 grid(ceil_div(M, kIbRows), (unsigned)S);
    for (int64_t t0 = 0; t0 < batch; t0 += kIbTok) {
        const int b = (int)(batch - t0 < kIbTok ? batch - t0 : kIbTok);
        i2s_gemv_bt<<<grid, kWG, 0, s>>>(packed, w_scale, act + t0 * K, act_scale + t0, y + t0 * M, partial, (int)M,
                                         (int)K, b);
        if (S > 1)
            i2s_bt_reduce<<<ceil_div((int64_t)b * M, kWG), kWG, 0, s>>>(partial, w_scale, act_scale + t0, y + t0 * M,
                                                                        (int)M, b, S);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_i2s_gemm(const uint8_t* w, const float* a, float* o, int64_t M, int64_t N, int64_t K,
                           hipStream_t s) {
    i2s_gemm_k<<<ceil_div(M * N, kWaves), kWG, 0, s>>>(w, a, o, M, N, K);
    return hipGetLastError();
}

hipError_t launch_i2s_gemm_vnni(const uint8_t* w, const int8_t* a, float* o, int64_t M, int64_t N, int64_t K,
                                hipStream_t s) {
    i2s_gemm_vnni_k<<<ceil_div(M * N, kWaves), kWG, 0, s>>>(w, a, o, M, N, K);
    return hipGetLastError();
}

hipError_t launch_tl1_gemm(const uint8_t* w, const float* a, float* o, int64_t M, int64_t N, int64_t K,
                           hipStream_t s) {
    tl1_gemm_k<<<ceil_div(M * N, kWaves), kWG, 0, s>>>(w, a, o, M, N, K);
    return hipGetLastError();
}

hipError_t launch_tl2_gemm(const uint8_t* w, const float* a, float* o, int64_t M, int64_t N, int64_t K,
                           hipStream_t s) {
    tl2_gemm_k<<<ceil_div(M * N, kWaves), kWG, 0, s>>>(w, a, o, M, N, K);
    return hipGetLastError();
}

}  // namespace mth
