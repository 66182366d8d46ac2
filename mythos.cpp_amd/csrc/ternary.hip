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
#include <algorithm>

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
    int M, int K, int batch, ResidOut res) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    int8_t* q = (int8_t*)lds_raw;
    __shared__ float red[kWaves];
    __shared__ double rsq[kWaves];
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
            const float v = fmul_rn(fmul_rn((float)acc, w_scale), inv);
            const int64_t i = (int64_t)t * M + row;
            if (!res.x) {
                if (li == 0 && rv) y[i] = v;
            } else {
                // residual epilogue (ResidOut, common.h): rows of this workgroup
                double sq = 0.0;
                if (li == 0 && rv) {
                    const float r = v + res.x[i];
                    res.x[i] = r;
                    res.xg[i] = r * res.gamma[row];
                    sq = (double)r * r;
                }
                sq = wave_sum_dbl(sq);
                if (lane == 0) rsq[wave] = sq;
                __syncthreads();
                if (tid == 0) res.ssp[(int64_t)t * gridDim.x + blockIdx.x] = ((rsq[0] + rsq[1]) + rsq[2]) + rsq[3];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// SwiGLU + per-token int8 quantisation fused into the I2_S down projection
// (decode batch 1).
// ---------------------------------------------------------------------------
//   a = silu(g * ni) * (u * ni)              (ni: the RMSNorm's 1 / rms, NormScale)
//   q = quantize_per_token(a)                (src/int8_quant.cpp:8-31)
//   y[m] = ((float)sum_k t(m, k) q[k] * w_scale) * (max|a| / 127)
// Every workgroup (16 waves, one row per wave: 16 rows) first computes the
// whole token's a exactly as silu_mul_quant_k does -- 1024 threads with the
// same columns per thread, the same NormScale summation order, the same max
// and rounding -- and keeps q in LDS; then each wave runs the i2s_gemv_fast
// dot product of its row (64 lanes, NSEG 16-byte segments per lane).  The
// SwiGLU is recomputed by every workgroup (one per CU at hidden 4096), which
// costs less than the launch and the int8 round trip it replaces.
// Loads in order of use: the norm's partial sums, g and u, then the row's
// weights (the CU returns loads in issue order).
// res (ResidOut): the residual epilogue of i2s_gemv_fast; its partial sums go
// to res.ssp, which must not be ns.ssp (other workgroups may still read it).
constexpr int kSwT = 1024, kSwQ = 12;  // as silu_mul_quant_k (kSQT, kSQ)

template <int NSEG>
__global__ __launch_bounds__(kSwT) void i2s_swiglu_k(const float* __restrict__ g, const float* __restrict__ u,
                                                     NormScale ns, const uint8_t* packed, float w_scale,
                                                     float* __restrict__ y, int M, int K, ResidOut res) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    int8_t* q = (int8_t*)lds_raw;  // K bytes
    __shared__ double nred[kSwT / 64];
    __shared__ float red[kSwT / 64];
    __shared__ double rsq[kSwT / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = blockIdx.x * (kSwT / 64) + wave;
    const int bpr = K >> 2, nseg = bpr >> 4;

    double npart[kNormBatch];
    if (ns.ssp) norm_issue(ns, 0, tid, kSwT, npart);
    float gv[kSwQ], uv[kSwQ];
#pragma unroll
    for (int j = 0; j < kSwQ; ++j) {
        const int i = tid + j * kSwT;
        gv[j] = i < K ? g[i] : 0.0f;
        uv[j] = i < K ? u[i] : 0.0f;
    }
    uint4 w[NSEG];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < NSEG; ++s)
        w[s] = ld_stream(packed + (int64_t)min(row, M - 1) * bpr + (int64_t)min(lane + 64 * s, nseg - 1) * 16);
    __builtin_amdgcn_sched_barrier(0);

    if (ns.ssp) {  // norm_scale<16>: per-thread sums, wave sums, waves in order
        double sum = wave_sum_dbl(norm_finish(ns, 0, tid, kSwT, npart));
        if (lane == 0) nred[wave] = sum;
        __syncthreads();
        sum = 0.0;
#pragma unroll
        for (int w2 = 0; w2 < kSwT / 64; ++w2) sum += nred[w2];
        const float ni = (float)(1.0 / sqrt(sum / (double)ns.dim + (double)ns.eps));
#pragma unroll
        for (int j = 0; j < kSwQ; ++j) {
            gv[j] *= ni;
            uv[j] *= ni;
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < kSwQ; ++j) {
        gv[j] = silu1(gv[j]) * uv[j];
        m = fmaxf(m, fabsf(gv[j]));
    }
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w2 = 1; w2 < kSwT / 64; ++w2) m = fmaxf(m, red[w2]);
    if (m < 1e-10f) m = 1e-10f;
    const float sc = __fdiv_rn(127.0f, m), inv = __fdiv_rn(m, 127.0f);
    // q is stored transposed within each 16-column group (column 4b + j of a
    // group at byte 4j + b), the operand order of tdot16, so a row's operands
    // are plain 16-byte reads
#pragma unroll
    for (int j = 0; j < kSwQ; ++j) {
        const int i = tid + j * kSwT;
        if (i < K) q[(i & ~15) | ((i & 3) << 2) | ((i >> 2) & 3)] = (int8_t)quant_i8(gv[j], sc);
    }
    __syncthreads();

    // lane's activations: A[s][d][j] byte b = a[seg*64 + 16d + 4b + j]
    uint32_t A[NSEG][4][4];
    int asum = 0;
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
        const int seg = lane + 64 * s;
        if (seg < nseg) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint4 n = *(const uint4*)(q + seg * 64 + 16 * d);
                A[s][d][0] = n.x, A[s][d][1] = n.y, A[s][d][2] = n.z, A[s][d][3] = n.w;
#pragma unroll
                for (int j = 0; j < 4; ++j) asum = dot4(A[s][d][j], 0x01010101u, asum);
            }
        } else {
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int j = 0; j < 4; ++j) A[s][d][j] = 0;
        }
    }
    int acc = 0;
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
        const bool sv = lane + 64 * s < nseg;
        const uint32_t pad = 0x55555555u;  // t = 0 codes past the row (they meet A = 0)
        acc = tdot16(sv ? w[s].x : pad, A[s][0], acc);
        acc = tdot16(sv ? w[s].y : pad, A[s][1], acc);
        acc = tdot16(sv ? w[s].z : pad, A[s][2], acc);
        acc = tdot16(sv ? w[s].w : pad, A[s][3], acc);
    }
    acc = group_sum_i<64>(acc - asum);
    const float v = fmul_rn(fmul_rn((float)acc, w_scale), inv);
    const bool rv = row < M;
    if (!res.x) {
        if (lane == 0 && rv) y[row] = v;
        return;
    }
    double sq = 0.0;
    if (lane == 0 && rv) {
        const float r = v + res.x[row];
        res.x[row] = r;
        res.xg[row] = r * res.gamma[row];
        sq = (double)r * r;
    }
    if (lane == 0) rsq[wave] = sq;
    __syncthreads();
    if (tid == 0) {
        double t = 0.0;
#pragma unroll
        for (int w2 = 0; w2 < kSwT / 64; ++w2) t += rsq[w2];
        res.ssp[blockIdx.x] = t;
    }
}

// ---------------------------------------------------------------------------
// I2_S down projection from a SwiGLU output computed elsewhere (decode batch 1)
// ---------------------------------------------------------------------------
// act = a (K floats) and amax = the maxima of |a| over groups of 8 columns
// (K / 8 of them, oil4_gemv_v2's SwiGLU epilogue): max|a| is the maximum of
// the maxima, q = quantize_per_token(a) (src/int8_quant.cpp:8-31) and
// y[m] = ((float)sum_k t(m, k) q[k] * w_scale) * (max|a| / 127), the values
// i2s_swiglu_k computes.  Workgroup = 8 waves, two rows per wave (16 rows):
// every wave holds the whole token's int8 operands in registers, so two rows
// per wave halve the LDS reads and the activation sums per row (16 waves of
// one row measured 8.0 us at 4096 x 11008, 8 waves of two 6.4 us, 4 of four
// 6.8 us).  Loads in order of use: maxima, activations (float4), the rows'
// weights.  The residual epilogue sums the 16 rows' squares in row order,
// as i2s_swiglu_k does.
constexpr int kIaR = 2, kIaT = 1024 / kIaR;

template <int NSEG>
__global__ __launch_bounds__(kIaT) void i2s_act_k(const float* __restrict__ act, const float* __restrict__ amax,
                                                  const uint8_t* packed, float w_scale, float* __restrict__ y, int M,
                                                  int K, ResidOut res) {
    constexpr int R = kIaR, T = kIaT, NW = T / 64;
    constexpr int NM = (kSwT * kSwQ / 8 + T - 1) / T, NA = (kSwT * kSwQ / 4 + T - 1) / T;  // K <= kSwT * kSwQ
    extern __shared__ __align__(16) uint8_t lds_raw[];
    int8_t* q = (int8_t*)lds_raw;  // K bytes
    __shared__ float red[NW];
    __shared__ double rsq[NW * R];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.x * (NW * R) + wave * R;
    const int bpr = K >> 2, nseg = bpr >> 4, nm = K >> 3, n4 = K >> 2;
    float mp[NM];
#pragma unroll
    for (int j = 0; j < NM; ++j) mp[j] = amax[min(tid + j * T, nm - 1)];
    float4 av[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j) av[j] = ((const float4*)act)[min(tid + j * T, n4 - 1)];
    // residual epilogue operands (lane r < R: row row0 + r), issued before the weights (clamped, unconditional)
    const int rrow = min(row0 + (lane % R), M - 1);
    const float rx0 = (res.x ? res.x : act)[res.x ? rrow : 0], rg0 = (res.x ? res.gamma : act)[res.x ? rrow : 0];
    uint4 w[R][NSEG];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int s = 0; s < NSEG; ++s)
            w[r][s] = ld_stream(packed + (int64_t)min(row0 + r, M - 1) * bpr +
                                (int64_t)min(lane + 64 * s, nseg - 1) * 16);
    __builtin_amdgcn_sched_barrier(0);

    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NM; ++j)
        if (tid + j * T < nm) m = fmaxf(m, mp[j]);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) m = fmaxf(m, red[w2]);
    if (m < 1e-10f) m = 1e-10f;
    const float sc = __fdiv_rn(127.0f, m), inv = __fdiv_rn(m, 127.0f);
    // q transposed within each 16-column group (column 4b + j at byte 4j + b), the operand order of tdot16
#pragma unroll
    for (int j = 0; j < NA; ++j) {
        const int i4 = tid + j * T;
        if (i4 < n4) {
            const float vv[4] = {av[j].x, av[j].y, av[j].z, av[j].w};
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int i = 4 * i4 + b;
                q[(i & ~15) | ((i & 3) << 2) | ((i >> 2) & 3)] = (int8_t)quant_i8(vv[b], sc);
            }
        }
    }
    __syncthreads();

    // lane's activations: A[s][d][j] byte b = a[seg*64 + 16d + 4b + j]
    uint32_t A[NSEG][4][4];
    int asum = 0;
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
        const int seg = lane + 64 * s;
        if (seg < nseg) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint4 n = *(const uint4*)(q + seg * 64 + 16 * d);
                A[s][d][0] = n.x, A[s][d][1] = n.y, A[s][d][2] = n.z, A[s][d][3] = n.w;
#pragma unroll
                for (int j = 0; j < 4; ++j) asum = dot4(A[s][d][j], 0x01010101u, asum);
            }
        } else {
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int j = 0; j < 4; ++j) A[s][d][j] = 0;
        }
    }
    float vr = 0.0f;  // lane r: row row0 + r
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int acc = 0;
#pragma unroll
        for (int s = 0; s < NSEG; ++s) {
            const bool sv = lane + 64 * s < nseg;
            const uint32_t pad = 0x55555555u;  // t = 0 codes past the row (they meet A = 0)
            acc = tdot16(sv ? w[r][s].x : pad, A[s][0], acc);
            acc = tdot16(sv ? w[r][s].y : pad, A[s][1], acc);
            acc = tdot16(sv ? w[r][s].z : pad, A[s][2], acc);
            acc = tdot16(sv ? w[r][s].w : pad, A[s][3], acc);
        }
        acc = group_sum_i<64>(acc - asum);
        const float v = fmul_rn(fmul_rn((float)acc, w_scale), inv);
        if (lane == r) vr = v;
    }
    const int row = row0 + lane;
    if (!res.x) {
        if (lane < R && row < M) y[row] = vr;
        return;
    }
    if (lane < R) {
        double sq = 0.0;
        if (row < M) {
            const float r = vr + rx0;
            res.x[row] = r;
            res.xg[row] = r * rg0;
            sq = (double)r * r;
        }
        rsq[wave * R + lane] = sq;
    }
    __syncthreads();
    if (tid == 0) {
        double t = 0.0;
#pragma unroll
        for (int i = 0; i < NW * R; ++i) t += rsq[i];
        res.ssp[blockIdx.x] = t;
    }
}

// ---------------------------------------------------------------------------
// I2_S GEMV, batch 1 (i2s_gemv_rows): R rows per wave, 4R per workgroup.
// ---------------------------------------------------------------------------
// A 4 MB GEMV is latency-bound, so everything is requested up front: the
// activations first, then every weight segment of the workgroup's rows (NSEG
// 128-bit loads per row and lane), and only then the absmax reduction and the
// quantisation run while the weights stream in.  Lane l owns 16-byte segments
// l + 64 s of every row (64 weights each) and its 64 activations per segment
// (byte-transposed from LDS, as in i2s_gemv_fast); the R row sums are reduced
// across the wave by a transposed butterfly.  K % 64 == 0, K <= 4096 NSEG,
// K <= 1024 XQ (FUSED).  Dynamic LDS: K bytes.
template <int R>
__device__ __forceinline__ int transposed_sum_i(int (&v)[R], int lane) { return transposed_reduce<R>(v, lane); }

template <int R, int NSEG, int XQ, bool FUSED>
__global__ __launch_bounds__(kWG) void i2s_gemv_rows(const uint8_t* packed, float w_scale,
                                                     const float* __restrict__ x, const int8_t* act,
                                                     const float* __restrict__ act_scale, float* __restrict__ y,
                                                     int M, int K) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    int8_t* q = (int8_t*)lds_raw;
    __shared__ float red[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bpr = K >> 2, nseg = bpr >> 4;
    const int row0 = (blockIdx.x * kWaves + wave) * R;

    float4 xr[XQ];
    if (FUSED) {
#pragma unroll
        for (int j = 0; j < XQ; ++j) {
            const int k = (tid + j * kWG) * 4;
            xr[j] = ldf4(x + (k < K ? k : 0));
        }
    }
    uint4 w[R][NSEG];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int s = 0; s < NSEG; ++s)
            w[r][s] = ld_stream(packed + (int64_t)min(row0 + r, M - 1) * bpr + (int64_t)min(lane + 64 * s, nseg - 1) * 16);

    float inv;
    if (FUSED) {
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < XQ; ++j) {
            const int k = (tid + j * kWG) * 4;
            if (k >= K) xr[j] = make_float4(0, 0, 0, 0);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(xr[j].x), fabsf(xr[j].y)), fmaxf(fabsf(xr[j].z), fabsf(xr[j].w))));
        }
        m = wave_max(m);
        if (lane == 0) red[wave] = m;
        __syncthreads();
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
        inv = act_scale[0];
        for (int k = tid * 16; k < K; k += kWG * 16) *(uint4*)(q + k) = ld16(act + k);
    }
    __syncthreads();

    uint32_t A[NSEG][4][4];
    int asum = 0;
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
        const int seg = lane + 64 * s;
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
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int a = 0;
#pragma unroll
        for (int s = 0; s < NSEG; ++s) {
            const bool sv = lane + 64 * s < nseg;
            const uint32_t pad = 0x55555555u;  // t = 0 codes for segments past the row
            a = tdot16(sv ? w[r][s].x : pad, A[s][0], a);
            a = tdot16(sv ? w[r][s].y : pad, A[s][1], a);
            a = tdot16(sv ? w[r][s].z : pad, A[s][2], a);
            a = tdot16(sv ? w[r][s].w : pad, A[s][3], a);
        }
        acc[r] = a - asum;
    }
    const int tot = transposed_sum_i<R>(acc, lane);
    constexpr int Lr = MTH_WAVE / R;
    const int row = row0 + lane / Lr;
    if ((lane % Lr) == 0 && row < M) y[row] = fmul_rn(fmul_rn((float)tot, w_scale), inv);
}

// I2_S GEMV, batch 1, K = 4096 exactly (i2s_gemv_k4096): i2s_gemv_rows with
// every lane holding one full 16-byte segment of each of its 4 rows and no
// bounds guard at all (the guarded kernel measured ~10% slower at this
// shape: its branches changed the compiler's wait placement).  Same loads in
// the same order, same quantisation and the same integer products, so the
// outputs are those of i2s_gemv_rows bit for bit.  Dynamic LDS: 4096 bytes.
constexpr int kK4096 = 4096;
__global__ __launch_bounds__(kWG) void i2s_gemv_k4096(const uint8_t* packed, float w_scale,
                                                      const float* __restrict__ x, float* __restrict__ y, int M) {
    constexpr int R = 4, XQ = kK4096 / (4 * kWG), bpr = kK4096 / 4;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    int8_t* q = (int8_t*)lds_raw;
    __shared__ float red[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = (blockIdx.x * kWaves + wave) * R;
    float4 xr[XQ];
#pragma unroll
    for (int j = 0; j < XQ; ++j) xr[j] = ldf4(x + (tid + j * kWG) * 4);
    uint4 w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) w[r] = ld_stream(packed + (int64_t)min(row0 + r, M - 1) * bpr + (int64_t)lane * 16);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < XQ; ++j)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xr[j].x), fabsf(xr[j].y)), fmaxf(fabsf(xr[j].z), fabsf(xr[j].w))));
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    float mx = red[0];
#pragma unroll
    for (int w2 = 1; w2 < kWaves; ++w2) mx = fmaxf(mx, red[w2]);
    if (mx < 1e-10f) mx = 1e-10f;
    const float sc = __fdiv_rn(127.0f, mx), inv = __fdiv_rn(mx, 127.0f);
#pragma unroll
    for (int j = 0; j < XQ; ++j) {
        const uint32_t b0 = (uint32_t)quant_i8(xr[j].x, sc) & 0xffu, b1 = (uint32_t)quant_i8(xr[j].y, sc) & 0xffu;
        const uint32_t b2 = (uint32_t)quant_i8(xr[j].z, sc) & 0xffu, b3 = (uint32_t)quant_i8(xr[j].w, sc) & 0xffu;
        *(uint32_t*)(q + (tid + j * kWG) * 4) = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
    __syncthreads();
    // lane's activations: A[d][j] byte b = a[lane*64 + 16d + 4b + j]
    uint32_t A[4][4];
    int asum = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint4 n = *(const uint4*)(q + lane * 64 + 16 * d);
        const uint32_t N[4] = {n.x, n.y, n.z, n.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            A[d][j] = ((N[0] >> (8 * j)) & 0xffu) | (((N[1] >> (8 * j)) & 0xffu) << 8) |
                      (((N[2] >> (8 * j)) & 0xffu) << 16) | (((N[3] >> (8 * j)) & 0xffu) << 24);
#pragma unroll
        for (int j = 0; j < 4; ++j) asum = dot4(N[j], 0x01010101u, asum);
    }
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int a = 0;
        a = tdot16(w[r].x, A[0], a);
        a = tdot16(w[r].y, A[1], a);
        a = tdot16(w[r].z, A[2], a);
        a = tdot16(w[r].w, A[3], a);
        acc[r] = a - asum;
    }
    const int tot = transposed_sum_i<R>(acc, lane);
    constexpr int Lr = MTH_WAVE / R;
    const int row = row0 + lane / Lr;
    if ((lane % Lr) == 0 && row < M) y[row] = fmul_rn(fmul_rn((float)tot, w_scale), inv);
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
        if (lane == 0) y[t * M + row] = fmul_rn(fmul_rn((float)acc, w_scale), inv);
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

// The same sums when every weight row is whole 16-byte segments (ceil(K/4)
// % 16 == 0, 16-byte aligned w).  The tl2_gemm codes are the I2_S codes (2
// bits per weight, weight i at bits 2(i % 4) of byte i / 4, decode_tl2
// :81-86: 00 -> -1, 01 -> 0, 1x -> +1), so the sum is the I2_S kernels'
// sum_k u q - sum_k q on v_dot4 (u = t + 1).  tl2_quant_k quantises each
// activation row once (the reference's per-row loop :118-129 is
// quantize_per_token's arithmetic: absmax with the 1e-10 floor, 127/max,
// round half away) straight into the operand order: byte-transposed per 16
// columns (column 4b + j at byte 4j + b) and zero-padded to whole 64-column
// segments, so codes past K meet q = 0.  tl2_rows_k: wave = R rows (m, n)
// of one activation row n; lane l takes segments l, l + 64, ... of its R
// rows (16 code bytes each) and the segment's 64 q bytes, loaded once for
// the R rows.  No weight is shared between outputs (every (m, n) has its
// own row in the reference's layout), so this is a streaming kernel.
__global__ __launch_bounds__(kWG) void tl2_quant_k(const float* __restrict__ a, int8_t* __restrict__ qt,
                                                   float* __restrict__ qscale, int K, int stride) {
    __shared__ float red[kWaves];
    const int64_t n = blockIdx.x;
    const float* x = a + n * K;
    const float sc = __fdiv_rn(127.0f, block_absmax(x, K, red));
    int8_t* dst = qt + n * stride;
    for (int i = threadIdx.x; i < stride; i += kWG)
        dst[(i & ~15) | ((i & 3) << 2) | ((i >> 2) & 3)] = i < K ? (int8_t)quant_i8(x[i], sc) : (int8_t)0;
    if (threadIdx.x == 0) qscale[n] = sc;
}

template <int R>
__global__ __launch_bounds__(kWG) void tl2_rows_k(const uint8_t* __restrict__ w, const int8_t* __restrict__ qt,
                                                  const float* __restrict__ qscale, float* __restrict__ o,
                                                  int64_t M, int64_t N, int bpr) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t n = blockIdx.y, m0 = ((int64_t)blockIdx.x * kWaves + wave) * R;
    if (m0 >= M) return;  // uniform per wave, no barrier in this kernel
    const int nseg = bpr / 16;
    const int8_t* qn = qt + n * (int64_t)nseg * 64;
    int acc[R], asum = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0;
    for (int seg = lane; seg < nseg; seg += 64) {
        uint4 wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t m = min(m0 + r, M - 1);
            wv[r] = ld_stream(w + (m * N + n) * bpr + (int64_t)seg * 16);
        }
        uint32_t A[4][4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint4 v = *(const uint4*)(qn + seg * 64 + 16 * d);
            A[d][0] = v.x, A[d][1] = v.y, A[d][2] = v.z, A[d][3] = v.w;
#pragma unroll
            for (int j = 0; j < 4; ++j) asum = dot4(A[d][j], 0x01010101u, asum);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = tdot16(wv[r].x, A[0], acc[r]);
            acc[r] = tdot16(wv[r].y, A[1], acc[r]);
            acc[r] = tdot16(wv[r].z, A[2], acc[r]);
            acc[r] = tdot16(wv[r].w, A[3], acc[r]);
        }
    }
    asum = group_sum_i<64>(asum);
    const float sc = qscale[n];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int tot = group_sum_i<64>(acc[r]) - asum;
        if (lane == 0 && m0 + r < M) o[(m0 + r) * N + n] = __fdiv_rn((float)tot, sc);
    }
}

__global__ __launch_bounds__(kWG) void dequantize_k(const int8_t* __restrict__ src, float* __restrict__ dst,
                                                    int64_t n, float inv) {
    const int64_t i = (int64_t)blockIdx.x * kWG + threadIdx.x;
    if (i < n) dst[i] = fmul_rn((float)src[i], inv);
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
// Workgroup = WV waves x 16 rows and a K slice of whole 256-column chunks;
// grid = (ceil(M / (16 WV)), S).  Per chunk, lane l (row r = l % 16, group
// g = l / 16) holds the 16 code bytes of its row at columns 64g .. 64g + 63
// and feeds 4 MFMAs; in MFMA j its A operand is the u-codes (t + 1, code 3
// read as 2) of columns 64g + 16j .. +15 in the byte order (col 4i + s at
// byte i of dword s), and its B operand the activations of token r at the
// same columns in the same order (transposed while staging into LDS).  So
// D = sum (t + 1) q, and the kernel subtracts sum q (accumulated while
// staging) to get sum t q.
// Loads: the CU returns loads in issue order across its waves, so every
// wave first issues the slice's activations (up to MAXC chunks: thread =
// token, 16-column group), then, after a barrier, all its weight loads of
// the slice; the activations are staged once and the chunk loop has no
// barrier.  Slices longer than MAXC chunks run in rounds.  With S > 1 every
// slice writes its exact integer partial (|sum| < 2^24, exact in FP32) and
// i2s_bt_reduce (or the consumer, as Slices) adds them in order and applies
// the epilogue.
typedef int i32x4 __attribute__((ext_vector_type(4)));
constexpr int kIbWaves = 8, kIbRows = 16 * kIbWaves, kIbTok = 16, kIbChunks = 8, kIbTokStride = 68;

__device__ __forceinline__ uint32_t byte_t4x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, int s) {
    // byte i of the result = byte s of the i-th input
    return ((a >> (8 * s)) & 0xffu) | (((b >> (8 * s)) & 0xffu) << 8) | (((c >> (8 * s)) & 0xffu) << 16) |
           (((d >> (8 * s)) & 0xffu) << 24);
}

// FP32 activations (the decode step of a batch, FA): act[t * lda + k] =
// silu(g * ni) * (u * ni) with amax[t][nmx] the maxima of |act| over blocks
// of it (oil4_gemv_bt_swiglu); the kernel quantises per token as
// quantize_per_token (src/int8_quant.cpp:8-31) -- max |act| (the maximum of
// the block maxima, floor 1e-10), q = round(act * (127 / max)) -- while
// staging, and workgroup (0, 0) writes inv[t] = max / 127 (the consumer's
// act scale).  nmx <= 16 kIbFaMx.
struct I2sF32Act {
    const float* act;  // row stride lda
    int64_t lda;
    const float* amax;
    int nmx;
    float* inv;
};
constexpr int kIbFaMx = 4, kIbFaChunks = 4;  // FA: block maxima per thread, chunks per round

// One round of NC chunks (NC is the exact count, so every load below is
// unconditional straight-line code and the waits before the staging and the
// MFMAs count only what they need).  FA: the activations are FP32 (arowf)
// and quantised with the token's scale sc while staging; in the first round
// sc is derived from the block maxima mxv (loaded at the kernel's start)
// after the weights are issued.
template <int NC, bool FA = false>
__device__ __forceinline__ void ib_round(const uint8_t* wrow, const int8_t* arow, bool sv, bool stager, int c0,
                                         bool first, uint32_t (*qs)[kIbTok * kIbTokStride], int st, int sg, int r,
                                         int g, int& asum, i32x4& acc, const float* arowf = nullptr,
                                         float* sc = nullptr, const float* mxv = nullptr,
                                         const I2sF32Act* fa = nullptr, float* tinv = nullptr) {
    uint4 an[FA ? 1 : NC], wv[NC];
    float4 af[FA ? NC : 1][4];
    if (stager) {
        if constexpr (FA) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) af[c][e] = ldf4(arowf + (int64_t)(c0 + c) * 256 + 4 * e);
        } else {
#pragma unroll
            for (int c = 0; c < NC; ++c) an[c] = ld16(arow + (int64_t)(c0 + c) * 256);  // a clamped row if !sv
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();  // every wave's activations are issued before any weights
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < NC; ++c) wv[c] = ld_stream(wrow + (int64_t)(c0 + c) * 64);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (FA) {
        if (first && stager) {  // the token's scale: 16 threads (sg) per token
            float m = 0.0f;
#pragma unroll
            for (int k = 0; k < kIbFaMx; ++k)
                if (sg + 16 * k < fa->nmx) m = fmaxf(m, mxv[k]);
            m = group_reduce<16>(m, MaxOp{});
            if (m < 1e-10f) m = 1e-10f;
            *sc = __fdiv_rn(127.0f, m);
            const float inv = __fdiv_rn(m, 127.0f);
            if (sg == 0) {
                tinv[st] = inv;
                if (blockIdx.x == 0 && blockIdx.y == 0 && sv) fa->inv[st] = inv;
            }
        }
    }
    if (!first) __syncthreads();  // the previous round's chunks have been read
    if (stager) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            uint32_t a4[4];
            if constexpr (FA) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 v = af[c][i];
                    a4[i] = sv ? ((uint32_t)quant_i8(v.x, *sc) & 0xffu) | (((uint32_t)quant_i8(v.y, *sc) & 0xffu) << 8) |
                                     (((uint32_t)quant_i8(v.z, *sc) & 0xffu) << 16) |
                                     (((uint32_t)quant_i8(v.w, *sc) & 0xffu) << 24)
                               : 0u;
                }
            } else {
                a4[0] = sv ? an[c].x : 0u, a4[1] = sv ? an[c].y : 0u, a4[2] = sv ? an[c].z : 0u;
                a4[3] = sv ? an[c].w : 0u;
            }
            // col 16sg + 4i + s at byte s of a4[i]
            uint4 o;
            o.x = byte_t4x4(a4[0], a4[1], a4[2], a4[3], 0);
            o.y = byte_t4x4(a4[0], a4[1], a4[2], a4[3], 1);
            o.z = byte_t4x4(a4[0], a4[1], a4[2], a4[3], 2);
            o.w = byte_t4x4(a4[0], a4[1], a4[2], a4[3], 3);
            *(uint4*)&qs[c][st * kIbTokStride + sg * 4] = o;
#pragma unroll
            for (int i = 0; i < 4; ++i) asum = dot4(a4[i], 0x01010101u, asum);
        }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const uint32_t wd[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t u = ucode(wd[j]);
            const i32x4 a = {(int)(u & 0x03030303u), (int)((u >> 2) & 0x03030303u), (int)((u >> 4) & 0x03030303u),
                             (int)((u >> 6) & 0x03030303u)};
            const i32x4 b = *(const i32x4*)(&qs[c][r * kIbTokStride + (4 * g + j) * 4]);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
        }
    }
}

template <int MAXC, int WV, bool FA = false>
__global__ __launch_bounds__(WV * 64) void i2s_gemv_bt(const uint8_t* packed, float w_scale, const int8_t* act,
                                                       const float* __restrict__ act_scale, float* __restrict__ y,
                                                       float* __restrict__ partial, int M, int K, int batch,
                                                       I2sF32Act fa = I2sF32Act{}) {
    static_assert(MAXC >= 1 && MAXC <= 8, "ib_round is dispatched for 1..8 chunks");
    // [chunk][token][16-col group][4 dwords], token stride kIbTokStride (64 + 4 dwords: the 16 tokens of an
    // MFMA operand read land on distinct banks)
    __shared__ __align__(16) uint32_t qs[MAXC][kIbTok * kIbTokStride];
    __shared__ int asum_p[kIbTok][16];
    __shared__ float tinv[kIbTok];  // FA: max / 127 per token
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.x * (WV * 16) + wave * 16;
    const int nsc = K / 256, S = gridDim.y;
    const int sc0 = (int)((int64_t)blockIdx.y * nsc / S), sc1 = (int)((int64_t)(blockIdx.y + 1) * nsc / S);
    const int bpr = K / 4;
    const uint8_t* wrow = packed + (int64_t)min(m0 + r, M - 1) * bpr + 16 * g;  // clamped rows
    // staging by the first 4 waves: thread = token st, 16-column group sg
    const int st = (tid >> 4) & 15, sg = tid & 15;
    const bool stager = __builtin_amdgcn_readfirstlane(wave) < 4;
    const bool sv = st < batch;
    const int8_t* arow = act + (int64_t)(sv ? st : 0) * K + 16 * sg;
    // FA: the token's block maxima first (16 threads per token, clamped)
    const float* arowf = FA ? fa.act + (int64_t)(sv ? st : 0) * fa.lda + 16 * sg : nullptr;
    float mxv[kIbFaMx], sc = 0.0f;
    if (FA && stager) {
        const float* am = fa.amax + (int64_t)(sv ? st : 0) * fa.nmx;
#pragma unroll
        for (int k = 0; k < kIbFaMx; ++k) mxv[k] = am[min(sg + 16 * k, fa.nmx - 1)];
    }
    int asum = 0;
    i32x4 acc = {0, 0, 0, 0};
    for (int c0 = sc0; c0 < sc1; c0 += MAXC) {
        const int nc = min(MAXC, sc1 - c0);
        const bool first = c0 == sc0;
        switch (nc) {
            case 1: ib_round<1, FA>(wrow, arow, sv, stager, c0, first, qs, st, sg, r, g, asum, acc, arowf, &sc, mxv, &fa, tinv); break;
            case 2: ib_round<2, FA>(wrow, arow, sv, stager, c0, first, qs, st, sg, r, g, asum, acc, arowf, &sc, mxv, &fa, tinv); break;
            case 3: ib_round<3, FA>(wrow, arow, sv, stager, c0, first, qs, st, sg, r, g, asum, acc, arowf, &sc, mxv, &fa, tinv); break;
            case 4: ib_round<4, FA>(wrow, arow, sv, stager, c0, first, qs, st, sg, r, g, asum, acc, arowf, &sc, mxv, &fa, tinv); break;
            case 5: ib_round<5 <= MAXC ? 5 : 1, FA>(wrow, arow, sv, stager, c0, first, qs, st, sg, r, g, asum, acc, arowf, &sc, mxv, &fa, tinv); break;
            case 6: ib_round<6 <= MAXC ? 6 : 1, FA>(wrow, arow, sv, stager, c0, first, qs, st, sg, r, g, asum, acc, arowf, &sc, mxv, &fa, tinv); break;
            case 7: ib_round<7 <= MAXC ? 7 : 1, FA>(wrow, arow, sv, stager, c0, first, qs, st, sg, r, g, asum, acc, arowf, &sc, mxv, &fa, tinv); break;
            default: ib_round<MAXC, FA>(wrow, arow, sv, stager, c0, first, qs, st, sg, r, g, asum, acc, arowf, &sc, mxv, &fa, tinv); break;
        }
    }
    if (stager) asum_p[st][sg] = asum;
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
            y[(int64_t)t * M + m] = fmul_rn(fmul_rn((float)v, w_scale), FA ? tinv[t] : act_scale[t]);
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
    const int64_t zs = (int64_t)kIbTok * M;
    float v[kMaxSlices];  // every load before the first add (at most kMaxSlices slices)
#pragma unroll
    for (int z = 0; z < kMaxSlices; ++z) v[z] = z < nslice ? p[z * zs] : 0.0f;
    float s = v[0];  // integers below 2^24: exact in any order
#pragma unroll
    for (int z = 1; z < kMaxSlices; ++z)
        if (z < nslice) s += v[z];
    y[i] = fmul_rn(fmul_rn(s, w_scale), act_scale[t]);
}

// K slices of the batched I2_S GEMV: about one workgroup per CU (256), at
// least 4 chunks of 256 columns per slice, at most kIbChunks where 16 slices
// allow.
inline int ib_slices(int64_t M, int64_t K) {
    const int64_t groups = (M + kIbRows - 1) / kIbRows, nsc = K / 256;
    int64_t S = std::min<int64_t>((256 + groups - 1) / groups, std::max<int64_t>(1, nsc / 4));
    S = std::max<int64_t>(S, (nsc + kIbChunks - 1) / kIbChunks);
    return (int)std::max<int64_t>(1, std::min<int64_t>({S, 16, nsc}));
}

// ---------------------------------------------------------------------------
// Ternary GEMM on int8 MFMA: i2s_gemm_vnni for many tokens (prefill)
// ---------------------------------------------------------------------------
//   out[m*N + n] = (float) sum_k t(m, k) * a[n][k]      (src/kernel_i2s.cpp:201-235)
// exact in int32.  v_mfma_i32_16x16x64_i8, A = weights (u-codes u = t + 1 in
// {0, 1, 2}), B = activations, D - sum_k a[n][k] = sum t a.  The MFMA's k
// order is permuted alike on both operands: in a 16-column group whose codes
// are the dword q (column 4b + f in field f of byte b), plane f of the u-codes,
// (ucode(q) >> 2f) & 0x03030303, holds column 4b + f at byte b -- two VALU
// per four weights -- and the activations' 16-byte group is put in the same
// order by a 4x4 byte transpose (8 v_perm) on its way into LDS; the token
// sums over k come from the same loads (v_dot4 with ones).
//   * workgroup tile 128 weight rows x 64 tokens, K steps of 256, one per CU
//     at config size (4096 x 512): per step 8 KB of codes and 16 KB of
//     activations enter the CU (a 64 x 128 tile needs 4 + 32 KB; the step
//     time follows the bytes the CU has in flight, not a unit's rate);
//   * tile order: the tn token tiles of one weight-row tile on consecutive
//     workgroups, i.e. spread over the XCDs (at tn = 8 each XCD's L2 holds one
//     token tile for all of its workgroups; blocking the XCDs' tiles so each
//     L2 serves a quarter of the codes measured slower);
//   * 8 waves: wave (wr, wk) holds rows 32wr..32wr+31 x all 64 tokens (2 x 4
//     accumulator tiles) over chunks 2wk, 2wk+1 (64 columns each) of a step;
//   * weights: each wave decodes its own rows and chunks straight into A
//     fragments in registers (no LDS): lane (r, g) loads 8 code bytes of row
//     r, whose two dwords are its fragments of the two chunks (the chunks' k
//     order is taken alike on the B side); codes 2 steps ahead;
//   * activations: each wave loads half the step of 16 tokens, 2 steps ahead
//     in registers, into a double-buffered LDS tile (XOR-swizzled 16-byte
//     slots, conflict-free).
constexpr int TGM = 128, TGN = 64, TGK = 256;

// LDS byte offset of 16-byte slot q (0..15) of token row n in a step tile
__device__ __forceinline__ int tg_off(int n, int q) { return n * TGK + 16 * (q ^ (n & 7)); }

// 4x4 byte transpose of a 16-byte group: byte i of dword s of the result is
// byte s of dword i of v (column 4i + s of the group -> byte position 4s + i)
__device__ __forceinline__ uint4 group_t4x4(const uint4& v) {
    const uint32_t lo_xy = __builtin_amdgcn_perm(v.y, v.x, 0x05010400u), hi_xy = __builtin_amdgcn_perm(v.y, v.x, 0x07030602u);
    const uint32_t lo_zw = __builtin_amdgcn_perm(v.w, v.z, 0x05010400u), hi_zw = __builtin_amdgcn_perm(v.w, v.z, 0x07030602u);
    return make_uint4(__builtin_amdgcn_perm(lo_zw, lo_xy, 0x05040100u), __builtin_amdgcn_perm(lo_zw, lo_xy, 0x07060302u),
                      __builtin_amdgcn_perm(hi_zw, hi_xy, 0x05040100u), __builtin_amdgcn_perm(hi_zw, hi_xy, 0x07060302u));
}

// ROWS: the decoder prefill's down projection -- out is y [N][M] with
// y[n][m] = ((float)sum * w_scale) * inv[n], each product rounded on its
// own: the reference's i2s_gemv epilogue (src/kernel_i2s.cpp:32-40) for
// every token row, bit for bit (the sums are exact integers below 2^24).
// 8 waves, two per SIMD (one SIMD's pair interleaves its decode, LDS reads and MFMAs: 41.2 -> 39.7 us against
// 4 waves of all four chunks at 4096 x 512 x 11008): wave (wr, wk) holds rows 32 wr .. 32 wr + 31 x all 64
// tokens for chunks 2 wk, 2 wk + 1 of every step; the two K halves' sums meet through LDS at the end.
constexpr int TGT = 512;
template <bool ROWS = false>
__global__ __launch_bounds__(TGT) void i2s_gemm_mfma(const uint8_t* w, const int8_t* a, float* __restrict__ out, int M,
                                                     int N, int K, float w_scale = 0.0f,
                                                     const float* __restrict__ inv = nullptr) {
    __shared__ __align__(16) uint8_t bt[2][TGN * TGK];
    __shared__ int asum[2][TGN];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 3, wk = wave >> 2;
    const int r16 = lane & 15, g = lane >> 4;
    const int tn = (N + TGN - 1) / TGN;
    const int m0 = (blockIdx.x / tn) * TGM, n0 = (blockIdx.x % tn) * TGN;
    const int bpr = K / 4, steps = K / TGK;

    // ---- codes: lane (r16, g), row tile i: row m0 + 32 wr + 16 i + r16, code dwords 4g + 2wk and 4g + 2wk + 1
    // of the step (16 columns each): the planes of dword 4g + c are the lane's A fragment of chunk c, so chunk
    // c's B fragment of lane (n, g) is the 16-column group 4g + c of token n (addresses: a uniform base per step
    // plus a loop-invariant 32-bit lane offset, so that no load's destination registers share a dying address)
    uint32_t woff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
        woff[i] = (uint32_t)min(m0 + 32 * wr + 16 * i + r16, M - 1) * (uint32_t)bpr + 16 * g + 8 * wk;
    constexpr int LEAD = 2;  // steps between a load's issue and its use (codes) / its LDS store (activations)
    uint2 cw[LEAD + 1][2];
    // ---- activations: wave (wr, wk) loads token n0 + 16 wr + r16, bytes 64 c + 16 g (group 4c + g) of the
    // step for c = 2 wk, 2 wk + 1
    const uint32_t boff = (uint32_t)min(n0 + 16 * wr + r16, N - 1) * (uint32_t)K + 16 * g + 128 * wk;
    uint4 bw[LEAD + 1][2];
    int tsum = 0;  // sum of the bytes this lane loads of its token
    auto load_codes = [&](int step, uint2 (&dst)[2]) {
        const uint8_t* base = w + (int64_t)min(step, steps - 1) * (TGK / 4);
#pragma unroll
        for (int i = 0; i < 2; ++i) dst[i] = *(const uint2*)(base + woff[i]);
    };
    auto load_acts = [&](int step, uint4 (&dst)[2]) {
        const int8_t* base = a + (int64_t)min(step, steps - 1) * TGK;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) dst[cc] = ld16(base + boff + 64 * cc);
    };
    // B(step) into LDS in the codes' k order, its bytes into tsum (steps past the end add nothing)
    auto store_acts = [&](const uint4 (&src)[2], uint8_t* tile, bool real) {
        const uint32_t ones = real ? 0x01010101u : 0u;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            *(uint4*)(tile + tg_off(16 * wr + r16, 4 * (2 * wk + cc) + g)) = group_t4x4(src[cc]);
            tsum = dot4(src[cc].x, ones, dot4(src[cc].y, ones, dot4(src[cc].z, ones, dot4(src[cc].w, ones, tsum))));
        }
    };
    i32x4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

    // prologue: the loads of steps 0 .. LEAD - 1 in the loop's order (B(t) then codes(t) per step t, so that
    // the loop head sees the same loads in flight from both of its predecessors); B(0) into LDS
#pragma unroll
    for (int k = 0; k < LEAD; ++k) {
        __builtin_amdgcn_sched_barrier(0);
        load_acts(k, bw[k]);
        load_codes(k, cw[k]);
    }
    __builtin_amdgcn_sched_barrier(0);
    store_acts(bw[0], bt[0], true);
    __syncthreads();
    constexpr int U = LEAD + 1;  // unroll: every register slot index a constant
    // the step count rounded up to whole unrolled rounds (no exit inside a round: an exit per step made the
    // compiler rotate the accumulators' registers at the loop head, waiting there for every load in flight);
    // the steps past the end take all-zero A fragments (the plane mask pm) and skip their products
    const int steps_u = (steps + U - 1) / U * U;
    for (int s0 = 0; s0 < steps_u; s0 += U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int step = s0 + u;
            const uint32_t pm = step < steps ? 0x03030303u : 0u;
            // loads at the top of the step: B(step + LEAD) and codes(step + LEAD) into the slots that B(step - 1)
            // and codes(step - 1) left
            __builtin_amdgcn_sched_barrier(0);
            load_acts(step + LEAD, bw[(u + LEAD) % U]);
            load_codes(step + LEAD, cw[(u + LEAD) % U]);
            __builtin_amdgcn_sched_barrier(0);
            // A fragments of this step
            i32x4 af[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint2 q = cw[u][i];
                const uint32_t d[2] = {q.x, q.y};
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    const uint32_t uc = ucode(d[cc]);
                    af[i][cc] = i32x4{(int)(uc & pm), (int)((uc >> 2) & pm), (int)((uc >> 4) & pm), (int)((uc >> 6) & pm)};
                }
            }
            // B(step + 1) into the other LDS tile (read by the previous step, before its barrier); the tiles
            // alternate by step parity (U is odd)
            store_acts(bw[(u + 1) % U], bt[(step + 1) & 1], step + 1 < steps);
            const uint8_t* cur = bt[step & 1];
            if (step < steps)  // (a padded step's products are zero: skip them)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                i32x4 bf[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) bf[j] = *(const i32x4*)(cur + tg_off(16 * j + r16, 4 * g + 2 * wk + cc));
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i][cc], bf[j], acc[i][j], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
        }
    }
    // token sums: the four lane groups l, l ^ 16, l ^ 32, l ^ 48 of token 16 wr + r16 (per K half), via LDS
    {
        uint32_t t = (uint32_t)tsum;
        const auto r32 = __builtin_amdgcn_permlane32_swap(t, t, false, false);
        t = lane_pin(r32[0]) + lane_pin(r32[1]);
        const auto r16s = __builtin_amdgcn_permlane16_swap(t, t, false, false);
        t = lane_pin(r16s[0]) + lane_pin(r16s[1]);
        if (g == 0) asum[wk][16 * wr + r16] = (int)t;
    }
    // the K halves' accumulators: waves 4-7 through LDS to waves 0-3
    int* red = (int*)&bt[0][0];
    if (wk == 1) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) *(i32x4*)(red + ((wr * 8 + i * 4 + j) * 64 + lane) * 4) = acc[i][j];
    }
    __syncthreads();
    if (wk == 1) return;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const i32x4 o = *(const i32x4*)(red + ((wr * 8 + i * 4 + j) * 64 + lane) * 4);
            acc[i][j] += o;
        }
    // D: lane l holds rows 32 wr + 16 i + 4 (l/16) + r, token 16 j + l%16
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + 16 * j + r16;
        if (n >= N) continue;
        const int as = asum[0][16 * j + r16] + asum[1][16 * j + r16];
        if constexpr (ROWS) {
            const float ts = inv[n];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int m = m0 + 32 * wr + 16 * i + 4 * g;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = fmul_rn(fmul_rn((float)(acc[i][j][r] - as), w_scale), ts);
                float* dst = out + (int64_t)n * M + m;
                if (m + 3 < M && ((uintptr_t)dst & 15u) == 0) {
                    *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (m + r < M) dst[r] = v[r];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + 32 * wr + 16 * i + 4 * g + r;
                    if (m < M) out[(int64_t)m * N + n] = (float)(acc[i][j][r] - as);
                }
        }
    }
}

template <int LPR, int NSEG>
hipError_t run_i2s_fast(const uint8_t* packed, float w_scale, const float* x, const int8_t* act,
                        const float* act_scale, float* y, int64_t M, int64_t K, int64_t batch, hipStream_t s) {
    constexpr int RPP = MTH_WAVE / LPR;
    const int grid = ceil_div(M, RPP * kWaves);
    const size_t lds = (size_t)((K + 15) / 16) * 16;
    if (x)
        i2s_gemv_fast<LPR, NSEG, true><<<grid, kWG, lds, s>>>(packed, w_scale, x, act, act_scale, y, (int)M,
                                                               (int)K, (int)batch, ResidOut{});
    else
        i2s_gemv_fast<LPR, NSEG, false><<<grid, kWG, lds, s>>>(packed, w_scale, x, act, act_scale, y, (int)M,
                                                                (int)K, (int)batch, ResidOut{});
    return hipGetLastError();
}

template <int LPR, int NSEG>
hipError_t run_i2s_fast_resid(const uint8_t* packed, float w_scale, const int8_t* act, const float* act_scale,
                              int64_t M, int64_t K, const ResidOut& ro, int* nparts, hipStream_t s) {
    constexpr int RPP = MTH_WAVE / LPR;
    *nparts = ceil_div(M, RPP * kWaves);
    const size_t lds = (size_t)((K + 15) / 16) * 16;
    i2s_gemv_fast<LPR, NSEG, false><<<*nparts, kWG, lds, s>>>(packed, w_scale, nullptr, act, act_scale, nullptr,
                                                              (int)M, (int)K, 1, ro);
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

bool i2s_resid_supported(const uint8_t* packed, const int8_t* act, int64_t M, int64_t K) {
    return K % 64 == 0 && K / 64 <= 256 && M < (1ll << 31) && aligned16(packed) && aligned16(act);
}

hipError_t launch_i2s_gemv_resid(const uint8_t* packed, float w_scale, const int8_t* act, const float* act_scale,
                                 int64_t M, int64_t K, const ResidOut& ro, int* nparts, hipStream_t s) {
    const int64_t nseg = K / 64;
    if (nseg <= 16) return run_i2s_fast_resid<16, 1>(packed, w_scale, act, act_scale, M, K, ro, nparts, s);
    if (nseg <= 32) return run_i2s_fast_resid<16, 2>(packed, w_scale, act, act_scale, M, K, ro, nparts, s);
    if (nseg <= 64) return run_i2s_fast_resid<32, 2>(packed, w_scale, act, act_scale, M, K, ro, nparts, s);
    if (nseg <= 128) return run_i2s_fast_resid<32, 4>(packed, w_scale, act, act_scale, M, K, ro, nparts, s);
    if (nseg <= 192) return run_i2s_fast_resid<64, 3>(packed, w_scale, act, act_scale, M, K, ro, nparts, s);
    return run_i2s_fast_resid<64, 4>(packed, w_scale, act, act_scale, M, K, ro, nparts, s);
}

bool i2s_swiglu_supported(const uint8_t* packed, int64_t M, int64_t K) {
    return K >= 64 && K % 64 == 0 && K <= kSwT * kSwQ && M < (1ll << 31) && aligned16(packed);
}

hipError_t launch_i2s_swiglu(const float* g, const float* u, const NormScale& ns, const uint8_t* packed, float w_scale,
                             float* y, int64_t M, int64_t K, const ResidOut& ro, int* nparts, hipStream_t s) {
    const int64_t nseg = K / 64;
    const int grid = ceil_div(M, kSwT / 64);
    const size_t lds = (size_t)K;
    if (nseg <= 64)
        i2s_swiglu_k<1><<<grid, kSwT, lds, s>>>(g, u, ns, packed, w_scale, y, (int)M, (int)K, ro);
    else if (nseg <= 128)
        i2s_swiglu_k<2><<<grid, kSwT, lds, s>>>(g, u, ns, packed, w_scale, y, (int)M, (int)K, ro);
    else
        i2s_swiglu_k<3><<<grid, kSwT, lds, s>>>(g, u, ns, packed, w_scale, y, (int)M, (int)K, ro);
    if (nparts) *nparts = grid;
    return hipGetLastError();
}

hipError_t launch_i2s_act(const float* act, const float* amax, const uint8_t* packed, float w_scale, float* y,
                          int64_t M, int64_t K, const ResidOut& ro, int* nparts, hipStream_t s) {
    if (!i2s_swiglu_supported(packed, M, K) || !aligned16(act)) return hipErrorInvalidValue;
    const int64_t nseg = K / 64;
    const int grid = ceil_div(M, kIaT / 64 * kIaR);
    const size_t lds = (size_t)K;
    if (nseg <= 64)
        i2s_act_k<1><<<grid, kIaT, lds, s>>>(act, amax, packed, w_scale, y, (int)M, (int)K, ro);
    else if (nseg <= 128)
        i2s_act_k<2><<<grid, kIaT, lds, s>>>(act, amax, packed, w_scale, y, (int)M, (int)K, ro);
    else
        i2s_act_k<3><<<grid, kIaT, lds, s>>>(act, amax, packed, w_scale, y, (int)M, (int)K, ro);
    if (nparts) *nparts = grid;
    return hipGetLastError();
}

hipError_t launch_i2s_gemv(const uint8_t* packed, float w_scale, const float* x, const int8_t* act,
                           const float* act_scale, float* y, int64_t M, int64_t K, int64_t batch,
                           hipStream_t s) {
    const int64_t nseg = K / 64;
    const bool fast = K % 64 == 0 && nseg <= 256 && M < (1ll << 31) && aligned16(packed) &&
                      (x ? aligned16(x) : aligned16(act));
    if (fast && batch == 1 && x && K <= 4096) {
        // batch 1, f32 activations: all loads up front, 16 rows per workgroup
        const int grid = ceil_div(M, 4 * kWaves);
        const size_t lds = (size_t)K;
        if (K == kK4096)
            i2s_gemv_k4096<<<grid, kWG, lds, s>>>(packed, w_scale, x, y, (int)M);
        else
            i2s_gemv_rows<4, 1, 4, true><<<grid, kWG, lds, s>>>(packed, w_scale, x, act, act_scale, y, (int)M,
                                                                (int)K);
        return hipGetLastError();
    }
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
        i2s_gemv_bt<kIbChunks, kIbWaves><<<grid, kIbWaves * 64, 0, s>>>(packed, w_scale, act + t0 * K, act_scale + t0, y + t0 * M, partial, (int)M,
                                         (int)K, b);
        if (S > 1)
            i2s_bt_reduce<<<ceil_div((int64_t)b * M, kWG), kWG, 0, s>>>(partial, w_scale, act_scale + t0, y + t0 * M,
                                                                        (int)M, b, S);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_i2s_gemv_bt_slices(const uint8_t* packed, float w_scale, const int8_t* act, const float* act_scale,
                                    float* y, int64_t M, int64_t K, int64_t batch, float* partial, Slices* out,
                                    hipStream_t s) {
    const int S = ib_slices(M, K);
    i2s_gemv_bt<kIbChunks, kIbWaves><<<dim3(ceil_div(M, kIbRows), (unsigned)S), kIbWaves * 64, 0, s>>>(packed, w_scale, act, act_scale, y, partial,
                                                                        (int)M, (int)K, (int)batch);
    *out = S == 1 ? plain_slices(y, M) : Slices{partial, M, kIbTok * M, S, w_scale, act_scale};
    return hipGetLastError();
}

hipError_t launch_i2s_gemv_bt_f32act(const uint8_t* packed, float w_scale, const float* act, int64_t lda,
                                     const float* amax, int nmx, float* inv, float* y, int64_t M, int64_t K,
                                     int64_t batch, float* partial, Slices* out, hipStream_t s) {
    if (!i2s_bt_supported(M, K, batch) || batch > kIbTok || nmx < 1 || nmx > 16 * kIbFaMx)
        return hipErrorInvalidValue;
    const int S = ib_slices(M, K);
    const I2sF32Act fa{act, lda, amax, nmx, inv};
    i2s_gemv_bt<kIbFaChunks, kIbWaves, true><<<dim3(ceil_div(M, kIbRows), (unsigned)S), kIbWaves * 64, 0, s>>>(
        packed, w_scale, nullptr, nullptr, y, partial, (int)M, (int)K, (int)batch, fa);
    *out = S == 1 ? plain_slices(y, M) : Slices{partial, M, kIbTok * M, S, w_scale, inv};
    return hipGetLastError();
}

hipError_t launch_i2s_gemv_bt_f32act_y(const uint8_t* packed, float w_scale, const float* act, int64_t lda,
                                       const float* amax, int nmx, float* inv, float* y, int64_t M, int64_t K,
                                       int64_t batch, float* partial, hipStream_t s) {
    Slices out{};
    const hipError_t e = launch_i2s_gemv_bt_f32act(packed, w_scale, act, lda, amax, nmx, inv, y, M, K, batch, partial,
                                                   &out, s);
    if (e != hipSuccess || out.n == 1) return e;
    i2s_bt_reduce<<<ceil_div(batch * M, kWG), kWG, 0, s>>>(partial, w_scale, inv, y, (int)M, (int)batch, out.n);
    return hipGetLastError();
}

hipError_t launch_i2s_gemm(const uint8_t* w, const float* a, float* o, int64_t M, int64_t N, int64_t K,
                           hipStream_t s) {
    i2s_gemm_k<<<ceil_div(M * N, kWaves), kWG, 0, s>>>(w, a, o, M, N, K);
    return hipGetLastError();
}

bool i2s_gemm_mfma_ok(int64_t M, int64_t N, int64_t K) {
    // (the kernel's lane offsets into the codes and the activations are 32-bit)
    return M >= 64 && N >= 64 && K % TGK == 0 && K < (1ll << 24) && M * (K / 4) < (1ll << 32) &&
           N * K < (1ll << 32) && ((M + TGM - 1) / TGM) * ((N + TGN - 1) / TGN) < (1ll << 31);
}

hipError_t launch_i2s_gemm_vnni(const uint8_t* w, const int8_t* a, float* o, int64_t M, int64_t N, int64_t K,
                                hipStream_t s) {
    if (i2s_gemm_mfma_ok(M, N, K) && (((uintptr_t)w | (uintptr_t)a) & 15u) == 0) {
        const unsigned grid = (unsigned)(((M + TGM - 1) / TGM) * ((N + TGN - 1) / TGN));
        i2s_gemm_mfma<<<grid, TGT, 0, s>>>(w, a, o, (int)M, (int)N, (int)K);
        return hipGetLastError();
    }
    i2s_gemm_vnni_k<<<ceil_div(M * N, kWaves), kWG, 0, s>>>(w, a, o, M, N, K);
    return hipGetLastError();
}

hipError_t launch_i2s_gemm_rows(const uint8_t* w, float w_scale, const int8_t* a, const float* inv, float* y, int64_t M,
                                int64_t N, int64_t K, hipStream_t s) {
    if (!i2s_gemm_mfma_ok(M, N, K) || (((uintptr_t)w | (uintptr_t)a) & 15u) != 0) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(((M + TGM - 1) / TGM) * ((N + TGN - 1) / TGN));
    i2s_gemm_mfma<true><<<grid, TGT, 0, s>>>(w, a, y, (int)M, (int)N, (int)K, w_scale, inv);
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

constexpr int kTl2R = 4;  // rows per wave

size_t tl2_workspace_bytes(const uint8_t* w, int64_t M, int64_t N, int64_t K) {
    const int64_t bpr = (2 * K + 7) / 8;  // = 16 * segments; the transposed q rows are 64 * segments bytes
    const bool fast = bpr % 16 == 0 && aligned16(w) && K <= (1 << 20) && N <= 65535 &&
                      (M + kWaves * kTl2R - 1) / (kWaves * kTl2R) < (1ll << 31);
    return fast ? (size_t)(((N * bpr * 4 + 255) / 256) * 256 + N * 4) : 0;
}

hipError_t launch_tl2_gemm_ws(const uint8_t* w, const float* a, float* o, int64_t M, int64_t N, int64_t K, void* ws,
                              hipStream_t s) {
    const int bpr = (int)((2 * K + 7) / 8), stride = 4 * bpr;
    int8_t* qt = (int8_t*)ws;
    float* qscale = (float*)((char*)ws + ((N * (int64_t)stride + 255) / 256) * 256);
    tl2_quant_k<<<(unsigned)N, kWG, 0, s>>>(a, qt, qscale, (int)K, stride);
    const dim3 grid((unsigned)((M + kWaves * kTl2R - 1) / (kWaves * kTl2R)), (unsigned)N);
    tl2_rows_k<kTl2R><<<grid, kWG, 0, s>>>(w, qt, qscale, o, M, N, bpr);
    return hipGetLastError();
}

}  // namespace mth
