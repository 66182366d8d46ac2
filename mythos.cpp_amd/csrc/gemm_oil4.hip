// gemm_oil4.hip — OIL4 prefill GEMM on gfx950 MFMA.
//
//   C[m][n] = bf16( sum_k A[m][k] * W[n][k] ),  A bf16 [M][K], W OIL4 [N][K]
//
// The per-token definition is the reference's oil4_gemm scalar loop
// (src/kernel_oil4.cpp:31-54) with per-128-weight-block FP16 codebooks.  Only
// here is the work a dense contraction, so it runs on the matrix cores:
//   * W tiles are dequantised in LDS: nibbles -> FP16 codebook value (exact);
//   * A tiles are converted bf16 -> FP16 (exact for |a| in [2^-14, 65504]);
//   * v_mfma_f32_16x16x32_f16 with FP32 accumulation; bf16 (RNE) output.
// Tile: 128 (m) x 128 (n) x 32 (k) per 256-thread workgroup, 2x2 waves of
// 64x64, register double-buffered global loads.
#include "common.h"
#include "launch.h"

namespace mth {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDA = BK + 8;  // halves per LDS row (80 B: 2-way bank aliasing at most)

__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t v) {
    const float lo = __uint_as_float(v << 16), hi = __uint_as_float(v & 0xffff0000u);
    const _Float16 hl = (_Float16)lo, hh = (_Float16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, hl) | ((uint32_t)__builtin_bit_cast(uint16_t, hh) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__global__ __launch_bounds__(256, 2) void oil4_gemm_prefill_k(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ nib, const uint16_t* __restrict__ cbs,
    int cb_block, uint16_t* __restrict__ C, int M, int N, int K) {
    __shared__ __align__(16) _Float16 As[BM * LDA];
    __shared__ __align__(16) _Float16 Bs[BN * LDA];
    __shared__ __align__(16) uint16_t Cb[BN * 16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int nb = K / cb_block;

    // global -> register staging
    uint4 ra[2];      // A: rows (tid>>2) and 64+(tid>>2), 8 halves at k (tid&3)*8
    uint2 rw;         // W: row tid>>1, 16 nibbles at k (tid&1)*16
    uint4 rc;         // codebook half: row tid>>1, entries (tid&1)*8..+7
    const int a_r = tid >> 2, a_c = (tid & 3) * 8;
    const int w_r = tid >> 1, w_h = tid & 1;

    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int m = m0 + a_r + 64 * i;
            ra[i] = m < M ? ld16(A + (int64_t)m * K + k0 + a_c) : make_uint4(0, 0, 0, 0);
        }
        const int n = n0 + w_r;
        if (n < N) {
            rw = *(const uint2*)(nib + (int64_t)n * (K >> 1) + (k0 >> 1) + w_h * 8);
            rc = ld16(cbs + ((int64_t)n * nb + k0 / cb_block) * 16 + w_h * 8);
        } else {
            rw = make_uint2(0, 0);
            rc = make_uint4(0, 0, 0, 0);
        }
    };

    float4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4v{0, 0, 0, 0};

    gload(0);
    for (int k0 = 0; k0 < K; k0 += BK) {
        // registers -> LDS (A converted, codebooks raw)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            uint4 v = ra[i];
            v.x = bf16x2_to_f16x2(v.x); v.y = bf16x2_to_f16x2(v.y);
            v.z = bf16x2_to_f16x2(v.z); v.w = bf16x2_to_f16x2(v.w);
            *(uint4*)&As[(a_r + 64 * i) * LDA + a_c] = v;
        }
        *(uint4*)&Cb[w_r * 16 + w_h * 8] = rc;
        const uint2 wv = rw;
        __syncthreads();
        // dequantise W: 16 nibbles of row w_r -> FP16 in Bs
        {
            const uint16_t* cbr = &Cb[w_r * 16];
            uint32_t out[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t byte = ((j < 4 ? wv.x : wv.y) >> (8 * (j & 3))) & 0xffu;
                out[j] = (uint32_t)cbr[byte & 0xfu] | ((uint32_t)cbr[byte >> 4] << 16);
            }
            uint4* dst = (uint4*)&Bs[w_r * LDA + w_h * 16];
            dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
            dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
        }
        if (k0 + BK < K) gload(k0 + BK);
        __syncthreads();

        // MFMA: lane l holds row (l%16), k-group (l/16)*8 of each 16x32 fragment
        half8 af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            af[i] = *(const half8*)&As[(wm * 64 + 16 * i + (lane & 15)) * LDA + (lane >> 4) * 8];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            bf[j] = *(const half8*)&Bs[(wn * 64 + 16 * j + (lane & 15)) * LDA + (lane >> 4) * 8];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        __syncthreads();
    }

    // D layout: lane l holds column (l%16), rows 4*(l/16) + r
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 64 + 16 * j + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 64 + 16 * i + 4 * (lane >> 4) + r;
                if (m < M && n < N) C[(int64_t)m * N + n] = f32_to_bf16_rne(acc[i][j][r]);
            }
        }
}

}  // namespace

bool oil4_gemm_prefill_supported(int64_t M, int64_t N, int64_t K, int64_t cb_block) {
    return K % BK == 0 && cb_block % BK == 0 && M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) &&
           (M + BM - 1) / BM < 65536;
}

hipError_t launch_oil4_gemm_prefill(const uint16_t* a_bf16, const uint8_t* nib, const uint16_t* cbs,
                                    int64_t cb_block, uint16_t* c_bf16, int64_t M, int64_t N, int64_t K,
                                    hipStream_t s) {
    dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    oil4_gemm_prefill_k<<<grid, 256, 0, s>>>(a_bf16, nib, cbs, (int)cb_block, c_bf16, (int)M, (int)N, (int)K);
    return hipGetLastError();
}

}  // namespace mth
