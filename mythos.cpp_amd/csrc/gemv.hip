// gemv.hip — OIL8 / OIL4 codebook GEMV for decode (batch 1..16) on gfx950.
//
// Replaces the CPU loops of src/kernel_oil8.cpp:14-71 and
// src/kernel_oil4.cpp:31-125 (reference semantics: sum_k cb[idx]*x[k] in
// FP32 with the codebook value exact in FP32).
//
// Fast path layout (row-major weights, as the reference stores them):
//   * a wave owns a run of rows; lane l streams 16-byte segments
//     seg = l + 64*s (s < NSEG) of every row with one 128-bit load each,
//     so a wave reads 1 KiB of contiguous weight bytes per instruction;
//   * the lane's activations x[seg*W .. +W) stay in VGPRs for the whole
//     wave (W = weights per segment), loaded once;
//   * OIL8: the 256-entry FP32 codebook is staged in LDS replicated over 32
//     bank columns (tab[e*32 + c]); lane l reads column l%32, so the 32 lanes
//     of a half-wave hit 32 different banks whatever the indices are;
//   * OIL4: the 16 codebook entries a lane needs are written (as FP32) into a
//     private LDS column of the lane's wave (tab[e*64 + lane]) and gathered
//     from there: again one bank per lane, no conflicts;
//   * per-row partial sums are reduced across the wave with xor-shuffles.
// Anything else (K not a multiple of 16, unaligned pointers, K beyond the
// register budget, the reference's per-(m,n) weight indexing) goes to the
// generic kernels at the bottom: one wave per output, lanes striding k.
#include "common.h"
#include "launch.h"

namespace mth {
namespace {

constexpr int kWG = 256;
constexpr int kWaves = kWG / MTH_WAVE;

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// ===================================================================
// OIL8
// ===================================================================
template <int NSEG, int RG>
__global__ __launch_bounds__(kWG, 2) void oil8_gemv_fast(
    const uint8_t* __restrict__ idx, const float* __restrict__ cb, const float* __restrict__ x,
    float* __restrict__ y, int M, int K, int batch, int rows_per_wave) {
    __shared__ float tab[256 * 32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nseg = K >> 4;
    const int r0 = (blockIdx.x * kWaves + wave) * rows_per_wave;
    const int r1 = min(M, r0 + rows_per_wave);

    auto load_rows = [&](uint4 (&w)[RG][NSEG], int r) {
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int s = 0; s < NSEG; ++s) {
                const int seg = lane + 64 * s;
                if (r + g < r1 && seg < nseg)
                    w[g][s] = ld_stream(idx + (int64_t)(r + g) * K + (int64_t)seg * 16);
                else
                    w[g][s] = make_uint4(0, 0, 0, 0);
            }
    };

    uint4 wc[RG][NSEG];
    load_rows(wc, r0);  // first weights in flight before the table is staged

#pragma unroll 4
    for (int i = 0; i < 32; ++i) {
        const int e = (tid >> 5) + 8 * i;
        tab[e * 32 + (tid & 31)] = cb[e];
    }
    __syncthreads();
    if (r0 >= M) return;
    const float* col = tab + (lane & 31);

    for (int t = 0; t < batch; ++t) {
        const float* xt = x + (int64_t)t * K;
        float xr[NSEG][16];
#pragma unroll
        for (int s = 0; s < NSEG; ++s) {
            const int seg = lane + 64 * s;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float4 v = seg < nseg ? ldf4(xt + seg * 16 + 4 * q) : make_float4(0, 0, 0, 0);
                xr[s][4 * q + 0] = v.x; xr[s][4 * q + 1] = v.y;
                xr[s][4 * q + 2] = v.z; xr[s][4 * q + 3] = v.w;
            }
        }
        if (t > 0) load_rows(wc, r0);
        for (int r = r0; r < r1; r += RG) {
            uint4 wn[RG][NSEG];
            const bool more = r + RG < r1;
            if (more) load_rows(wn, r + RG);
            float acc[RG];
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                acc[g] = 0.0f;
#pragma unroll
                for (int s = 0; s < NSEG; ++s) {
                    if (s == NSEG - 1 && lane + 64 * s >= nseg) continue;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t wd = u4get(wc[g][s], d);
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const uint32_t e = (wd >> (8 * b)) & 0xffu;
                            acc[g] = fmaf(col[e * 32], xr[s][4 * d + b], acc[g]);
                        }
                    }
                }
            }
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                const float v = group_sum<64>(acc[g]);
                if (lane == 0 && r + g < r1) y[(int64_t)t * M + r + g] = v;
            }
            if (more) {
#pragma unroll
                for (int g = 0; g < RG; ++g)
#pragma unroll
                    for (int s = 0; s < NSEG; ++s) wc[g][s] = wn[g][s];
            }
        }
    }
}

// Generic: one wave per output element.  Row r uses weights base + r*K and
// activation row (r % xmod) + t; out[t*ldy + r].
__global__ __launch_bounds__(kWG) void oil8_generic(
    const uint8_t* __restrict__ idx, const float* __restrict__ cb, const float* __restrict__ act,
    float* __restrict__ out, int64_t R, int64_t K, int64_t xmod, int64_t batch, int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (r >= R) return;
    const uint8_t* w = idx + r * K;
    for (int64_t t = 0; t < batch; ++t) {
        const float* a = act + ((r % xmod) + t) * K;
        float s = 0.0f;
        for (int64_t k = lane; k < K; k += 64) s = fmaf(cb[w[k]], a[k], s);
        s = group_sum<64>(s);
        if (lane == 0) out[t * ldy + r] = s;
    }
}

// ===================================================================
// OIL4
// ===================================================================
// 16 bytes of nibbles = 32 weights per segment; element k of a row is the low
// nibble of byte k/2 for even k, the high nibble for odd k.
template <int NSEG, int RG, bool SHARED>
__global__ __launch_bounds__(kWG, 2) void oil4_gemv_fast(
    const uint8_t* __restrict__ nib, const uint16_t* __restrict__ cbs, int cb_block,
    const float* __restrict__ x, float* __restrict__ y, int M, int K, int batch, int rows_per_wave) {
    __shared__ float tab[kWaves][16 * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nseg = K >> 5;
    const int nb = SHARED ? 1 : K / cb_block;
    const int seg_per_blk = SHARED ? 1 : cb_block >> 5;
    const int r0 = (blockIdx.x * kWaves + wave) * rows_per_wave;
    const int r1 = min(M, r0 + rows_per_wave);
    float* col = &tab[wave][lane];

    auto load_rows = [&](uint4 (&w)[RG][NSEG], uint4 (&c)[RG][NSEG][2], int r) {
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int s = 0; s < NSEG; ++s) {
                const int seg = lane + 64 * s;
                if (r + g < r1 && seg < nseg) {
                    w[g][s] = ld_stream(nib + (int64_t)(r + g) * (K >> 1) + (int64_t)seg * 16);
                    if (!SHARED) {
                        const uint16_t* cp = cbs + ((int64_t)(r + g) * nb + seg / seg_per_blk) * 16;
                        c[g][s][0] = ld16(cp);
                        c[g][s][1] = ld16(cp + 8);
                    }
                } else {
                    w[g][s] = make_uint4(0, 0, 0, 0);
                    if (!SHARED) c[g][s][0] = c[g][s][1] = make_uint4(0, 0, 0, 0);
                }
            }
    };

    uint4 wc[RG][NSEG], cc[RG][NSEG][2];
    load_rows(wc, cc, r0);
    if (SHARED) {
        // one codebook for the tensor: every wave fills its own columns once
        const uint4 c0 = ld16(cbs), c1 = ld16(cbs + 8);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t wd = u4get(e < 8 ? c0 : c1, (e & 7) >> 1);
            col[e * 64] = (e & 1) ? h2f_hi(wd) : h2f_lo(wd);
        }
    }
    if (r0 >= M) return;

    for (int t = 0; t < batch; ++t) {
        const float* xt = x + (int64_t)t * K;
        float xr[NSEG][32];
#pragma unroll
        for (int s = 0; s < NSEG; ++s) {
            const int seg = lane + 64 * s;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                float4 v = seg < nseg ? ldf4(xt + seg * 32 + 4 * q) : make_float4(0, 0, 0, 0);
                xr[s][4 * q + 0] = v.x; xr[s][4 * q + 1] = v.y;
                xr[s][4 * q + 2] = v.z; xr[s][4 * q + 3] = v.w;
            }
        }
        if (t > 0) load_rows(wc, cc, r0);
        for (int r = r0; r < r1; r += RG) {
            uint4 wn[RG][NSEG], cn[RG][NSEG][2];
            const bool more = r + RG < r1;
            if (more) load_rows(wn, cn, r + RG);
            float acc[RG];
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                acc[g] = 0.0f;
#pragma unroll
                for (int s = 0; s < NSEG; ++s) {
                    if (s == NSEG - 1 && lane + 64 * s >= nseg) continue;
                    if (!SHARED) {
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            const uint32_t wd = u4get(cc[g][s][e >> 3], (e & 7) >> 1);
                            col[e * 64] = (e & 1) ? h2f_hi(wd) : h2f_lo(wd);
                        }
                    }
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t wd = u4get(wc[g][s], d);
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const uint32_t e = (wd >> (4 * j)) & 0xfu;
                            acc[g] = fmaf(col[e * 64], xr[s][8 * d + j], acc[g]);
                        }
                    }
                }
            }
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                const float v = group_sum<64>(acc[g]);
                if (lane == 0 && r + g < r1) y[(int64_t)t * M + r + g] = v;
            }
            if (more) {
#pragma unroll
                for (int g = 0; g < RG; ++g)
#pragma unroll
                    for (int s = 0; s < NSEG; ++s) {
                        wc[g][s] = wn[g][s];
                        cc[g][s][0] = cn[g][s][0];
                        cc[g][s][1] = cn[g][s][1];
                    }
            }
        }
    }
}

// Generic OIL4: one wave per output.  Weight row r starts at byte
// (r*K)/2 (the reference's `((m*N+n)*K)/2`), element k uses nibble k%2 of
// byte k/2 of that row.  Codebook: shared (cb_block == 0) or per block of
// row r (codebooks of row r at cbs + r*(K/cb_block)*16).
__global__ __launch_bounds__(kWG) void oil4_generic(
    const uint8_t* __restrict__ nib, const uint16_t* __restrict__ cbs, int64_t cb_block,
    const float* __restrict__ act, float* __restrict__ out, int64_t R, int64_t K, int64_t xmod,
    int64_t batch, int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (r >= R) return;
    const uint8_t* w = nib + (r * K) / 2;
    const uint16_t* cb = cb_block ? cbs + r * (K / cb_block) * 16 : cbs;
    for (int64_t t = 0; t < batch; ++t) {
        const float* a = act + ((r % xmod) + t) * K;
        float s = 0.0f;
        for (int64_t k = lane; k < K; k += 64) {
            const uint32_t byte = w[k >> 1];
            const uint32_t e = (k & 1) ? (byte >> 4) & 0xfu : byte & 0xfu;
            const uint16_t h = cb_block ? cb[(k / cb_block) * 16 + e] : cb[e];
            s = fmaf(h2f(h), a[k], s);
        }
        s = group_sum<64>(s);
        if (lane == 0) out[t * ldy + r] = s;
    }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Rows per wave: enough waves for >= 2 workgroups per CU on 256 CUs, at
// least RG rows each.
inline int pick_rows_per_wave(int64_t M, int rg) {
    const int64_t target_waves = 256 * 2 * kWaves;
    int64_t rpw = (M + target_waves - 1) / target_waves;
    rpw = ((rpw + rg - 1) / rg) * rg;
    return (int)(rpw < rg ? rg : rpw);
}

}  // namespace

hipError_t launch_oil8_gemv(const uint8_t* idx, const float* cb, const float* x, float* y,
                            int64_t M, int64_t K, int64_t batch, hipStream_t s) {
    const bool fast = (K % 16 == 0) && K <= 4096 && M < (1ll << 31) && aligned16(idx) && aligned16(x);
    if (fast) {
        constexpr int RG = 2;
        const int rpw = pick_rows_per_wave(M, RG);
        const int grid = ceil_div(ceil_div(M, rpw), kWaves);
        const int nseg = (int)(K / 16);
        if (nseg <= 64)
            oil8_gemv_fast<1, RG><<<grid, kWG, 0, s>>>(idx, cb, x, y, (int)M, (int)K, (int)batch, rpw);
        else if (nseg <= 128)
            oil8_gemv_fast<2, RG><<<grid, kWG, 0, s>>>(idx, cb, x, y, (int)M, (int)K, (int)batch, rpw);
        else if (nseg <= 192)
            oil8_gemv_fast<3, RG><<<grid, kWG, 0, s>>>(idx, cb, x, y, (int)M, (int)K, (int)batch, rpw);
        else
            oil8_gemv_fast<4, RG><<<grid, kWG, 0, s>>>(idx, cb, x, y, (int)M, (int)K, (int)batch, rpw);
    } else {
        oil8_generic<<<ceil_div(M, kWaves), kWG, 0, s>>>(idx, cb, x, y, M, K, 1, batch, M);
    }
    return hipGetLastError();
}

hipError_t launch_oil8_gemm_mn(const uint8_t* idx, const float* cb, const float* act, float* out,
                               int64_t M, int64_t N, int64_t K, hipStream_t s) {
    if (N == 1) return launch_oil8_gemv(idx, cb, act, out, M, K, 1, s);
    const int64_t R = M * N;
    oil8_generic<<<ceil_div(R, kWaves), kWG, 0, s>>>(idx, cb, act, out, R, K, N, 1, R);
    return hipGetLastError();
}

hipError_t launch_oil4_gemv(const uint8_t* nib, const uint16_t* cbs, int64_t cb_block,
                            const float* x, float* y, int64_t M, int64_t K, int64_t batch,
                            hipStream_t s) {
    const bool fast = (K % 32 == 0) && K <= 4096 && M < (1ll << 31) && aligned16(nib) && aligned16(x) &&
                      aligned16(cbs) && (cb_block == 0 || cb_block % 32 == 0);
    if (fast) {
        constexpr int RG = 2;
        const int rpw = pick_rows_per_wave(M, RG);
        const int grid = ceil_div(ceil_div(M, rpw), kWaves);
        const int nseg = (int)(K / 32);
        const int blk = (int)cb_block;
        if (cb_block == 0) {
            if (nseg <= 64)
                oil4_gemv_fast<1, RG, true><<<grid, kWG, 0, s>>>(nib, cbs, blk, x, y, (int)M, (int)K, (int)batch, rpw);
            else
                oil4_gemv_fast<2, RG, true><<<grid, kWG, 0, s>>>(nib, cbs, blk, x, y, (int)M, (int)K, (int)batch, rpw);
        } else {
            if (nseg <= 64)
                oil4_gemv_fast<1, RG, false><<<grid, kWG, 0, s>>>(nib, cbs, blk, x, y, (int)M, (int)K, (int)batch, rpw);
            else
                oil4_gemv_fast<2, RG, false><<<grid, kWG, 0, s>>>(nib, cbs, blk, x, y, (int)M, (int)K, (int)batch, rpw);
        }
    } else {
        oil4_generic<<<ceil_div(M, kWaves), kWG, 0, s>>>(nib, cbs, cb_block, x, y, M, K, 1, batch, M);
    }
    return hipGetLastError();
}

hipError_t launch_oil4_gemm_mn(const uint8_t* nib, const uint16_t* cb, const float* act, float* out,
                               int64_t M, int64_t N, int64_t K, hipStream_t s) {
    if (N == 1 && K % 2 == 0) return launch_oil4_gemv(nib, cb, 0, act, out, M, K, 1, s);
    const int64_t R = M * N;
    oil4_generic<<<ceil_div(R, kWaves), kWG, 0, s>>>(nib, cb, 0, act, out, R, K, N, 1, R);
    return hipGetLastError();
}

}  // namespace mth
