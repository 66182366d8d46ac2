// gemm_oil4.hip — OIL4 prefill GEMM on gfx950 MFMA.
//
//   C[m][n] = bf16( sum_k A[m][k] * W[n][k] ),  A bf16 [M][K], W OIL4 [N][K]
//
// The per-token definition is the reference's oil4_gemm scalar loop
// (src/kernel_oil4.cpp:31-54) with per-128-weight-block FP16 codebooks.  Only
// here is the work a dense contraction, so it runs on the matrix cores:
//   * W tiles are dequantised in LDS: nibbles -> FP16 codebook value (exact);
//   * each row of A is scaled by a power of two 2^s (max|a| 2^s in [2^14,
//     2^15), oil4_prefill_rowshift) and converted bf16 -> FP16, which is exact
//     for every value within 2^-31 of the row's maximum; the output row is
//     scaled back by 2^-s (exact) before its bf16 rounding, so no input range
//     overflows FP16 or is flushed by it;
//   * v_mfma_f32_16x16x32_f16 with FP32 accumulation; bf16 (RNE) output.
// Tile: 128 (m) x 128 (n) x 32 (k) per 256-thread workgroup, 2x2 waves of
// 64x64, register double-buffered global loads.
#include "common.h"
#include "launch.h"
#include "oil4_common.h"

#include <type_traits>

namespace mth {
namespace {

typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDA = BK + 8;  // halves per LDS row (80 B: 2-way bank aliasing at most)

// two bf16 -> two FP16 of a * 2^s (s: the row's shift)
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t v, int s) {
    const float lo = ldexpf(__uint_as_float(v << 16), s), hi = ldexpf(__uint_as_float(v & 0xffff0000u), s);
    const _Float16 hl = (_Float16)lo, hh = (_Float16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, hl) | ((uint32_t)__builtin_bit_cast(uint16_t, hh) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Per-row power-of-two shifts of A (one workgroup per row): rsh[m] = s with
// max|a[m][*]| 2^s in [2^14, 2^15) (0 for an all-zero row or one holding
// Inf / NaN), the scale fp16_scale_shift gives the decode kernels' x.
__global__ __launch_bounds__(256) void oil4_prefill_rowshift(const uint16_t* __restrict__ a, int* __restrict__ rsh,
                                                             int M, int K) {
    __shared__ uint32_t red[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const uint16_t* p = a + (int64_t)row * K;
    uint32_t mb = 0;
    // rounds of 2 chunks of 2048 columns, both loads issued before the first
    // use (clamped to the row's last chunk, which is in bounds)
    const int last = K - 8;
    for (int c0 = 0; c0 < K; c0 += 4096) {
        const uint4 v0 = ld16(p + min(c0 + 8 * tid, last)), v1 = ld16(p + min(c0 + 2048 + 8 * tid, last));
        const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) mb = max(mb, max(w[i] & 0x7fffu, (w[i] >> 16) & 0x7fffu));
    }
    mb = group_reduce<64>(mb, UMaxOp{});
    if ((tid & 63) == 0) red[tid >> 6] = mb;
    __syncthreads();
    if (tid == 0) rsh[row] = fp16_scale_shift(__uint_as_float(max(max(red[0], red[1]), max(red[2], red[3])) << 16));
}

__global__ __launch_bounds__(256, 2) void oil4_gemm_prefill_k(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ nib, const uint16_t* __restrict__ cbs,
    int cb_block, uint16_t* __restrict__ C, int M, int N, int K, const int* __restrict__ rsh) {
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
    const int ash[2] = {rsh[min(m0 + a_r, M - 1)], rsh[min(m0 + 64 + a_r, M - 1)]};

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
            v.x = bf16x2_to_f16x2(v.x, ash[i]); v.y = bf16x2_to_f16x2(v.y, ash[i]);
            v.z = bf16x2_to_f16x2(v.z, ash[i]); v.w = bf16x2_to_f16x2(v.w, ash[i]);
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
                if (m < M && n < N) C[(int64_t)m * N + n] = f32_to_bf16_rne(ldexpf(acc[i][j][r], -rsh[m]));
            }
        }
}

// ===================================================================
// Production kernel (oil4_prefill_mfma)
// ===================================================================
// C[m][n] = bf16(sum_k A[m][k] * W[n][k]) with FP32 accumulation on
// v_mfma_f32_16x16x32_f16: W is exact in FP16 (the codebook entries) and A
// is converted bf16 -> FP16 when its fragments are read (exact for
// 2^-14 <= |a| <= 65504; smaller values keep FP16's subnormal precision).
// Rounding W to bf16 instead would add a second 2^-8 rounding per weight and
// put the result over the 2e-3 budget of this path.
//
//   * workgroup tile 256 (m) x BN (n), K steps of 64; 4 waves stacked along m,
//     each 64 x BN = 4 x BN/16 MFMA tiles held in accumulators;
//   * A: each wave instruction reads 8 rows x 128 contiguous bytes; the
//     choice of source chunk per lane XOR-swizzles the 16-byte chunks of a row
//     in LDS so that the MFMA fragment reads hit distinct banks;
//   * W: two threads per row each stream 32 nibbles per step and dequantise
//     them with v_perm byte-plane lookups (oil4_common.h) into the FP16 tile;
//   * one barrier per K step; A loaded 2 steps ahead and W nibbles and
//     codebooks 4 steps ahead into VGPR rings (covering L2 / HBM latency),
//     A and dequantised W tiles double-buffered in LDS.
constexpr int PBM = 256, PBK = 64;

// byte offset of 16-byte chunk c (0..7) of row r in a 128-byte-row tile
__device__ __forceinline__ int pf_off(int r, int c) { return r * 128 + 16 * (c ^ ((r & 7) ^ ((r >> 3) & 1))); }

// 8 bf16 -> 8 FP16 of a * 2^s (through FP32: v_cvt_pk_f16_f32 rounds to
// nearest even; exact inside FP16's range)
__device__ __forceinline__ half8 bf16x8_to_f16(uint4 v, int s) {
    half8 r;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r[2 * i] = (_Float16)ldexpf(__uint_as_float(w[i] << 16), s);
        r[2 * i + 1] = (_Float16)ldexpf(__uint_as_float(w[i] & 0xffff0000u), s);
    }
    return r;
}

template <int BN>
struct PfLds {
    static constexpr int a = PBM * 128;  // one A tile (double-buffered)
    static constexpr int w = BN * 128;   // one dequantised W tile (double-buffered)
    static constexpr int bytes = 2 * a + 2 * w;
};

template <int BN>
__global__ __launch_bounds__(256, 1) void oil4_prefill_mfma(const uint16_t* __restrict__ A, const uint8_t* nib,
                                                            const uint16_t* cbs, int cb_block,
                                                            uint16_t* __restrict__ C, int M, int N, int K,
                                                            const int* __restrict__ rsh) {
    using L = PfLds<BN>;
    constexpr int NT = BN / 16;
    __shared__ __align__(16) uint8_t lds[L::bytes];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * PBM, n0 = blockIdx.x * BN;
    const int nb = K / cb_block;
    const int steps = K / PBK;
    int ash[4];  // shifts of this lane's A fragment rows
#pragma unroll
    for (int i = 0; i < 4; ++i) ash[i] = rsh[min(m0 + 64 * wave + 16 * i + (lane & 15), M - 1)];

    // ---- A: thread T loads 8 16-byte chunks per step (chunk id 256 i + T:
    // row id/8, 16-byte slot id%8 of that row in LDS, holding source chunk
    // slot ^ f(row)); each wave instruction reads 8 rows x 128 contiguous bytes.
    uint4 av[2][8];
    auto load_a = [&](int step, int slot) {
        const int k0 = step * PBK;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int id = i * 256 + tid;
            const int r = id >> 3;
            const int c = (id & 7) ^ ((r & 7) ^ ((r >> 3) & 1));
            av[slot][i] = ld16(A + (int64_t)min(m0 + r, M - 1) * K + k0 + 8 * c);
        }
    };
    auto store_a = [&](int slot, uint8_t* base) {
#pragma unroll
        for (int i = 0; i < 8; ++i) *(uint4*)(base + (i * 256 + tid) * 16) = av[slot][i];
    };

    // ---- W: thread T < 2 BN dequantises row T/2, columns 32 (T%2) .. +31 of
    // each step.  Every thread loads (the others a clamped row), so that all
    // waves issue the same number of loads per step.  Ring of 4 steps in
    // VGPRs: the nibbles and codebook of step s are loaded at step s - 4.
    const bool wt = tid < 2 * BN;
    const int wn = tid >> 1, wh = tid & 1;
    const int wrow = min(n0 + (wt ? wn : 0), N - 1);
    const uint8_t* wnib = nib + (int64_t)wrow * (K >> 1) + 16 * wh;
    const uint16_t* wcb = cbs + (int64_t)wrow * nb * 16;
    uint4 nv[4], ca[4], cc[4];
    auto load_w = [&](int step, int slot) {
        const int k0 = step * PBK;
        nv[slot] = ld_stream(wnib + (k0 >> 1));
        const uint16_t* cp = wcb + (k0 / cb_block) * 16;
        ca[slot] = ld16(cp);
        cc[slot] = ld16(cp + 8);
    };

    floatx4 acc[4][NT];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // Pipeline (all loads into VGPR rings, so the compiler tracks every wait):
    // step s stores A(s) (loaded at s - 2) and the dequantised W(s) (nibbles
    // and codebook loaded at s - 4) into LDS buffers s % 2, passes the one
    // barrier of the step, issues A(s + 2) and W(s + 4) (clamped to the last
    // step near the end) and runs its MFMAs.
#pragma unroll
    for (int u = 0; u < 4; ++u) load_w(u < steps ? u : steps - 1, u);
    load_a(0, 0);
    load_a(steps > 1 ? 1 : 0, 1);
    for (int s0 = 0; s0 < steps; s0 += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int step = s0 + u;
            uint8_t* ab = lds + (u & 1) * L::a;
            uint8_t* wb = lds + 2 * L::a + (u & 1) * L::w;
            store_a(u & 1, ab);
            if (wt) {
                const CbPlanes pl = cb_planes(ca[u], cc[u]);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    *(half8*)(wb + pf_off(wn, 4 * wh + i)) = lookup8_natural(u4get(nv[u], i), pl);
            }
            __syncthreads();
            load_a(min(step + 2, steps - 1), u & 1);
            load_w(min(step + 4, steps - 1), u);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int c = 4 * kk + (lane >> 4);
                half8 af[4], bfr[NT];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    af[i] = bf16x8_to_f16(*(const uint4*)(ab + pf_off(64 * wave + 16 * i + (lane & 15), c)), ash[i]);
#pragma unroll
                for (int j = 0; j < NT; ++j) bfr[j] = *(const half8*)(wb + pf_off(16 * j + (lane & 15), c));
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bfr[j], acc[i][j], 0, 0, 0);
            }
        }
    }

    // D layout: lane l holds column (l%16), rows 4*(l/16) + r
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int n = n0 + 16 * j + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 64 * wave + 16 * i + 4 * (lane >> 4) + r;
                if (m < M && n < N) C[(int64_t)m * N + n] = f32_to_bf16_rne(ldexpf(acc[i][j][r], -rsh[m]));
            }
        }
}

// ===================================================================
// Prefill with FP16 A in MFMA fragment order (oil4_prefill_a16 + oil4_prefill_ws)
// ===================================================================
// oil4_prefill_a16 converts A (bf16) once per call and writes it in the
// order the MFMA reads it: for 16-row group g and 32-column chunk kc, the 64
// lanes' 16-byte A fragments (lane l: row 16g + l % 16, columns 32kc +
// 8(l / 16) .. + 7) are 1 KB contiguous.  Each fragment load of the GEMM is
// then one 1 KB run (8 full 128-byte lines); read in the natural row-major
// order, a fragment load touches 16 rows x 64 bytes (16 half-used lines at
// an 8 KB stride), which measured 96 -> 83 us at config 4.
// One workgroup per row: the row's maximum first (its shift rsh[row], as
// oil4_prefill_rowshift), then its 8-column pieces scaled, converted and
// written to their fragment slots (the second read of the row hits the
// cache).  The workgroups of one 16-row group run on one XCD (workgroup w on
// XCD w % 8: w = 128 (g / 8) + 8 i + g % 8 for row i of group g), so the
// group's 16-byte pieces of each 1 KB run meet in one L2.  Rows past M
// repeat row M - 1 (their outputs are never stored); the workspace holds
// ceil(M / 16) * 16 rows.
__global__ __launch_bounds__(256) void oil4_prefill_a16(const uint16_t* __restrict__ a, uint16_t* __restrict__ a16,
                                                        int M, int K, int* __restrict__ rsh) {
    __shared__ uint32_t red[4];
    const int w = blockIdx.x, tid = threadIdx.x;
    const int g = 8 * (w >> 7) + (w & 7), i = (w >> 3) & 15;
    const int row = 16 * g + i;
    if (16 * g >= M) return;  // a group past the last (grid rounded up to 8 groups)
    const int src = min(row, M - 1);
    const uint16_t* p = a + (int64_t)src * K;
    const int nch = K / 8;  // 8-column pieces
    uint32_t mb = 0;
    for (int c = tid; c < nch; c += 256) {
        const uint4 v = ld16(p + 8 * c);
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) mb = max(mb, max(u[e] & 0x7fffu, (u[e] >> 16) & 0x7fffu));
    }
    mb = group_reduce<64>(mb, UMaxOp{});
    if ((tid & 63) == 0) red[tid >> 6] = mb;
    __syncthreads();
    const int sh = fp16_scale_shift(__uint_as_float(max(max(red[0], red[1]), max(red[2], red[3])) << 16));
    if (tid == 0 && row < M) rsh[row] = sh;
    const int kc32 = K / 32;
    uint16_t* dst = a16 + (int64_t)g * kc32 * 512 + 8 * i;  // lane i of chunk 0
    for (int c = tid; c < nch; c += 256)
        *(half8*)(dst + (int64_t)(c >> 2) * 512 + 128 * (c & 3)) = bf16x8_to_f16(ld16(p + 8 * c), sh);
}

// ===================================================================
// Prefill kernel, producer / consumer waves (oil4_prefill_ws)
// ===================================================================
// A workgroup has 8 waves, two per SIMD (or 12 with CW = 8 consumers), and computes a 256 x BN tile of C:
// waves 0-3 (consumers) hold the accumulators of 64 rows each (32 with CW = 8) and run
// v_mfma_f32_16x16x32_f16 with A fragments loaded from L2 into a ring of PA
// registers sets (PA - 1 K steps ahead); waves CW .. CW + 3 (producers) dequantise W
// (v_perm lookups, oil4_common.h) into a ring of 2 BS FP16 tiles in LDS, one
// tile per K step of 64, BS steps ahead of the consumers; one barrier per BS
// steps hands the tiles over.  The SIMD interleaves the two waves, so the
// dequantisation runs under the MFMAs.  A CU returns vector loads in issue
// order across its waves, so the consumers' A loads (L2 hits) come back
// behind the producers' weight stream (HBM): the A ring runs 3 steps ahead
// where the registers allow it (BN <= 112; measured 79 -> 74 us at config 4
// with BS = 2).  Producer thread pairs stream 32 nibbles per K step of one
// row (4 steps ahead); a row's codebook block (32 bytes) covers two K steps
// (cb_block % 128 == 0) and is loaded once per pair of steps, half by each
// thread of the pair, the halves exchanged with a DPP lane swap.  Workgroups
// on one XCD share an M tile (WG i runs on XCD i % 8), so an XCD's L2 holds
// one M tile's rows of A.  C is staged through LDS as bf16 and written in
// 16-byte pieces.
template <int BN, int BS, bool X32 = false>
struct Pf2Lds {
    static constexpr int w = BN * 128;                   // one K step's dequantised W tile
    static constexpr int stage = 256 * BN * (X32 ? 4 : 2);  // C tile (bf16, or FP32 sums), after the main loop
    static constexpr int bytes = (2 * BS * w > stage) ? 2 * BS * w : stage;
};

// X32 (the decoder's FP32 prompt rows, oil4_prefill_x32): M counts virtual
// rows, 256 per tile: tile T's rows 0-127 are the FP16 hi parts and rows
// 128-255 the lo parts of real rows 128 T .. 128 T + 127 (Mr real rows);
// the epilogue adds the two halves' FP32 sums (products exact, sums FP32:
// the FP32 dot product) and writes FP32 C [Mr][N].
// CW: consumer waves (4: 64 rows each, one per SIMD; 8: 32 rows each, two per SIMD beside the producer wave);
// the workgroup has ws_threads(CW) threads.
constexpr int ws_threads(int cw) { return 64 * (cw + 4); }
template <int BN, int PA, int BS, bool X32 = false, int CW = 4>
__global__ __launch_bounds__(ws_threads(CW)) void oil4_prefill_ws(const uint16_t* __restrict__ A16, const uint8_t* nib,
                                                       const uint16_t* cbs, int cb_block, void* __restrict__ Cv,
                                                       int M, int N, int K, const int* __restrict__ rsh, int Mr = 0) {
    using L = Pf2Lds<BN, BS, X32>;
    constexpr int NT = BN / 16, PW = 4;
    static_assert(PA == 2 || PA == 4, "A ring index");
    static_assert(BS == 1 || BS == 2 || BS == 4, "barrier interval");
    __shared__ __align__(16) uint8_t lds[L::bytes];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tm = (M + PBM - 1) / PBM, tn = N / BN;
    int mt, nt;
    {
        const int id = blockIdx.x, total = tm * tn;
        if (total % 8 == 0 && 8 % tm == 0) {
            const int grp = 8 / tm, xcd = id % 8, slot = id / 8;
            mt = xcd / grp;
            nt = slot * grp + xcd % grp;
        } else {
            mt = id / tn;
            nt = id % tn;
        }
    }
    const int m0 = mt * PBM, n0 = nt * BN;
    const int steps = K / PBK;

    static_assert(CW == 4 || CW == 8, "consumer waves");
    constexpr int NG = 16 / CW;  // 16-row groups per consumer wave
    constexpr int NTH = ws_threads(CW);
    if (wave >= CW) {
        // ---------------- producers ----------------
        const int t = tid - 64 * CW;
        const bool wt = t < 2 * BN;
        const int wn = t >> 1, wh = t & 1;
        const int wrow = n0 + (wt ? wn : 0);
        const uint8_t* wnib = nib + (int64_t)wrow * (K >> 1) + 16 * wh;
        const uint16_t* wcb = cbs + (int64_t)wrow * (K / cb_block) * 16 + 8 * wh;
        const int pairs = steps >> 1;
        uint4 nv[PW], cbh[2];
        auto load_n = [&](int step, int slot) { nv[slot] = ld_stream(wnib + ((step * PBK) >> 1)); };
        auto load_c = [&](int pair, int slot) { cbh[slot] = ld16(wcb + ((pair * 2 * PBK) / cb_block) * 16); };
        // Dequantise K step x (x % 4 == XM) into its ring tile, then refill x's nibble slot with step x + 4 and,
        // after the second step of a pair, the pair's codebook slot with the pair after next.
        auto produce = [&](int x, auto xm) {
            constexpr int XM = decltype(xm)::value;
            const uint4 mine = cbh[(XM >> 1) & 1];
            uint4 oth;
            oth.x = dpp_u<0xB1>(mine.x);  // quad_perm [1,0,3,2]: the pair partner's half
            oth.y = dpp_u<0xB1>(mine.y);
            oth.z = dpp_u<0xB1>(mine.z);
            oth.w = dpp_u<0xB1>(mine.w);
            if (wt) {
                uint8_t* wb = lds + (x % (2 * BS)) * L::w;
                const CbPlanes pl = wh ? cb_planes(oth, mine) : cb_planes(mine, oth);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    *(half8*)(wb + pf_off(wn, 4 * wh + i)) = lookup8_natural(u4get(nv[XM], i), pl);
            }
            load_n(min(x + PW, steps - 1), XM);
            if (XM & 1) load_c(min((x >> 1) + 2, pairs - 1), (XM >> 1) & 1);
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
#pragma unroll
        for (int u = 0; u < PW; ++u) load_n(min(u, steps - 1), u);
        load_c(0, 0);
        load_c(min(1, pairs - 1), 1);
        produce(0, I0{});
        if constexpr (BS >= 2) produce(1, I1{});
        if constexpr (BS >= 4) {
            produce(2, I2{});
            produce(3, I3{});
        }
        __syncthreads();
        for (int s0 = 0; s0 < steps; s0 += 4) {
            // steps s0 + BS .. s0 + 3 + BS while the consumers run s0 .. s0 + 3 (tiles of steps >= steps are unused)
            produce(s0 + BS, std::integral_constant<int, BS % 4>{});
            if constexpr (BS == 1) __syncthreads();
            produce(s0 + 1 + BS, std::integral_constant<int, (1 + BS) % 4>{});
            if constexpr (BS <= 2) __syncthreads();
            produce(s0 + 2 + BS, std::integral_constant<int, (2 + BS) % 4>{});
            if constexpr (BS == 1) __syncthreads();
            produce(s0 + 3 + BS, std::integral_constant<int, (3 + BS) % 4>{});
            __syncthreads();
        }
        __syncthreads();  // consumers stage C
    } else {
        // ---------------- consumers ----------------
        const int kc32 = K / 32;
        const int g0 = (m0 >> 4) + NG * wave, gmax = ((M + 15) >> 4) - 1;
        const half8* af16 = (const half8*)A16 + lane;
        half8 af[PA][NG][2];
        auto load_a = [&](int step, int b) {
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                const int g = min(g0 + i, gmax);
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) af[b][i][kk] = af16[((int64_t)g * kc32 + 2 * step + kk) * 64];
            }
        };
        floatx4 acc[NG][NT];
#pragma unroll
        for (int i = 0; i < NG; ++i)
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < PA - 1; ++u) load_a(min(u, steps - 1), u);
        __syncthreads();
        for (int s0 = 0; s0 < steps; s0 += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int step = s0 + u;
                const uint8_t* cur = lds + (step % (2 * BS)) * L::w;
                load_a(min(step + PA - 1, steps - 1), (u + PA - 1) % PA);  // into the set of A(step - 1)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    half8 bfr[NT];
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        bfr[j] = *(const half8*)(cur + pf_off(16 * j + (lane & 15), 4 * kk + (lane >> 4)));
#pragma unroll
                    for (int i = 0; i < NG; ++i)
#pragma unroll
                        for (int j = 0; j < NT; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[u % PA][i][kk], bfr[j], acc[i][j], 0,
                                                                               0, 0);
                }
                if ((u + 1) % BS == 0) __syncthreads();
            }
        }
        __syncthreads();
        if constexpr (X32) {
            float* st = (float*)lds;
#pragma unroll
            for (int i = 0; i < NG; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rr = 16 * NG * wave + 16 * i + 4 * (lane >> 4) + r;
#pragma unroll
                    for (int j = 0; j < NT; ++j) st[rr * BN + 16 * j + (lane & 15)] = acc[i][j][r];
                }
        } else {
            uint16_t* st = (uint16_t*)lds;
            // the rows' shifts loaded together (each load behind the bf16 rounding's branches waited alone)
            int shv[NG][4];
#pragma unroll
            for (int i = 0; i < NG; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) shv[i][r] = rsh[min(m0 + 16 * NG * wave + 16 * i + 4 * (lane >> 4) + r, M - 1)];
#pragma unroll
            for (int i = 0; i < NG; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rr = 16 * NG * wave + 16 * i + 4 * (lane >> 4) + r;
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        st[rr * BN + 16 * j + (lane & 15)] = f32_to_bf16_rne(ldexpf(acc[i][j][r], -shv[i][r]));
                }
        }
    }
    __syncthreads();
    if constexpr (X32) {
        // real row 128 mt + r: (hi sum + lo sum) * 2^-shift
        float* C = (float*)Cv;
        const float* st = (const float*)lds;
        constexpr int CPR = BN / 4, IT = (128 * CPR + NTH - 1) / NTH;
        int shv[IT];  // the rows' shifts loaded together
#pragma unroll
        for (int it = 0; it < IT; ++it) shv[it] = rsh[min(128 * mt + min((tid + it * NTH) / CPR, 127), Mr - 1)];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int c = tid + it * NTH;
            if (c >= 128 * CPR) break;
            const int r = c / CPR, q = c % CPR, row = 128 * mt + r;
            if (row < Mr) {
                const int sh = shv[it];
                const float4 hi = *(const float4*)(st + r * BN + 4 * q), lo = *(const float4*)(st + (r + 128) * BN + 4 * q);
                // oil4_hi_lo: an infinite hi sum (an infinite codebook entry) is the result, as the reference's
                // single product w * x_k gives, not hi + lo, which is NaN where the lo part has the other sign
                *(float4*)(C + (int64_t)row * N + n0 + 4 * q) =
                    make_float4(ldexpf(oil4_hi_lo(hi.x, lo.x), -sh), ldexpf(oil4_hi_lo(hi.y, lo.y), -sh),
                                ldexpf(oil4_hi_lo(hi.z, lo.z), -sh), ldexpf(oil4_hi_lo(hi.w, lo.w), -sh));
            }
        }
    } else {
        uint16_t* C = (uint16_t*)Cv;
        const uint16_t* st = (const uint16_t*)lds;
        constexpr int CPR = BN * 2 / 16;
        for (int c = tid; c < 256 * CPR; c += NTH) {
            const int r = c / CPR, q = c % CPR;
            if (m0 + r < M) *(uint4*)(C + (int64_t)(m0 + r) * N + n0 + 8 * q) = *(const uint4*)(st + r * BN + 8 * q);
        }
    }
}

// FP32 rows of A as FP16 hi / lo fragments for oil4_prefill_ws<X32> and
// oil8_prefill_ws: one workgroup per real row r (XCD-grouped as
// oil4_prefill_a16): the row's maximum gives its shift (rsh[r], max|a| 2^s in
// [2^14, 2^15); 0 for an all-zero row; kRowNonFinite for a row holding Inf /
// NaN, converted with s = 0: its hi / lo parts then carry NaN, and the OIL8
// GEMM's workgroups over such a row take the FP32 path); a 2^s = hi + lo,
// hi = fp16(a 2^s), lo = fp16(a 2^s - hi), hi into virtual row
// 256 (r / 128) + r % 128, lo 128 rows below it.  Virtual rows of real rows
// past the last (Mr) hold zeros.
__global__ __launch_bounds__(256) void oil4_prefill_a16x(const float* __restrict__ a, uint16_t* __restrict__ a16,
                                                         int Mr, int K, int* __restrict__ rsh, int cover) {
    __shared__ uint32_t red[4];
    const int w = blockIdx.x, tid = threadIdx.x;
    const int g = 8 * (w >> 7) + (w & 7), i = (w >> 3) & 15;
    const int row = 16 * g + i;
    if (row >= cover) return;
    const bool real = row < Mr;
    const float* p = a + (int64_t)(real ? row : 0) * K;
    const int nch = K / 8;
    uint32_t mb = 0;
    if (real)
        for (int c = tid; c < nch; c += 256) {
            const float4 v0 = ldf4(p + 8 * c), v1 = ldf4(p + 8 * c + 4);
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) mb = max(mb, __float_as_uint(v[e]) & 0x7fffffffu);
        }
    mb = group_reduce<64>(mb, UMaxOp{});
    if ((tid & 63) == 0) red[tid >> 6] = mb;
    __syncthreads();
    const uint32_t rmax = max(max(red[0], red[1]), max(red[2], red[3]));
    const int sh = fp16_scale_shift(__uint_as_float(rmax));
    if (tid == 0 && real) rsh[row] = rmax >= 0x7f800000u ? kRowNonFinite : sh;
    const int kc32 = K / 32;
    const int vr = 256 * (row >> 7) + (row & 127);  // virtual row of the hi part; lo: vr + 128
    uint16_t* dh = a16 + (int64_t)(vr >> 4) * kc32 * 512 + 8 * (vr & 15);
    uint16_t* dl = a16 + (int64_t)((vr + 128) >> 4) * kc32 * 512 + 8 * (vr & 15);
    for (int c = tid; c < nch; c += 256) {
        half8 h, l;
        if (real) {
            const float4 v0 = ldf4(p + 8 * c), v1 = ldf4(p + 8 * c + 4);
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xs = ldexpf(v[e], sh);
                h[e] = (_Float16)xs;
                l[e] = (_Float16)(xs - (float)h[e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = l[e] = (_Float16)0.0f;
        }
        const int64_t off = (int64_t)(c >> 2) * 512 + 128 * (c & 3);
        *(half8*)(dh + off) = h;
        *(half8*)(dl + off) = l;
    }
}

// BN of oil4_prefill_ws for N (N % BN == 0), best fill of 256 CUs, or 0
inline int pick_bn_v2(int64_t M, int64_t N) {
    const int cand[4] = {128, 112, 96, 64};
    int best = 0;
    double beff = -1.0;
    for (int bn : cand) {
        if (N % bn) continue;
        const int64_t tiles = (N / bn) * ((M + PBM - 1) / PBM);
        const double eff = (double)tiles / (double)(((tiles + 255) / 256) * 256);
        if (eff > beff + 1e-9) {
            beff = eff;
            best = bn;
        }
    }
    return best;
}

// BN with the best fill of 256 CUs (ties: the larger tile)
inline int pick_bn(int64_t M, int64_t N) {
    const int cand[3] = {128, 112, 96};
    int best = 128;
    double beff = -1.0;
    for (int bn : cand) {
        const int64_t tiles = ((N + bn - 1) / bn) * ((M + PBM - 1) / PBM);
        const int64_t rounds = (tiles + 255) / 256;
        const double eff = (double)tiles / (double)(rounds * 256) * ((double)N / (double)(((N + bn - 1) / bn) * bn));
        if (eff > beff + 1e-9) {
            beff = eff;
            best = bn;
        }
    }
    return best;
}

}  // namespace

// oil4_prefill_ws serves K % 256 == 0, codebook blocks of a multiple of 128 and an N that one of the tile widths
// divides; the workspace is A in FP16 fragment order (ceil(M / 16) * 16 rows)
size_t oil4_prefill_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t cb_block) {
    const bool v2 = K % (4 * PBK) == 0 && cb_block % (2 * PBK) == 0 && pick_bn_v2(M, N) != 0 && M < (1ll << 31) &&
                    ((M + PBM - 1) / PBM) * (N / 64) < (1ll << 31) && M * K < (1ll << 40);
    return v2 ? (size_t)(((M + 15) / 16) * 16 * K * 2) : 0;
}

size_t oil4_prefill_shift_bytes(int64_t M) { return (size_t)((M * 4 + 255) / 256 * 256); }

static void launch_rowshift(const uint16_t* a_bf16, int* rsh, int64_t M, int64_t K, hipStream_t s) {
    oil4_prefill_rowshift<<<(unsigned)M, 256, 0, s>>>(a_bf16, rsh, (int)M, (int)K);
}

hipError_t launch_oil4_gemm_prefill_a16(const uint16_t* a_bf16, const uint8_t* nib, const uint16_t* cbs,
                                        int64_t cb_block, uint16_t* c_bf16, int64_t M, int64_t N, int64_t K,
                                        void* ws, hipStream_t s) {
    int* rsh = (int*)ws;
    uint16_t* a16 = (uint16_t*)((char*)ws + oil4_prefill_shift_bytes(M));
    const int64_t groups = (M + 15) / 16;
    oil4_prefill_a16<<<(unsigned)(((groups + 7) / 8) * 128), 256, 0, s>>>(a_bf16, a16, (int)M, (int)K, rsh);
    const int bn = pick_bn_v2(M, N);
    const unsigned grid = (unsigned)(((M + PBM - 1) / PBM) * (N / bn));
    const int cbk = (int)cb_block, m = (int)M, n = (int)N, k = (int)K;
    constexpr int T4 = ws_threads(4);
    switch (bn) {
        case 128: oil4_prefill_ws<128, 2, 1><<<grid, T4, 0, s>>>(a16, nib, cbs, cbk, c_bf16, m, n, k, rsh); break;
        case 112: oil4_prefill_ws<112, 4, 2><<<grid, T4, 0, s>>>(a16, nib, cbs, cbk, c_bf16, m, n, k, rsh); break;
        case 96: oil4_prefill_ws<96, 4, 2><<<grid, T4, 0, s>>>(a16, nib, cbs, cbk, c_bf16, m, n, k, rsh); break;
        default: oil4_prefill_ws<64, 4, 2><<<grid, T4, 0, s>>>(a16, nib, cbs, cbk, c_bf16, m, n, k, rsh); break;
    }
    return hipGetLastError();
}

hipError_t launch_prefill_a16x(const float* a, int64_t Mr, int64_t K, void* ws, hipStream_t s, int64_t cover) {
    if (cover == 0) cover = (Mr + 127) / 128 * 128;
    if (cover < Mr || cover % 128 != 0) return hipErrorInvalidValue;
    int* rsh = (int*)ws;
    uint16_t* a16 = (uint16_t*)((char*)ws + oil4_prefill_shift_bytes(Mr));
    // one workgroup per real row of the covered rows (rows past Mr write zeros)
    oil4_prefill_a16x<<<(unsigned)cover, 256, 0, s>>>(a, a16, (int)Mr, (int)K, rsh, (int)cover);
    return hipGetLastError();
}

bool oil4_gemm_x32_supported(int64_t Mr, int64_t N, int64_t K, int64_t cb_block) {
    const int64_t mv = 256 * ((Mr + 127) / 128);
    return Mr >= 1 && cb_block > 0 && oil4_prefill_workspace_bytes(mv, N, K, cb_block) != 0 && K <= (1 << 20);
}

size_t oil4_gemm_x32_workspace_bytes(int64_t Mr, int64_t K) {
    const int64_t mv = 256 * ((Mr + 127) / 128);
    return oil4_prefill_shift_bytes(Mr) + (size_t)(mv * K * 2);
}

hipError_t launch_oil4_gemm_x32(const float* a, const uint8_t* nib, const uint16_t* cbs, int64_t cb_block, float* c,
                                int64_t Mr, int64_t N, int64_t K, void* ws, hipStream_t s) {
    if (!oil4_gemm_x32_supported(Mr, N, K, cb_block)) return hipErrorInvalidValue;
    const hipError_t e = launch_prefill_a16x(a, Mr, K, ws, s);
    if (e != hipSuccess) return e;
    const int* rsh = (const int*)ws;
    const uint16_t* a16 = (const uint16_t*)((const char*)ws + oil4_prefill_shift_bytes(Mr));
    const int64_t tiles = (Mr + 127) / 128, mv = 256 * tiles;
    // 128-column tiles whenever they fill a round of 256 CUs: they halve the
    // A fragment loads per product and the W tile is dequantised for twice the
    // columns per barrier (measured at 1024 rows x 22016 x 4096: 528 -> 461 us
    // against the best-fill 64-column tiles), on 8 consumer waves of 32 rows
    // (two per SIMD: one issues MFMAs while the other waits; 468 -> 434 us;
    // at config 4's 512 x 14336 x 4096 they measured slower, 70 -> 73-78 us)
    const int bn = (N % 128 == 0 && tiles * (N / 128) >= 256) ? 128 : pick_bn_v2(mv, N);
    const unsigned grid = (unsigned)(tiles * (N / bn));
    const int cbk = (int)cb_block, m = (int)mv, n = (int)N, k = (int)K, mr = (int)Mr;
    constexpr int T4 = ws_threads(4);
    switch (bn) {
        case 128:
            oil4_prefill_ws<128, 4, 1, true, 8><<<grid, ws_threads(8), 0, s>>>(a16, nib, cbs, cbk, c, m, n, k, rsh, mr);
            break;
        case 112: oil4_prefill_ws<112, 4, 2, true><<<grid, T4, 0, s>>>(a16, nib, cbs, cbk, c, m, n, k, rsh, mr); break;
        case 96: oil4_prefill_ws<96, 4, 2, true><<<grid, T4, 0, s>>>(a16, nib, cbs, cbk, c, m, n, k, rsh, mr); break;
        default: oil4_prefill_ws<64, 4, 2, true><<<grid, T4, 0, s>>>(a16, nib, cbs, cbk, c, m, n, k, rsh, mr); break;
    }
    return hipGetLastError();
}

bool oil4_gemm_prefill_supported(int64_t M, int64_t N, int64_t K, int64_t cb_block) {
    return K % BK == 0 && cb_block % BK == 0 && M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) &&
           (M + BM - 1) / BM < 65536;
}

hipError_t launch_oil4_gemm_prefill(const uint16_t* a_bf16, const uint8_t* nib, const uint16_t* cbs,
                                    int64_t cb_block, uint16_t* c_bf16, int64_t M, int64_t N, int64_t K,
                                    int* rsh, hipStream_t s) {
    launch_rowshift(a_bf16, rsh, M, K, s);
    if (K % (4 * PBK) == 0 && cb_block % PBK == 0 && (M + PBM - 1) / PBM < 65536) {
        const int bn = pick_bn(M, N);
        const dim3 g2((unsigned)((N + bn - 1) / bn), (unsigned)((M + PBM - 1) / PBM));
        if (bn == 112)
            oil4_prefill_mfma<112><<<g2, 256, 0, s>>>(a_bf16, nib, cbs, (int)cb_block, c_bf16, (int)M, (int)N, (int)K,
                                           rsh);
        else if (bn == 96)
            oil4_prefill_mfma<96><<<g2, 256, 0, s>>>(a_bf16, nib, cbs, (int)cb_block, c_bf16, (int)M, (int)N, (int)K,
                                           rsh);
        else
            oil4_prefill_mfma<128><<<g2, 256, 0, s>>>(a_bf16, nib, cbs, (int)cb_block, c_bf16, (int)M, (int)N, (int)K,
                                           rsh);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    oil4_gemm_prefill_k<<<grid, 256, 0, s>>>(a_bf16, nib, cbs, (int)cb_block, c_bf16, (int)M, (int)N, (int)K, rsh);
    return hipGetLastError();
}

}  // namespace mth
