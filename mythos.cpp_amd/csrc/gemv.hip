// gemv.hip — OIL8 / OIL4 codebook GEMV for decode on gfx950.
//
// Replaces the CPU loops of src/kernel_oil8.cpp:14-71 and
// src/kernel_oil4.cpp:31-125 (reference semantics: sum_k cb[idx]*x[k] in FP32
// with the codebook value exact in FP32).  Weights stay in the reference's
// row-major layout.  The CU's memory pipeline returns loads in issue order, so
// the small operands every wave needs first (x, the codebook) are issued
// before the weight stream and the stream itself is software-pipelined.
//
// OIL8 (oil8_gemv_k):
//   * workgroup = 4 waves x R rows; wave w owns columns [1024w, 1024w+1024),
//     lane l the 16 consecutive indices at 1024w + 16l (one 128-bit load per
//     row), its 16 activations live in VGPRs;
//   * the 256-entry FP32 codebook is staged once per workgroup in LDS and
//     gathered with one ds_read_b32 per weight;
//   * R row sums are reduced across the wave by a transposed butterfly
//     (log2(R) halving steps, then a plain butterfly) and across the 4 waves
//     through LDS in a fixed order (deterministic).
// OIL4 (oil4_gemv_mfma, batch 1):
//   * workgroup = 16 rows; wave w owns K/4 columns in chunks of 128 (one
//     codebook block);  the dequantised weights go straight into the A operand
//     of v_mfma_f32_16x16x32_f16: lane (r = l%16, g = l/16) holds row r,
//     k = 32g + 8i + v of MFMA i, i.e. exactly the 8 nibbles of dword i of its
//     own 16-byte load;
//   * the row's 16 FP16 codebook entries are written into two LDS columns
//     (r and r+16) per wave; a nibble-spread dword gives each gather address
//     with one v_perm_b32 and ds_read_u16_d16[_hi] packs the FP16 values into
//     the MFMA operand registers directly (no conversions);
//   * x is split per wave into FP16 hi + lo parts after a power-of-two scale
//     (x*2^s = hi + lo + O(2^-22)), placed as B columns 0 and 1, so
//     D[:,0] + D[:,1] is the FP32 dot product; products are exact, sums FP32.
//     Only the 8 lanes holding columns 0 and 1 read B from LDS; the other
//     columns hold don't-care values and their outputs are discarded.
// Other shapes (K not a multiple of 16/512, K > 4096, unaligned pointers,
// batched OIL4, codebook blocks that are not multiples of 128, the
// reference's per-(m,n) indexing) run on oil4_gemv_valu or the generic
// one-wave-per-output kernels.
#include "common.h"
#include "launch.h"
#include "oil4_common.h"

namespace mth {
namespace {

constexpr int kWG = 256;
constexpr int kWaves = kWG / MTH_WAVE;


inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }


// v_perm selector building the LDS byte address (byte b of S0 << 8) | S1.byte0
__device__ __forceinline__ uint32_t perm_addr(uint32_t packed, uint32_t lane4, int b) {
    return __builtin_amdgcn_perm(packed, lane4, 0x0c0c0000u | ((uint32_t)(4 + b) << 8));
}

// Transposed reduction of R per-lane values over the 64 lanes (common.h):
// every lane then holds the wave total of row lane / (64/R).
template <int R>
__device__ __forceinline__ float transposed_sum(float (&v)[R], int lane) { return transposed_reduce<R>(v, lane); }

// ===================================================================
// OIL8
// ===================================================================
// Issue order: x and the thread's codebook entry first (a load issued behind
// other waves' weight loads waits for them: the CU returns loads in order),
// then the R rows' index bytes, and only then the table store and the
// barrier, so the weight stream is in flight while the table is staged
// (measured ~1 us earlier than staging first).  The single unreplicated 1 KiB
// table costs ~1.9x a conflict-free gather (gfx950: 3.6 vs 1.9 cycles per
// wave64 ds_read_b32) but needs one store per thread to fill; a 64-copy
// conflict-free table measured no faster (its fill costs what the gathers
// save).
template <int R>
__global__ __launch_bounds__(kWG) __attribute__((amdgpu_waves_per_eu(4, 4)))
void oil8_gemv_k(Oil8SegArgs sg, const float* x, int K, int batch, ResidOut ro) {
    __shared__ float tab[256];
    __shared__ float part[kWaves][R];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kq = wave * 1024 + lane * 16;  // first column of this lane
    const bool act = kq < K;
    const int kl = act ? kq : K - 16;        // clamped: every load below is unconditional
    const int sgi = seg_of_group(sg, blockIdx.x);
    const uint8_t* idx = sg.idx[sgi];
    const float* __restrict__ cb = sg.cb[sgi];
    float* __restrict__ y = sg.y[sgi];
    const int M = sg.rows[sgi];
    const int m0 = (blockIdx.x - sg.g0[sgi]) * R;

    float4 xq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) xq[q] = ldf4(x + kl + 4 * q);
    const float cbv = cb[tid];
    // residual epilogue operands of token 0 (lane r of wave 0: row m0 + r), issued before the weight stream so the
    // epilogue does not wait for a round trip at the end; every lane loads (clamped), no branch around the loads
    const int rrow = min(m0 + (lane % R), M - 1);
    const float* rxp = ro.x ? ro.x : x;
    const float* rgp = ro.x ? ro.gamma : x;
    const float rx0 = rxp[ro.x ? rrow : 0], rg0 = rgp[ro.x ? rrow : 0];
    __builtin_amdgcn_sched_barrier(0);
    uint4 w[R];
    // (32-bit byte offsets from the segment's base: the launchers keep rows * K below 2^32)
#pragma unroll
    for (int r = 0; r < R; ++r) w[r] = ld_stream(idx + ((uint32_t)min(m0 + r, M - 1) * (uint32_t)K + (uint32_t)kl));
    __builtin_amdgcn_sched_barrier(0);
    tab[tid] = cbv;
    __syncthreads();

    for (int t = 0; t < batch; ++t) {
        float xr[16];
        if (t > 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q) xq[q] = ldf4(x + (int64_t)t * K + kl + 4 * q);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = act ? xq[q] : make_float4(0, 0, 0, 0);
            xr[4 * q] = v.x; xr[4 * q + 1] = v.y; xr[4 * q + 2] = v.z; xr[4 * q + 3] = v.w;
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.0f;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t wd = u4get(w[r], d);
#pragma unroll
                for (int b = 0; b < 4; ++b) acc[r] = fmaf(tab[(wd >> (8 * b)) & 0xffu], xr[4 * d + b], acc[r]);
            }
            if (!act) acc[r] = 0.0f;
        }
        const float s = transposed_sum<R>(acc, lane);
        constexpr int L = MTH_WAVE / R;
        if ((lane % L) == 0) part[wave][lane / L] = s;
        __syncthreads();
        if (wave == 0) {
            const bool wr = lane < R && m0 + lane < M;
            const float v = lane < R ? ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane] : 0.0f;
            const int64_t i = (int64_t)t * M + m0 + lane;
            if (!ro.x) {
                if (wr) y[i] = v;
            } else {
                // residual epilogue (ResidOut, common.h): rows of this workgroup
                double sq = 0.0;
                if (wr) {
                    const float r = v + (t == 0 ? rx0 : ro.x[i]);
                    ro.x[i] = r;
                    ro.xg[i] = r * (t == 0 ? rg0 : ro.gamma[m0 + lane]);
                    sq = (double)r * r;
                }
                sq = wave_sum_dbl(sq);
                if (lane == 0) ro.ssp[(int64_t)t * gridDim.x + blockIdx.x] = sq;
            }
        }
        __syncthreads();
    }
}

// Generic: one wave per output element.  Row r uses weights idx + r*K and
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
// OIL4, batch 1, matrix cores
// ===================================================================
// LDS of oil4_gemv_mfma (byte offsets, one static array).  The codebook table
// sits at offset 0, so a gather address is the v_perm result itself: entry e of
// wave w, column c (0..31) is the low half of the dword at
//     ((e*NW/2 + w/2) << 8) | ((w & 1) << 7) | (c << 2).
// Lanes l and l+32 share a column and always read the same row's table; the
// two 32-lane halves of a wave64 access are serviced separately, so gathers
// never conflict.
template <int NW, int NC>
struct Oil4Lds {
    static constexpr int KW = NC * 128;
    static constexpr int tab = 0;
    static constexpr int tab_bytes = 16 * NW * 128;
    // per wave: the hi block (KW halves), 64 bytes of skew, the lo block.  The
    // skew puts hi and lo of one k-group on different banks, so the 8 lanes
    // that read B (columns 0 and 1 of 4 k-groups) hit 32 distinct banks.
    static constexpr int xf = tab_bytes;
    static constexpr int lo_off = KW * 2 + 64;
    static constexpr int xf_wave = lo_off + KW * 2;
    static constexpr int part = xf + NW * xf_wave;
    static constexpr int bytes = part + NW * 16 * 4;
};

template <int NW, int NC, int PD, bool SHARED, bool CB128>
__global__ __launch_bounds__(NW * 64) void oil4_gemv_mfma(const uint8_t* nib, const uint16_t* cbs,
                                                          int cb_block, const float* __restrict__ x,
                                                          float* __restrict__ y, int M, int K) {
    using L = Oil4Lds<NW, NC>;
    constexpr int KW = L::KW;                  // columns per wave
    constexpr int HS = (NW == 8) ? 2 : 1;      // nibble shift leaving room for w/2 in the index byte
    constexpr int NMF = NC * 4;                // MFMAs per wave
    __shared__ __align__(16) uint8_t lds[L::bytes];  // the kernel's only LDS object
    _Float16* xf = (_Float16*)(lds + L::xf);
    float* part = (float*)(lds + L::part);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int row = blockIdx.x * 16 + r;
    const int rowc = min(row, M - 1);  // clamped: all loads are unconditional
    const int k0 = wave * KW;
    const int nb = SHARED ? 1 : K / cb_block;

    // Issue order.  The CU's memory pipeline returns data in issue order, so
    // a load issued behind another wave's HBM stream waits for that stream.
    // Every wave therefore issues its x loads first, a plain s_barrier (no
    // fence: it does not wait for the loads) makes sure the whole workgroup
    // has issued them, and only then are the codebook and nibble streams
    // issued.  nib / cbs are not __restrict__, so these loads stay below.
    const bool xl = lane * 16 < KW;
    float4 xq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) xq[q] = ldf4(x + k0 + (xl ? lane * 16 : 0) + 4 * q);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // The stream is software-pipelined: chunk c + PD is issued before chunk c
    // is consumed.
    uint2 wc[NC];
    uint4 wn[NC];
    const uint16_t* cbrow = cbs + (int64_t)rowc * nb * 16 + 4 * g;
    const uint8_t* nrow = nib + (int64_t)rowc * (K >> 1) + 16 * g;
    auto issue = [&](int c) {
        const int kc = k0 + c * 128;
        const int blk = CB128 ? (kc >> 7) : kc / cb_block;
        const uint16_t* cp = SHARED ? cbs + 4 * g : cbrow + blk * 16;
        wc[c] = *(const uint2*)cp;
        wn[c] = ld_stream(nrow + (kc >> 1));
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int c = 0; c < (PD < NC ? PD : NC); ++c) issue(c);

    // x slice of this wave -> power-of-two scale -> FP16 hi/lo B fragments
    // (wave-private LDS: only the wave's own program order matters)
    _Float16* xw = xf + wave * (L::xf_wave / 2);
    float xv[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        xv[4 * q] = xl ? xq[q].x : 0.0f; xv[4 * q + 1] = xl ? xq[q].y : 0.0f;
        xv[4 * q + 2] = xl ? xq[q].z : 0.0f; xv[4 * q + 3] = xl ? xq[q].w : 0.0f;
    }
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) mx = fmaxf(mx, fabsf(xv[j]));
    mx = wave_max(mx);
    int e = 0;
    if (mx > 0.0f && mx <= 3.0e38f) (void)frexpf(mx, &e);
    const int sh = (mx > 0.0f && mx <= 3.0e38f) ? 15 - e : 0;  // max|x|*2^sh < 2^15
    if (xl) {
        const int c = lane >> 3, gg = (lane & 7) >> 1;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int i = 2 * (lane & 1) + q;
            half8 hi, lo;
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                const float xs = ldexpf(xv[8 * q + v], sh);
                const _Float16 h = (_Float16)xs;
                hi[v] = h;
                lo[v] = (_Float16)(xs - (float)h);
            }
            *(half8*)&xw[((c * 4 + i) * 4 + gg) * 8] = hi;
            *(half8*)&xw[L::lo_off / 2 + ((c * 4 + i) * 4 + gg) * 8] = lo;
        }
    }
    wave_lds_order();

    const int n = lane & 15;
    const uint32_t col4 = ((uint32_t)(wave & 1) << 7) | ((uint32_t)(lane & 31) << 2);
    const uint32_t wmask = 0x01010101u * (uint32_t)(wave >> 1);
    uint32_t* tab = (uint32_t*)lds;
    // B fragment of MFMA m = c*4 + i: column n's block at byte offset m*64;
    // columns >= 2 are zero and only lanes n < 2 read LDS
    const int xb = L::xf + wave * L::xf_wave + (n == 1 ? L::lo_off : 0) + g * 16;

    auto write_table = [&](int c) {
        // row r's entries 4g..4g+3 into columns r and r+16 (fp16 in the low
        // half).  Lanes of odd g write the two copies in the opposite order,
        // so the two k-groups of a 32-lane half store to different banks.
        const uint32_t ev[4] = {wc[c].x, wc[c].x >> 16, wc[c].y, wc[c].y >> 16};
        const int c0 = r + 16 * (g & 1), c1 = r + 16 * (~g & 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int slot = ((4 * g + j) * (NW / 2) + (wave >> 1)) * 64 + (wave & 1) * 32;
            tab[slot + c0] = ev[j];
            tab[slot + c1] = ev[j];
        }
        wave_lds_order();
    };
    struct Frag { half8 a, b; };
    auto gather = [&](int m) {
        const int c = m >> 2, i = m & 3;
        const uint32_t d = u4get(wn[c], i);
        // index bytes e*NW/2 + wave/2 for the even (low) and odd (high) nibbles
        const uint32_t lo4 = ((d << HS) & (0x0f0f0f0fu << HS)) | wmask;
        const uint32_t hi4 = ((d >> (4 - HS)) & (0x0f0f0f0fu << HS)) | wmask;
        Frag f;
#pragma unroll
        for (int v = 0; v < 8; ++v) f.a[v] = *(const _Float16*)(lds + perm_addr((v & 1) ? hi4 : lo4, col4, v >> 1));
        // D column n depends on B column n only, so the unused columns may
        // hold any value: lanes n >= 2 skip the read and keep stale registers.
        half8 b = __builtin_nondeterministic_value(b);
        if (n < 2) b = *(const half8*)(lds + xb + m * 64);
        f.b = b;
        return f;
    };

    // Software-pipelined in source order: the gathers of MFMA m+1 are issued
    // before MFMA m consumes its operands (the compiler tracks the waits).
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    write_table(0);
    Frag cur = gather(0);
#pragma unroll
    for (int m = 0; m < NMF; ++m) {
        Frag nxt;
        if (m + 1 < NMF) {
            if (((m + 1) & 3) == 0) {  // next chunk: prefetch, then its table
                const int c1 = (m + 1) >> 2;
                if (c1 + PD - 1 < NC) issue(c1 + PD - 1);
                write_table(c1);
            }
            nxt = gather(m + 1);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.a, cur.b, acc, 0, 0, 0);
        if (m + 1 < NMF) cur = nxt;
    }
    // D[4g+i][n]: rows' hi (n = 0) + lo (n = 1) parts (oil4_hi_lo)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float s = oil4_hi_lo(acc[i], lane_xor1(acc[i]));
        if (n == 0) part[wave * 16 + 4 * g + i] = ldexpf(s, -sh);
    }
    __syncthreads();
    if (tid < 16 && blockIdx.x * 16 + tid < M) {
        float sum = part[tid];
#pragma unroll
        for (int w = 1; w < NW; ++w) sum += part[w * 16 + tid];
        y[blockIdx.x * 16 + tid] = sum;
    }
}

// ===================================================================
// OIL4, batch 1 (oil4_gemv_v2): 128-byte row runs, v_perm codebook lookups
// ===================================================================
// Workgroup = 16 rows x K; wave w owns columns [w*KW, (w+1)*KW) as NPH phases
// of 256 (weight path: oil4_common.h).  x is split per wave into FP16 hi + lo
// parts after a power-of-two scale (x*2^s = hi + lo + O(2^-22)), placed as B
// columns 0 and 1, so D[:,0] + D[:,1] is the FP32 dot product: products are
// exact, sums FP32.
template <int NW, int NPH, bool SHARED>
struct Oil4V2Lds {
    static constexpr int KW = NPH * 256;             // columns per wave
    static constexpr int lo_off = KW * 2 + 64;       // B: hi block, 64 B skew, lo block
    static constexpr int bwave = lo_off + KW * 2;
    static constexpr int stage = SHARED ? 0 : 2048;  // codebook stage
    static constexpr int per_wave = bwave + stage;
    static constexpr int part = NW * per_wave;
    static constexpr int bytes = part + NW * 16 * 4;
};

// PAIR: the SwiGLU epilogue of the fused gate/up projection (decode batch
// 1).  Weight rows [0, F) are the gate, [F, 2F) the up projection (M = 2F,
// F % 8 == 0, grid F / 8); workgroup t computes gate rows 8t..8t+7 as tile
// rows 0-7 and the matching up rows as tile rows 8-15, then writes
//   act[i] = silu(g_i * ni) * (u_i * ni),  amax[t] = max over its 8 |act|,
// ni: the RMSNorm's 1 / rms (NormScale) with norm_scale<16>'s summation
// order (16 waves of 64 threads, partials i = thread, thread + 1024, ...,
// wave sums, waves in order), g_i and u_i summed as the plain output is:
// act is bit-identical to silu_mul_quant_k's SwiGLU of that output.
struct SwigluTile {
    NormScale ns;
    float* act;
    float* amax;
    int F;
};

template <int NW, int NPH, bool SHARED, bool PAIR = false>
__global__ __launch_bounds__(NW * 64, PAIR && NW >= 4 ? 5 : 1) void oil4_gemv_v2(const uint8_t* nib, const uint16_t* cbs,
                                                        const float* __restrict__ x, float* __restrict__ y,
                                                        int M, int K, SwigluTile sw = SwigluTile{}) {
    using L = Oil4V2Lds<NW, NPH, SHARED>;
    constexpr int KW = L::KW;
    __shared__ __align__(16) uint8_t lds[L::bytes];
    __shared__ double nred[PAIR ? 16 : 1];
    float* part = (float*)(lds + L::part);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, q = lane >> 4;
    const int row0 = blockIdx.x * 16;
    const int k0 = wave * KW;

    // x first (and the norm's partial sums), then (once every wave of the
    // workgroup has issued them) the weight streams: the CU returns loads in
    // issue order.
    // x: KW / 64 values per lane (every lane), XS B-fragment slots of 8
    constexpr int XS = KW / 512;
    static_assert(KW % 512 == 0 && XS >= 1 && XS <= 2, "oil4_gemv_v2: 2 or 4 phases of 256 columns per wave");
    constexpr int VW = PAIR ? (16 + NW - 1) / NW : 1;  // norm_scale<16> waves taken by this wave
    double np1[VW];
    if (PAIR && sw.ns.ssp) {
        const int last = sw.ns.nparts - 1;
#pragma unroll
        for (int i = 0; i < VW; ++i)
            np1[i] = last >= 0 ? sw.ns.ssp[min((wave + i * NW) * 64 + lane, last)] : 0.0;
    }
    float4 xq[2 * XS];
#pragma unroll
    for (int i = 0; i < 2 * XS; ++i) xq[i] = ldf4(x + k0 + lane * 8 * XS + 4 * i);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    Oil4TileLoads<NPH, SHARED> w;
    const int rowA = PAIR ? blockIdx.x * 8 : row0, rowB = PAIR ? sw.F + blockIdx.x * 8 : row0 + 8;
    // Phase 0's weights (and its phase pair's codebooks) now, the other phases' after the x conversion: a CU
    // returns loads in issue order, so the phase-0 data of every workgroup on the CU comes back before any
    // workgroup's later phases and each wave computes phase 0 while the rest streams in (11008 x 4096:
    // 11.08 -> 10.40 us against issuing every phase here; after phase 0's products instead: 11.01 us).
    w.template issue_phases<0, 1>(nib, cbs, rowA, rowB, M, K, k0, lane);
    CbPlanes shared_planes;
    if (SHARED) shared_planes = cb_planes(ld16(cbs), ld16(cbs + 8));
    // (PAIR) norm_scale<16>'s wave sums of this wave's virtual waves, before
    // the x conversion, so that the partials' registers are free at its peak
    if (PAIR && sw.ns.ssp) {
#pragma unroll
        for (int i = 0; i < VW; ++i) {
            const int vw = wave + i * NW, vt = vw * 64 + lane;
            double t = vt < sw.ns.nparts ? np1[i] : 0.0;
            for (int k = vt + 1024; k < sw.ns.nparts; k += 1024) t += sw.ns.ssp[k];
            t = wave_sum_dbl(t);
            if (lane == 0 && vw < 16) nred[vw] = t;
        }
    }

    // ---- x slice -> power-of-two scale -> FP16 hi/lo B fragments --------
    // lane l holds columns 8 XS l .. 8 XS l + 8 XS - 1; slot s of them starts
    // at column c0 = 8 (XS l + s): phase c0 / 256, group (c0 % 256) / 64,
    // MFMA (c0 % 64) / 8.  max|x| is taken over the magnitudes' bit patterns
    // (no NaN canonicalisation; a NaN, above every finite pattern, gives
    // shift 0, and the output is NaN either way).
    uint8_t* wl = lds + wave * L::per_wave;
    _Float16* xw = (_Float16*)wl;
    float xv[8 * XS];
#pragma unroll
    for (int i = 0; i < 2 * XS; ++i) {
        xv[4 * i] = xq[i].x, xv[4 * i + 1] = xq[i].y, xv[4 * i + 2] = xq[i].z, xv[4 * i + 3] = xq[i].w;
    }
    uint32_t mb = 0, mn = 0xffffffffu;  // max |x| bits; min nonzero |x| bits - 1 (0 -> all ones)
#pragma unroll
    for (int i = 0; i < 8 * XS; ++i) {
        const uint32_t ab = __float_as_uint(xv[i]) & 0x7fffffffu;
        mb = max(mb, ab);
        mn = min(mn, ab - 1u);
    }
    const uint32_t wmax = group_reduce<64>(mb, UMaxOp{});
    const int sh = fp16_scale_shift(__uint_as_float(wmax));  // max|x|*2^sh < 2^15
    // A nonzero x_k more than 2^28 below max|x| (binade difference > 28) has
    // an FP16 hi part that is subnormal or 0: its product keeps fewer than 11
    // bits, and an infinite codebook entry times a hi part of 0 gives NaN
    // where the reference's w * x_k is +-Inf (src/kernel_oil4.cpp:50).  Such a
    // wave (also any wave whose x slice holds Inf or NaN) recomputes its rows
    // with FP32 products below.
    const bool lossy = __builtin_amdgcn_ballot_w64(
                           mn != 0xffffffffu && (int)(wmax >> 23) - (int)((mn + 1u) >> 23) > 28) != 0;
#pragma unroll
    for (int h = 0; h < XS; ++h) {
        const int c0 = 8 * (XS * lane + h);
        const int p = c0 >> 8, qq = (c0 & 255) >> 6, m = (c0 & 63) >> 3;
        half8 vh, vl;
        // two columns per conversion (v_cvt_pk_f16_f32, round to nearest even as the scalar conversion)
        typedef _Float16 h2v __attribute__((ext_vector_type(2)));
        typedef float f2v __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int t = 0; t < 8; t += 2) {
            const f2v xs = {ldexpf(xv[8 * h + oil4_elem_col(t)], sh), ldexpf(xv[8 * h + oil4_elem_col(t + 1)], sh)};
            const h2v hh = __builtin_convertvector(xs, h2v);
            const h2v ll = __builtin_convertvector(f2v{xs[0] - (float)hh[0], xs[1] - (float)hh[1]}, h2v);
            vh[t] = hh[0], vh[t + 1] = hh[1];
            vl[t] = ll[0], vl[t + 1] = ll[1];
        }
        const int slot = ((p * 8 + m) * 4 + qq) * 8;
        *(half8*)&xw[slot] = vh;
        *(half8*)&xw[L::lo_off / 2 + slot] = vl;
    }
    wave_lds_order();
    __builtin_amdgcn_sched_barrier(0);  // no weight-data wait above this point
    if constexpr (NPH > 1) {
        w.template issue_phases<1, NPH>(nib, cbs, rowA, rowB, M, K, k0, lane);
        __builtin_amdgcn_sched_barrier(0);
    }

    // B of MFMA (p, m): column 0 = hi, column 1 = lo; D column n depends on B
    // column n only, so the other columns repeat them and are discarded.
    const int xb = ((j & 1) ? L::lo_off : 0) + q * 16;
    auto bfrag = [&](int pm) { return *(const half8*)(wl + xb + pm * 64); };

    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    half8 bnext = bfrag(0);
#pragma unroll
    for (int p = 0; p < NPH; ++p) {
        const CbPlanes pl = SHARED ? shared_planes : w.planes(p, wl + L::bwave, lane);
        uint4 xa, yb;
        w.exchange(p, lane, xa, yb);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int pm = p * 8 + m;
            const half8 b = bnext;
            if (pm + 1 < NPH * 8) bnext = bfrag(pm + 1);  // one MFMA ahead
            const half8 a = lookup8(m < 4 ? u4get(xa, m) : u4get(yb, m - 4), pl);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
        }
    }
    // D[4q+i][n]: rows' hi (n = 0) + lo (n = 1) parts (oil4_hi_lo)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float s = oil4_hi_lo(acc[i], lane_xor1(acc[i]));
        if (j == 0) part[wave * 16 + 4 * q + i] = ldexpf(s, -sh);
    }
    if (lossy) {
        // the wave's 16 rows again with FP32 products (the reference's
        // arithmetic): lane l takes columns 8 XS l .. of each row, the lanes'
        // sums are added across the wave
        const int nbr = K >> 7;
        for (int r = 0; r < 16; ++r) {
            const int row = PAIR ? (r < 8 ? blockIdx.x * 8 + r : sw.F + blockIdx.x * 8 + r - 8) : min(row0 + r, M - 1);
            float sum = 0.0f;
#pragma unroll
            for (int h = 0; h < XS; ++h) {
                const int c0 = k0 + 8 * (XS * lane + h);
                const uint32_t d = *(const uint32_t*)(nib + (int64_t)row * (K >> 1) + (c0 >> 1));
                const uint16_t* cb = SHARED ? cbs : cbs + ((int64_t)row * nbr + (c0 >> 7)) * 16;
                const half8 wv = lookup8(d, cb_planes(ld16(cb), ld16(cb + 8)));
                const float4 x0 = ldf4(x + c0), x1 = ldf4(x + c0 + 4);
                const float xf[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int t = 0; t < 8; ++t) sum = fmaf((float)wv[t], xf[oil4_elem_col(t)], sum);
            }
            sum = group_reduce<64>(sum, AddOp{});
            if (lane == 0) part[wave * 16 + r] = sum;
        }
    }
    __syncthreads();
    if (PAIR) {
        if (tid < 8) {
            float g = part[tid], u = part[8 + tid];
#pragma unroll
            for (int w2 = 1; w2 < NW; ++w2) {
                g += part[w2 * 16 + tid];
                u += part[w2 * 16 + 8 + tid];
            }
            if (sw.ns.ssp) {
                double t = 0.0;
#pragma unroll
                for (int v = 0; v < 16; ++v) t += nred[v];
                const float ni = (float)(1.0 / sqrt(t / (double)sw.ns.dim + (double)sw.ns.eps));
                g *= ni;
                u *= ni;
            }
            const float a = silu1(g) * u;
            sw.act[blockIdx.x * 8 + tid] = a;
            const float m = group_reduce<8>(fabsf(a), MaxOp{});  // lanes 0-7, all active
            if (tid == 0) sw.amax[blockIdx.x] = m;
        }
        return;
    }
    if (tid < 16 && row0 + tid < M) {
        float sum = part[tid];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) sum += part[w2 * 16 + tid];
        y[row0 + tid] = sum;
    }
}

// ===================================================================
// OIL4, vector-ALU path (batched decode and other block sizes)
// ===================================================================
// 16 bytes of nibbles = 32 weights per segment; element k of a row is the low
// nibble of byte k/2 for even k, the high nibble for odd k.  Each lane writes
// the 16 entries of its segment's codebook (FP32) into a private LDS column.
template <int NSEG, int RG, bool SHARED>
__global__ __launch_bounds__(kWG, 2) void oil4_gemv_valu(
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

    auto load_rows = [&](uint4 (&w)[RG][NSEG], uint4 (&c)[RG][NSEG][2], int rr) {
#pragma unroll
        for (int gi = 0; gi < RG; ++gi)
#pragma unroll
            for (int s = 0; s < NSEG; ++s) {
                const int seg = lane + 64 * s;
                if (rr + gi < r1 && seg < nseg) {
                    w[gi][s] = ld_stream(nib + (int64_t)(rr + gi) * (K >> 1) + (int64_t)seg * 16);
                    if (!SHARED) {
                        const uint16_t* cp = cbs + ((int64_t)(rr + gi) * nb + seg / seg_per_blk) * 16;
                        c[gi][s][0] = ld16(cp);
                        c[gi][s][1] = ld16(cp + 8);
                    }
                } else {
                    w[gi][s] = make_uint4(0, 0, 0, 0);
                    if (!SHARED) c[gi][s][0] = c[gi][s][1] = make_uint4(0, 0, 0, 0);
                }
            }
    };

    uint4 wc[RG][NSEG], cc[RG][NSEG][2];
    load_rows(wc, cc, r0);
    if (SHARED) {
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
        for (int rr = r0; rr < r1; rr += RG) {
            uint4 wn[RG][NSEG], cn[RG][NSEG][2];
            const bool more = rr + RG < r1;
            if (more) load_rows(wn, cn, rr + RG);
            float acc[RG];
#pragma unroll
            for (int gi = 0; gi < RG; ++gi) {
                acc[gi] = 0.0f;
#pragma unroll
                for (int s = 0; s < NSEG; ++s) {
                    if (s == NSEG - 1 && lane + 64 * s >= nseg) continue;
                    if (!SHARED) {
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            const uint32_t wd = u4get(cc[gi][s][e >> 3], (e & 7) >> 1);
                            col[e * 64] = (e & 1) ? h2f_hi(wd) : h2f_lo(wd);
                        }
                    }
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t wd = u4get(wc[gi][s], d);
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const uint32_t e = (wd >> (4 * j)) & 0xfu;
                            acc[gi] = fmaf(col[e * 64], xr[s][8 * d + j], acc[gi]);
                        }
                    }
                }
            }
#pragma unroll
            for (int gi = 0; gi < RG; ++gi) {
                const float v = group_sum<64>(acc[gi]);
                if (lane == 0 && rr + gi < r1) y[(int64_t)t * M + rr + gi] = v;
            }
            if (more) {
#pragma unroll
                for (int gi = 0; gi < RG; ++gi)
#pragma unroll
                    for (int s = 0; s < NSEG; ++s) {
                        wc[gi][s] = wn[gi][s];
                        cc[gi][s][0] = cn[gi][s][0];
                        cc[gi][s][1] = cn[gi][s][1];
                    }
            }
        }
    }
}

// Generic OIL4: one wave per output.  Weight row r starts at byte (r*K)/2
// (the reference's `((m*N+n)*K)/2`), element k uses nibble k%2 of byte k/2 of
// that row.  Codebook: shared (cb_block == 0) or per block of row r.
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

inline int pick_rows_per_wave(int64_t M, int rg) {
    const int64_t target_waves = 256 * 2 * kWaves;
    int64_t rpw = (M + target_waves - 1) / target_waves;
    rpw = ((rpw + rg - 1) / rg) * rg;
    return (int)(rpw < rg ? rg : rpw);
}

#ifndef MTH_OIL4_NW
#define MTH_OIL4_NW 4
#endif
#ifndef MTH_OIL4_PD
#define MTH_OIL4_PD 2
#endif
#ifndef MTH_OIL4_V2_NPH
#define MTH_OIL4_V2_NPH 2
#endif
// oil4_gemv_v2 with NPH phases of 256 columns per wave, K / (256 NPH) waves
template <int NPH, bool SHARED>
bool run_oil4_v2(const uint8_t* nib, const uint16_t* cbs, const float* x, float* y, int64_t M, int64_t K,
                 hipStream_t s) {
    if (K % (256 * NPH)) return false;
    const int grid = ceil_div(M, 16);
    switch (K / (256 * NPH)) {
#define MTH_V2_CASE(NW)                                                                                      \
    case NW:                                                                                                 \
        oil4_gemv_v2<NW, NPH, SHARED><<<grid, NW * 64, 0, s>>>(nib, cbs, x, y, (int)M, (int)K);             \
        return true;
        MTH_V2_CASE(1) MTH_V2_CASE(2) MTH_V2_CASE(3) MTH_V2_CASE(4)
        MTH_V2_CASE(5) MTH_V2_CASE(6) MTH_V2_CASE(7) MTH_V2_CASE(8)
#undef MTH_V2_CASE
        default: return false;
    }
}
template <int NW, int NC>
void run_oil4_mfma(const uint8_t* nib, const uint16_t* cbs, int64_t cb_block, const float* x, float* y, int64_t M,
                   int64_t K, hipStream_t s) {
    constexpr int PD = MTH_OIL4_PD;  // chunks in flight per wave
    const int grid = ceil_div(M, 16);
    if (cb_block == 0)
        oil4_gemv_mfma<NW, NC, PD, true, false><<<grid, NW * 64, 0, s>>>(nib, cbs, 0, x, y, (int)M, (int)K);
    else if (cb_block == 128)
        oil4_gemv_mfma<NW, NC, PD, false, true><<<grid, NW * 64, 0, s>>>(nib, cbs, 128, x, y, (int)M, (int)K);
    else
        oil4_gemv_mfma<NW, NC, PD, false, false><<<grid, NW * 64, 0, s>>>(nib, cbs, (int)cb_block, x, y, (int)M,
                                                                        (int)K);
}

}  // namespace

bool oil4_swiglu_supported(const uint8_t* nib, const uint16_t* cbs, const float* x, int64_t F, int64_t K) {
    // the K range where launch_oil4_gemv runs oil4_gemv_v2 with MTH_OIL4_V2_NPH phases
    constexpr int KP = 256 * MTH_OIL4_V2_NPH;
    return F > 0 && F % 8 == 0 && 2 * F < (1ll << 31) && 2 * F * (K / 2) < (1ll << 32) && K % KP == 0 && K >= 512 &&
           K <= 4096 && aligned16(nib) && aligned16(cbs) && aligned16(x);
}

hipError_t launch_oil4_swiglu(const uint8_t* nib, const uint16_t* cbs, const float* x, const NormScale& ns,
                              float* act, float* amax, int64_t F, int64_t K, hipStream_t s) {
    if (!oil4_swiglu_supported(nib, cbs, x, F, K)) return hipErrorInvalidValue;
    const SwigluTile sw{ns, act, amax, (int)F};
    const int grid = (int)(F / 8);
    constexpr int NPH = MTH_OIL4_V2_NPH;
    switch (K / (256 * NPH)) {
#define MTH_SW_CASE(NW)                                                                                     \
    case NW:                                                                                                \
        oil4_gemv_v2<NW, NPH, false, true><<<grid, NW * 64, 0, s>>>(nib, cbs, x, nullptr, (int)(2 * F),      \
                                                                    (int)K, sw);                            \
        break;
        MTH_SW_CASE(1) MTH_SW_CASE(2) MTH_SW_CASE(3) MTH_SW_CASE(4)
        MTH_SW_CASE(5) MTH_SW_CASE(6) MTH_SW_CASE(7) MTH_SW_CASE(8)
#undef MTH_SW_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_oil8_gemv(const uint8_t* idx, const float* cb, const float* x, float* y,
                            int64_t M, int64_t K, int64_t batch, hipStream_t s) {
    const bool fast = (K % 16 == 0) && K <= 4096 && M * K < (1ll << 32) && aligned16(idx) && aligned16(x);
    if (fast) {
        const Oil8Seg seg{idx, cb, y, M};
        return launch_oil8_gemv_segs(&seg, 1, x, K, batch, s);
    } else {
        oil8_generic<<<ceil_div(M, kWaves), kWG, 0, s>>>(idx, cb, x, y, M, K, 1, batch, M);
    }
    return hipGetLastError();
}

bool oil8_segs_fusable(const Oil8Seg* seg, int nseg, int64_t K) {
    if (nseg < 1 || nseg > kOil8MaxSegs || K % 16 != 0 || K > 4096) return false;
    int64_t total = 0;
    for (int i = 0; i < nseg; ++i) {
        if (seg[i].rows < 1 || seg[i].rows * K >= (1ll << 32) || !aligned16(seg[i].idx)) return false;
        total += seg[i].rows;
    }
    return total < (1ll << 31);
}

hipError_t launch_oil8_gemv_segs(const Oil8Seg* seg, int nseg, const float* x, int64_t K, int64_t batch,
                                 hipStream_t s) {
    for (int i = 0; i < nseg; ++i)  // the kernel's byte offsets into a segment's indices are 32-bit
        if (seg[i].rows * K >= (1ll << 32)) return hipErrorInvalidValue;
    constexpr int R = 4;
    const Oil8SegArgs a = make_seg_args(seg, nseg, R);
    oil8_gemv_k<R><<<seg_groups(seg, nseg, R), kWG, 0, s>>>(a, x, (int)K, (int)batch, ResidOut{});
    return hipGetLastError();
}

hipError_t launch_oil8_gemv_resid(const Oil8Seg& seg, const float* x, int64_t K, const ResidOut& ro, int* nparts,
                                  hipStream_t s) {
    if (seg.rows * K >= (1ll << 32)) return hipErrorInvalidValue;  // 32-bit byte offsets into the indices
    constexpr int R = 4;
    const Oil8SegArgs a = make_seg_args(&seg, 1, R);
    *nparts = seg_groups(&seg, 1, R);
    oil8_gemv_k<R><<<*nparts, kWG, 0, s>>>(a, x, (int)K, 1, ro);
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
    const bool aligned = aligned16(nib) && aligned16(x) && aligned16(cbs);
    // (oil4_gemv_v2's tile loads use 32-bit byte offsets: M * K / 2 < 2^32)
    if (batch == 1 && aligned && M * (K / 2) < (1ll << 32) && (cb_block == 0 || cb_block == 128) && K >= 512 &&
        K <= 4096) {
        constexpr int NPH = MTH_OIL4_V2_NPH;
        bool done = cb_block == 0 ? run_oil4_v2<NPH, true>(nib, cbs, x, y, M, K, s)
                                  : run_oil4_v2<NPH, false>(nib, cbs, x, y, M, K, s);
        if (!done && NPH != 2)
            done = cb_block == 0 ? run_oil4_v2<2, true>(nib, cbs, x, y, M, K, s)
                                 : run_oil4_v2<2, false>(nib, cbs, x, y, M, K, s);
        if (done) return hipGetLastError();
    }
    const bool mfma = batch == 1 && aligned && M < (1ll << 31) && (cb_block == 0 || cb_block % 128 == 0) &&
                      (K == 512 || K == 1024 || K == 2048 || K == 4096);
    if (mfma) {
        // K split over the waves of a workgroup: 8 waves (K/8 columns each)
        // for the long rows, so that ~5 waves per SIMD are in flight
        switch (K) {
            case 512: run_oil4_mfma<4, 1>(nib, cbs, cb_block, x, y, M, K, s); break;
            case 1024: run_oil4_mfma<8, 1>(nib, cbs, cb_block, x, y, M, K, s); break;
            case 2048: run_oil4_mfma<8, 2>(nib, cbs, cb_block, x, y, M, K, s); break;
            default: run_oil4_mfma<MTH_OIL4_NW, 4096 / (128 * MTH_OIL4_NW)>(nib, cbs, cb_block, x, y, M, K, s); break;
        }
        return hipGetLastError();
    }
    const bool valu = (K % 32 == 0) && K <= 4096 && M < (1ll << 31) && aligned && (cb_block == 0 || cb_block % 32 == 0);
    if (valu) {
        constexpr int RG = 2;
        const int rpw = pick_rows_per_wave(M, RG);
        const int grid = ceil_div(ceil_div(M, rpw), kWaves);
        const int nseg = (int)(K / 32);
        const int blk = (int)cb_block;
        if (cb_block == 0) {
            if (nseg <= 64)
                oil4_gemv_valu<1, RG, true><<<grid, kWG, 0, s>>>(nib, cbs, blk, x, y, (int)M, (int)K, (int)batch, rpw);
            else
                oil4_gemv_valu<2, RG, true><<<grid, kWG, 0, s>>>(nib, cbs, blk, x, y, (int)M, (int)K, (int)batch, rpw);
        } else {
            if (nseg <= 64)
                oil4_gemv_valu<1, RG, false><<<grid, kWG, 0, s>>>(nib, cbs, blk, x, y, (int)M, (int)K, (int)batch, rpw);
            else
                oil4_gemv_valu<2, RG, false><<<grid, kWG, 0, s>>>(nib, cbs, blk, x, y, (int)M, (int)K, (int)batch, rpw);
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
