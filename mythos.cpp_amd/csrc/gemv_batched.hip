// gemv_batched.hip — OIL4 and OIL8 GEMVs for decode batches of 2..16 tokens
// on gfx950 (the OIL8 kernel is described at its definition).
//
//   y[t][m] = sum_k cb[m][k/128][nib(m, k)] * x[t][k]   (t < batch <= 16)
//
// the per-token definition of src/kernel_oil4.cpp:31-54 with per-128-weight
// codebooks, weights shared by the batch.  Dequantised weights are the A
// operand of v_mfma_f32_16x16x32_f16 (16 rows, weight path in
// oil4_common.h); the B operand is 16 tokens.  Each token is split into FP16
// hi + lo parts after a power-of-two scale per (token, phase), and two MFMAs
// (B = hi parts, B = lo parts) share every A, so the sums are FP32-accurate
// as for batch 1.
//
// Tiling.  Workgroup = 4 waves x 16 rows = 64 rows and one K slice of
// NPH x 256 columns; grid = (ceil(M / 64), K / (256 NPH)).  The slice's x for
// 16 tokens is loaded once per workgroup, converted phase by phase into a
// double-buffered B area in LDS by all 256 threads and shared by the four
// waves (so the conversion costs a quarter of what a per-wave copy would).
// With more than one slice, each workgroup writes its partial sums to the
// workspace and a second kernel adds the slices in the order 0, 1, ... and
// writes y: deterministic, and the kernel boundary orders the data.  (A
// device-scope fence inside the kernel compiles to a writeback and an
// invalidation of the whole L2 of the XCD, per workgroup — far slower.)
#include "common.h"
#include "launch.h"
#include "oil4_common.h"

namespace mth {
namespace {

constexpr int kBtRows = 64;  // rows per workgroup: 4 waves x 16
constexpr int kBtTok = 16;   // tokens per launch (B columns)

template <int NPH, bool SHARED>
struct Oil4BtLds {
    static constexpr int frag = 8 * 4 * kBtTok * 16;  // B of one phase: 8 MFMAs x 4 groups x 16 tokens x 16 B
    static constexpr int buf = 2 * frag;              // hi, lo
    static constexpr int stage = 2 * buf;             // double-buffered B, then the codebook stages
    static constexpr int shifts = stage + (SHARED ? 0 : 4 * 2048);
    static constexpr int bytes = shifts + 2 * kBtTok * 4;
};

// B fragment (MFMA m, group q, token n) of one phase: 16-byte slots, tokens
// XOR-permuted per (m, q) so that both the 16 lanes reading one (m, q) and
// the 16 threads writing one token hit distinct banks.
__device__ __forceinline__ int bt_slot(int m, int q, int n) {
    const int mq = m * 4 + q;
    return (mq * kBtTok + (n ^ (mq & 15))) * 16;
}

template <int NPH, bool SHARED>
__global__ __launch_bounds__(256) void oil4_gemv_bt(const uint8_t* nib, const uint16_t* cbs,
                                                    const float* __restrict__ x, float* __restrict__ y,
                                                    float* __restrict__ partial, int M, int K, int batch) {
    using L = Oil4BtLds<NPH, SHARED>;
    constexpr int KS = NPH * 256;  // columns per slice
    __shared__ __align__(16) uint8_t lds[L::bytes];
    int* shifts = (int*)(lds + L::shifts);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, q = lane >> 4;
    const int row0 = blockIdx.x * kBtRows;
    const int row0w = row0 + 16 * wave;
    const int ks = blockIdx.y * KS;
    const int nslice = gridDim.y;

    // ---- x of the slice: thread T -> token T/16, columns 16(T%16)+0..15 of
    // each phase; tokens >= batch read token 0 and use zeros.  Issued before
    // the weight stream (loads return in issue order).
    const int tt = tid >> 4, u = tid & 15;
    const bool tok = tt < batch;
    const float* xr = x + (int64_t)(tok ? tt : 0) * K + ks + 16 * u;
    float4 xq[NPH][4];
#pragma unroll
    for (int p = 0; p < NPH; ++p)
#pragma unroll
        for (int i = 0; i < 4; ++i) xq[p][i] = ldf4(xr + 256 * p + 4 * i);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    Oil4TileLoads<NPH, SHARED> w;
    w.issue(nib, cbs, row0w, M, K, ks, lane);
    CbPlanes shared_planes;
    if (SHARED) shared_planes = cb_planes(ld16(cbs), ld16(cbs + 8));
    uint8_t* stage = lds + L::stage + (SHARED ? 0 : wave * 2048);

    floatx4 ysum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int p = 0; p < NPH; ++p) {
        uint8_t* bbuf = lds + (p & 1) * L::buf;
        // ---- this phase's x -> per-token power-of-two scale -> FP16 hi/lo
        {
            float xv[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xv[4 * i] = tok ? xq[p][i].x : 0.0f; xv[4 * i + 1] = tok ? xq[p][i].y : 0.0f;
                xv[4 * i + 2] = tok ? xq[p][i].z : 0.0f; xv[4 * i + 3] = tok ? xq[p][i].w : 0.0f;
            }
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(xv[i]));
            const int sh = fp16_scale_shift(row16_max(mx));  // the 16 threads of token tt form one DPP row
            if (u == 0) shifts[(p & 1) * kBtTok + tt] = sh;
            const int qq = u >> 2;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int m = 2 * (u & 3) + h;
                half8 vh, vl;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float xs = ldexpf(xv[8 * h + oil4_elem_col(e)], sh);
                    const _Float16 hh = (_Float16)xs;
                    vh[e] = hh;
                    vl[e] = (_Float16)(xs - (float)hh);
                }
                *(half8*)(bbuf + bt_slot(m, qq, tt)) = vh;
                *(half8*)(bbuf + L::frag + bt_slot(m, qq, tt)) = vl;
            }
        }
        __syncthreads();  // B of phase p complete; the other buffer is free again after this phase

        const CbPlanes pl = SHARED ? shared_planes : w.planes(p, stage, lane);
        uint4 xa, yb;
        w.exchange(p, lane, xa, yb);
        // hi and lo parts in separate accumulators (combined by oil4_hi_lo)
        floatx4 acc_h = {0.0f, 0.0f, 0.0f, 0.0f}, acc_l = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const half8 a = lookup8(m < 4 ? u4get(xa, m) : u4get(yb, m - 4), pl);
            const half8 bh = *(const half8*)(bbuf + bt_slot(m, q, j));
            const half8 bl = *(const half8*)(bbuf + L::frag + bt_slot(m, q, j));
            acc_h = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh, acc_h, 0, 0, 0);
            acc_l = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl, acc_l, 0, 0, 0);
        }
        // D[4q+i][n] of token n = j, in units of 2^sh(n)
        const int shn = shifts[(p & 1) * kBtTok + j];
#pragma unroll
        for (int i = 0; i < 4; ++i) ysum[i] += ldexpf(oil4_hi_lo(acc_h[i], acc_l[i]), -shn);
    }

    // ---- output: rows row0w + 4q + i, token j ----
    if (nslice == 1) {
        if (j < batch)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (row0w + 4 * q + i < M) y[(int64_t)j * M + row0w + 4 * q + i] = ysum[i];
        return;
    }
    if (j < batch)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (row0w + 4 * q + i < M)
                partial[((int64_t)blockIdx.y * kBtTok + j) * M + row0w + 4 * q + i] = ysum[i];
}

// y[t][m] = sum over slices z = 0, 1, ... of partial[z][t][m]; all loads
// are issued before the first add (at most 16 slices).
__global__ __launch_bounds__(256) void oil4_bt_reduce(const float* __restrict__ partial, float* __restrict__ y,
                                                      int M, int batch, int nslice) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)batch * M) return;
    const int64_t t = i / M, m = i - t * M;
    const float* p = partial + t * M + m;
    const int64_t zs = (int64_t)kBtTok * M;
    float v[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) v[z] = z < nslice ? p[z * zs] : 0.0f;
    float s = v[0];
#pragma unroll
    for (int z = 1; z < 16; ++z)
        if (z < nslice) s += v[z];
    y[i] = s;
}

// oil4_bt_reduce of a gate/up projection (rows [0, F) the gate, [F, 2F) the
// up) with the SwiGLU after it (the decode step of a batch): the same sums,
// then act[t * lda + i] = silu(g * ni) * (u * ni) (ni: the RMSNorm's 1 / rms
// from ns, in norm_scale<16>'s order; ns.ssp null: 1) -- the activations of
// silu_mul_quant_k bit for bit -- and per workgroup the maximum of |act|
// over its 256 columns in amax[t][blockIdx.x] for the down projection's
// quantisation.  act may be the gate half of the input itself (partial ==
// act, lda == 2F, one slice): each thread writes only the element it alone
// has read.  grid (ceil(F / 256), batch).
__global__ __launch_bounds__(256) void oil4_bt_swiglu_reduce(const float* partial, NormScale ns, float* act,
                                                             int64_t lda, float* __restrict__ amax, int F,
                                                             int nslice) {
    __shared__ double nred[16];
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = blockIdx.y, i = blockIdx.x * 256 + tid, M = 2 * F;
    const int ic = i < F ? i : F - 1;
    // the norm's partial sums (four of norm_scale<16>'s waves per wave)
    double np4[4];
    if (ns.ssp) {
        const int last = ns.nparts - 1;
#pragma unroll
        for (int v = 0; v < 4; ++v) np4[v] = last >= 0 ? ns.ssp[(int64_t)t * ns.nparts + min((wave + 4 * v) * 64 + lane, last)] : 0.0;
    }
    const float* pg = partial + (int64_t)t * M + ic;
    const int64_t zs = (int64_t)kBtTok * M;
    float vg[16], vu[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) {
        vg[z] = z < nslice ? pg[z * zs] : 0.0f;
        vu[z] = z < nslice ? pg[z * zs + F] : 0.0f;
    }
    float g = vg[0], u = vu[0];
#pragma unroll
    for (int z = 1; z < 16; ++z)
        if (z < nslice) {
            g += vg[z];
            u += vu[z];
        }
    if (ns.ssp) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int vt = (wave + 4 * v) * 64 + lane;
            double a = vt < ns.nparts ? np4[v] : 0.0;
            for (int k = vt + 1024; k < ns.nparts; k += 1024) a += ns.ssp[(int64_t)t * ns.nparts + k];
            a = wave_sum_dbl(a);
            if (lane == 0) nred[wave + 4 * v] = a;
        }
        __syncthreads();
        double sum = 0.0;
#pragma unroll
        for (int w = 0; w < 16; ++w) sum += nred[w];
        const float ni = (float)(1.0 / sqrt(sum / (double)ns.dim + (double)ns.eps));
        g *= ni;
        u *= ni;
    }
    const float a = silu1(g) * u;
    if (i < F) act[(int64_t)t * lda + i] = a;
    float m = i < F ? fabsf(a) : 0.0f;
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    if (tid == 0) amax[(int64_t)t * gridDim.x + blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

inline int ceil_div_i(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// ===================================================================
// OIL8, batch 2..16, on FP16 MFMA (three products per weight block)
// ===================================================================
//   y[t][m] = sum_k cb[idx[m][k]] * x[t][k]
// The codebook is scaled by 2^sw (max|cb| 2^sw < 2^15) and each entry split
// into FP16 hi + lo parts, c 2^sw = ch + cl; each token's activations of the
// K slice alike with its own 2^sx, x 2^sx = xh + xl.  Every residual is
// below 2^-22 of the value, every FP16 product is exact in FP32, and
//   D = Ah Bh + Ah Bl + Al Bh          (v_mfma_f32_16x16x32_f16, FP32 sums)
// leaves out only Al Bl (2^-22 of the product), so D 2^-(sw+sx) is the FP32
// dot product to FP32 accuracy.  Three FP16 MFMAs cost a sixth of the
// sixteen FP32 MFMAs (v_mfma_f32_16x16x4_f32) the same 512 products take.
//
// Tiling.  Workgroup = WV waves x NT tiles of 16 rows, one K slice of
// 128 PH columns.  Per 128-column phase a wave loads each tile in two
// 128-byte-per-row instructions (rows 0-7, rows 8-15, 8 lanes per row) and
// a DPP row rotation hands lane (j = l % 16, q = l / 16) the 32 index bytes
// of row j at columns 32q .. 32q + 31; MFMA m takes bytes 8m .. 8m + 7 as
// its A column group q (k order 32q + 8m + e on both operands).  The
// 256-entry table of (hi, lo) pairs sits in LDS (one ds_read_b32 gather per
// weight gives both parts); the slice's activations for 16 tokens are
// converted once into hi / lo B fragments in LDS (8 KB per phase) and read
// by all waves, so the main loop has no barrier.  Every load is issued up
// front, activations of all waves before any weights (see the kernel).
// Slices (grid.y) write partial sums that oil8_seg_reduce adds in slice
// order (deterministic).
//
// Non-finite values.  Inf cannot be split (Inf - Inf is NaN), so a
// workgroup whose codebook or activations hold a non-finite value computes
// its outputs with FP32 FMAs over the reference's products in column order
// instead (a uniform branch; same outputs up to the summation order).
constexpr int kH3Tok = 16;
constexpr int kH3Hdr = 1280;   // table (1 KB), token maxima, wave maxima
constexpr int kH3Phase = 8192; // B of one 128-column phase: hi 4 KB, then lo 4 KB

// B slot (MFMA m, column group q, token n): 16 bytes, tokens XOR-permuted
// per (m, q) so that the 16 threads storing one token and the 16 lanes
// reading one (m, q) both hit distinct banks.
__device__ __forceinline__ int h3_slot(int m, int q, int n) {
    const int mq = m * 4 + q;
    return (mq * kH3Tok + (n ^ mq)) * 16;
}

// lane (j, q) <- row j, pieces 2q (a) and 2q + 1 (b) of a 16-row tile loaded
// as wx (rows 0-7) and wy (rows 8-15), lane (j, q) holding piece 2q + j/8
// of row j % 8 (see Oil4TileLoads::exchange)
__device__ __forceinline__ void h3_exchange(const uint4& wx, const uint4& wy, int lane, uint4& a, uint4& b) {
    const bool keep = (lane & 15) < 8;
    const uint32_t ry0 = dpp_ror8(wy.x), ry1 = dpp_ror8(wy.y), ry2 = dpp_ror8(wy.z), ry3 = dpp_ror8(wy.w);
    const uint32_t rx0 = dpp_ror8(wx.x), rx1 = dpp_ror8(wx.y), rx2 = dpp_ror8(wx.z), rx3 = dpp_ror8(wx.w);
    a = make_uint4(keep ? wx.x : ry0, keep ? wx.y : ry1, keep ? wx.z : ry2, keep ? wx.w : ry3);
    b = make_uint4(keep ? rx0 : wy.x, keep ? rx1 : wy.y, keep ? rx2 : wy.z, keep ? rx3 : wy.w);
}

__device__ __forceinline__ uint32_t h3_pair(float c) {
    const _Float16 h = (_Float16)c;
    const _Float16 l = (_Float16)(c - (float)h);
    return (uint32_t)__builtin_bit_cast(uint16_t, h) | ((uint32_t)__builtin_bit_cast(uint16_t, l) << 16);
}

template <int WV, int NT, int PH>
__global__ __launch_bounds__(WV * 64) void oil8_gemv_h3(Oil8SegArgs sg, const float* x, float* __restrict__ partial,
                                                        int K, int batch) {
    constexpr int KS = 128 * PH;
    constexpr int XG = WV / 4;          // thread groups of 256; phase p is converted by group p % XG
    constexpr int XP = PH / XG;         // phases converted per thread
    static_assert(PH % XG == 0, "phases split over the thread groups");
    __shared__ __align__(16) uint8_t lds[kH3Hdr + PH * kH3Phase];
    uint32_t* tab = (uint32_t*)lds;
    float* tmax = (float*)(lds + 1024);          // [XG][16] token maxima
    float* wmax = (float*)(lds + 1024 + 4 * 2 * kH3Tok);
    uint8_t* bsm = lds + kH3Hdr;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, q = lane >> 4, jj8 = j & 7, hi8 = j >> 3;
    const int sgi = seg_of_group(sg, blockIdx.x);
    const uint8_t* idx = sg.idx[sgi];
    const int M = sg.rows[sgi];
    const int row0w = (blockIdx.x - sg.g0[sgi]) * (WV * 16 * NT) + wave * 16 * NT;
    const int k0 = blockIdx.y * KS;

    // ---- loads.  The CU returns loads in issue order, across its waves: so
    // every wave first issues the small operands (its codebook entry and the
    // activations it converts: token tt, columns 8u .. 8u+7 of the phases
    // p = xg, xg + XG, ...), and only after a barrier the weights, phase by
    // phase with a barrier between phases.  The activations then arrive
    // ahead of the weight stream and are converted while it streams, and
    // each phase's MFMAs wait only for that phase.
    const int tt = (tid >> 4) & 15, u = tid & 15, xg = tid >> 8;
    const bool tok = tt < batch;
    const float* xr = x + (int64_t)(tok ? tt : 0) * K + k0 + 8 * u;
    const float cbv = sg.cb[sgi][tid & 255];
    float4 xa[XP], xb[XP];
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        xa[i] = ldf4(xr + 128 * (XG * i + xg));
        xb[i] = ldf4(xr + 128 * (XG * i + xg) + 4);
    }
    const uint8_t* px[NT];
    const uint8_t* py[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        px[t] = idx + (int64_t)min(row0w + 16 * t + jj8, M - 1) * K + k0 + 16 * (2 * q + hi8);
        py[t] = idx + (int64_t)min(row0w + 16 * t + 8 + jj8, M - 1) * K + k0 + 16 * (2 * q + hi8);
    }
    // Phase 0 before the activations' conversion, the others after it: the phase-0 weights of every
    // workgroup on the CU then come back before any workgroup's later phases (4096 x 4096 at 16 tokens:
    // 11.39 -> 10.75 us against every phase here; decode batch 16 +3.7 %).
    uint4 wx[NT][PH], wy[NT][PH];
    constexpr int PF = 1;
    auto issue = [&](int p) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            wx[t][p] = ld_stream(px[t] + 128 * p);
            wy[t][p] = ld_stream(py[t] + 128 * p);
        }
    };
#pragma unroll
    for (int p = 0; p < PF; ++p) issue(p);
    __builtin_amdgcn_sched_barrier(0);

    // ---- scales: token max over the slice (16 threads of one DPP row per
    // phase group, then the groups through LDS), codebook max over the first
    // 256 threads; any non-finite value -> FMA path
    float xm = 0.0f;
    bool fin = __builtin_isfinite(cbv);
    if (tok) {
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const float v[8] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w, xb[i].x, xb[i].y, xb[i].z, xb[i].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                xm = fmaxf(xm, fabsf(v[e]));
                fin = fin && __builtin_isfinite(v[e]);
            }
        }
    }
    xm = row16_max(xm);
    const float cm = wave_max(fabsf(cbv));
    if (wave < 4 && lane == 0) wmax[wave] = cm;
    if (u == 0) tmax[xg * kH3Tok + tt] = xm;
    const bool special = __syncthreads_or(!fin) != 0;

    auto token_shift = [&](int n) {
        float m = tmax[n];
#pragma unroll
        for (int g = 1; g < XG; ++g) m = fmaxf(m, tmax[g * kH3Tok + n]);
        return fp16_scale_shift(m);
    };
    floatx4 ysum[NT];
    if (!special) {
        const int sw = fp16_scale_shift(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
        if (tid < 256) tab[tid] = h3_pair(ldexpf(cbv, sw));
        const int sx = token_shift(tt);
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int p = XG * i + xg;
            const float v[8] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w, xb[i].x, xb[i].y, xb[i].z, xb[i].w};
            half8 vh, vl;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xs = tok ? ldexpf(v[e], sx) : 0.0f;
                const _Float16 h = (_Float16)xs;
                vh[e] = h;
                vl[e] = (_Float16)(xs - (float)h);
            }
            uint8_t* bp = bsm + p * kH3Phase + h3_slot(u & 3, u >> 2, tt);
            *(half8*)bp = vh;
            *(half8*)(bp + 4096) = vl;
        }
        __syncthreads();
#pragma unroll
        for (int p = PF; p < PH; ++p) issue(p);
        __builtin_amdgcn_sched_barrier(0);

        floatx4 acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int p = 0; p < PH; ++p) {
            uint4 a[NT], b[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) h3_exchange(wx[t][p], wy[t][p], lane, a[t], b[t]);
            const uint8_t* bp = bsm + p * kH3Phase;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const half8 bh = *(const half8*)(bp + h3_slot(m, q, j));
                const half8 bl = *(const half8*)(bp + 4096 + h3_slot(m, q, j));
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const uint32_t w0 = m == 0 ? a[t].x : m == 1 ? a[t].z : m == 2 ? b[t].x : b[t].z;
                    const uint32_t w1 = m == 0 ? a[t].y : m == 1 ? a[t].w : m == 2 ? b[t].y : b[t].w;
                    uint32_t gv[8];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        gv[e] = tab[(w0 >> (8 * e)) & 0xffu];
                        gv[4 + e] = tab[(w1 >> (8 * e)) & 0xffu];
                    }
                    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
                    u32x4v ah, al;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        ah[d] = __builtin_amdgcn_perm(gv[2 * d + 1], gv[2 * d], 0x05040100u);
                        al[d] = __builtin_amdgcn_perm(gv[2 * d + 1], gv[2 * d], 0x07060302u);
                    }
                    const half8 Ah = __builtin_bit_cast(half8, ah), Al = __builtin_bit_cast(half8, al);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, bh, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, bl, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, bh, acc[t], 0, 0, 0);
                }
            }
        }
        const int un = sw + token_shift(j);
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) ysum[t][i] = ldexpf(acc[t][i], -un);
    }

    if (special) {
        // a non-finite codebook entry or activation: FP32 FMAs over the
        // slice's columns in order instead (rows 4q + i, token j)
        const float* cb = sg.cb[sgi];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = row0w + 16 * t + 4 * q + i;
                float sum = 0.0f;
                if (j < batch && row < M) {
                    const uint8_t* wr = idx + (int64_t)row * K + k0;
                    const float* xx = x + (int64_t)j * K + k0;
                    for (int k = 0; k < KS; ++k) sum = fmaf(cb[wr[k]], xx[k], sum);
                }
                ysum[t][i] = sum;
            }
    }

    // ---- D[4q + i][j]: rows row0w + 16t + 4q + i of token j, consecutive in
    // y and in the partial layout [slice][token][rows]: one 16-byte store
    // where all four rows exist and the address is aligned
    if (j >= batch) return;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int row = row0w + 16 * t + 4 * q;
        if (row >= M) continue;
        float* dst = gridDim.y == 1 ? sg.y[sgi] + (int64_t)j * M + row
                                    : partial + ((int64_t)blockIdx.y * kH3Tok + j) * sg.mtot + sg.off[sgi] + row;
        const float4 v = make_float4(ysum[t][0], ysum[t][1], ysum[t][2], ysum[t][3]);
        if (row + 3 < M && ((uintptr_t)dst & 15u) == 0) {
            *(float4*)dst = v;
        } else {
            dst[0] = v.x;
            if (row + 1 < M) dst[1] = v.y;
            if (row + 2 < M) dst[2] = v.z;
            if (row + 3 < M) dst[3] = v.w;
        }
    }
}

// y of segment s, token t, row r = sum over slices z = 0, 1, ... of
// partial[z][t][off[s] + r] (slice order: deterministic).
__global__ __launch_bounds__(256) void oil8_seg_reduce(const float* __restrict__ partial, Oil8SegArgs sg, int batch,
                                                       int nslice) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)batch * sg.mtot) return;
    const int t = (int)(i / sg.mtot), r = (int)(i - (int64_t)t * sg.mtot);
    const int s = seg_of_row(sg, r);
    const float* p = partial + (int64_t)t * sg.mtot + r;
    const int64_t zs = (int64_t)kH3Tok * sg.mtot;
    float sum = p[0];
    for (int z0 = 1; z0 < nslice; z0 += 8) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = z0 + e < nslice ? p[(z0 + e) * zs] : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (z0 + e < nslice) sum += v[e];
    }
    sg.y[s][(int64_t)t * sg.rows[s] + (r - sg.off[s])] = sum;
}

// phases of 128 columns per K slice
inline int h3_phases(int64_t K) { return K % 512 == 0 ? 4 : (K % 256 == 0 ? 2 : 1); }

template <int WV, int NT, int PH>
void run_h3(const Oil8Seg* seg, int nseg, const float* x, int64_t K, int b, float* partial, bool reduce,
            hipStream_t s) {
    const Oil8SegArgs a = make_seg_args(seg, nseg, WV * 16 * NT);
    const int S = (int)(K / (128 * PH));
    const dim3 grid((unsigned)seg_groups(seg, nseg, WV * 16 * NT), (unsigned)S);
    oil8_gemv_h3<WV, NT, PH><<<grid, WV * 64, 0, s>>>(a, x, partial, (int)K, b);
    if (S > 1 && reduce) oil8_seg_reduce<<<ceil_div_i((int64_t)b * a.mtot, 256), 256, 0, s>>>(partial, a, b, S);
}

// 8 waves (128 rows) share one activation staging where the phases split
// over two thread groups
void h3_dispatch(const Oil8Seg* seg, int nseg, const float* x, int64_t K, int b, float* partial, bool reduce,
                 hipStream_t s) {
    const int ph = h3_phases(K);
    if (ph == 4) run_h3<8, 1, 4>(seg, nseg, x, K, b, partial, reduce, s);
    else if (ph == 2) run_h3<8, 1, 2>(seg, nseg, x, K, b, partial, reduce, s);
    else run_h3<4, 1, 1>(seg, nseg, x, K, b, partial, reduce, s);
}

// ===================================================================
// OIL4, batch 2..16, per-128-column codebooks: persistent workgroups
// ===================================================================
// The arithmetic of oil4_gemv_bt (same A and B fragments, same hi/lo MFMA
// pair, same per-(token, phase) scale), organised so that the activations
// are converted once per workgroup and the weight stream overlaps the
// dequantisation:
//   * about one 8-wave workgroup per CU.  Workgroup b owns K slice
//     z = b % S (NPH phases of 256 columns) and the 16-row tiles [t0, t1)
//     of share p = b / S; it converts the slice's activations for 16 tokens
//     into hi / lo B fragments in LDS once and uses them for all its tiles;
//   * its waves walk the (tile, phase) units of the range in tile-major
//     order, wave w the contiguous run [w NU / A, (w + 1) NU / A) of the
//     NU = (t1 - t0) NPH units (A = active waves), so runs differ by at
//     most one unit;
//   * each wave keeps kBpDepth units of weight loads in flight in a
//     register ring, refilled as a unit is consumed;
//   * a tile's sum is the sum of its runs' parts: the part of the run that
//     covers its phase 0 goes to LDS slot 0, the other (if any) to slot 1,
//     and the tile's result is slot 0 + slot 1 (fixed order:
//     deterministic).  Runs are at least NPH units long (A = min(8, tiles)),
//     so no tile has more than two parts.
// Slices write partial sums for oil4_bt_reduce (or the consumer) as before.
constexpr int kBpMaxTiles = 24;  // 16-row tiles per workgroup (LDS sums)
constexpr int kBpDepth = 4;      // units in flight per wave
constexpr int kBpCUs = 256;      // MI355X

template <int NPH, int WV>
struct BpLds {
    static constexpr int frag = Oil4BtLds<NPH, false>::frag;  // B of one phase, hi or lo (8 KB)
    static constexpr int bphase = 2 * frag;
    static constexpr int stage = NPH * bphase;                // codebook stage: 2 KB per wave
    static constexpr int sums = stage + WV * 2048;            // [tile][slot][token][row] f32
    static constexpr int dummy = sums + kBpMaxTiles * 2 * 1024;  // 1 KB, shared: stores between tiles
    static constexpr int shifts = dummy + 1024;
    static constexpr int bytes = shifts + NPH * kBtTok * 4;
};

// Weight loads of one unit: 16 rows x 256 columns starting at column kcol
// (two 8-row x 128-byte nibble reads), and the codebooks of the unit's phase
// pair (two 8-row x 128-byte reads), in the layout of Oil4TileLoads.
struct BpSlot {
    uint4 c0, c1, wx, wy;
};

// Per-lane byte offsets of those reads from the tile's first row; rows past
// M read row M - 1 (lim = M - 1 - row0 >= 15 for a full tile).
struct BpOff {
    uint32_t c0, c1, wx, wy;
};

__device__ __forceinline__ BpOff bp_off(int lim, int K, int lane) {
    const int j = lane & 15, q = lane >> 4, jj8 = j & 7, hi8 = j >> 3;
    const uint32_t hk = (uint32_t)K >> 1, cbr = (uint32_t)K >> 2;  // row bytes: nibbles, codebooks
    BpOff o;
    o.c0 = (uint32_t)min(lane >> 3, lim) * cbr + 16 * (lane & 7);
    o.c1 = (uint32_t)min(8 + (lane >> 3), lim) * cbr + 16 * (lane & 7);
    o.wx = (uint32_t)min(jj8, lim) * hk + 16 * (2 * q + hi8);
    o.wy = (uint32_t)min(8 + jj8, lim) * hk + 16 * (2 * q + hi8);
    return o;
}

// The tile base is uniform (scalar registers), the lane offsets 32-bit.
__device__ __forceinline__ void bp_issue(BpSlot& s, const uint8_t* nib, const uint16_t* cbs, int row0, int K,
                                         int kcol, const BpOff& o) {
    const uint8_t* nb = nib + (int64_t)row0 * (K >> 1) + (kcol >> 1);
    const uint8_t* cb = (const uint8_t*)cbs + (int64_t)row0 * (K >> 2) + (int64_t)((kcol >> 7) & ~3) * 32;
    s.c0 = ld16(cb + o.c0);
    s.c1 = ld16(cb + o.c1);
    s.wx = ld_stream(nb + o.wx);
    s.wy = ld_stream(nb + o.wy);
}

template <int NPH, int WV>
__global__ __launch_bounds__(WV * 64) void oil4_gemv_bp(const uint8_t* nib, const uint16_t* cbs,
                                                              const float* __restrict__ x, float* __restrict__ y,
                                                              float* __restrict__ partial, int M, int K, int batch,
                                                              int tiles, int per_slice) {
    using L = BpLds<NPH, WV>;
    static_assert(WV >= 8, "the first 8 waves convert the activations");
    __shared__ __align__(16) uint8_t lds[L::bytes];
    int* shifts = (int*)(lds + L::shifts);
    float* sums = (float*)(lds + L::sums);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, q = lane >> 4;
    const int S = K / (256 * NPH);
    const int z = blockIdx.x % S, p = blockIdx.x / S;
    const int t0 = (int)((int64_t)p * tiles / per_slice), t1 = (int)((int64_t)(p + 1) * tiles / per_slice);
    const int nt = t1 - t0;
    if (nt <= 0) return;  // uniform, before any barrier
    const int k0 = z * 256 * NPH;

    // ---- activations of the slice first (loads return in issue order):
    // thread of the first 8 waves -> token tt, 16-column group u, phases
    // hp, hp + 2, ...
    constexpr int XPH = NPH / 2;
    const bool conv = wave < 8;  // uniform
    const int tt = (tid >> 4) & 15, u = tid & 15, hp = (tid >> 8) & 1;
    const bool tok = tt < batch;
    const float* xr = x + (int64_t)(tok ? tt : 0) * K + k0 + 16 * u;
    float4 xq[XPH][4];
    if (conv) {
#pragma unroll
        for (int e = 0; e < XPH; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i) xq[e][i] = ldf4(xr + 256 * (hp + 2 * e) + 4 * i);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // ---- this wave's run; the first kBpDepth units' loads
    const int NU = nt * NPH, act = min(WV, nt);
    const int u0 = wave < act ? (int)((int64_t)wave * NU / act) : NU;
    const int u1 = wave < act ? (int)((int64_t)(wave + 1) * NU / act) : NU;
    const int ulast = u0 < u1 ? u1 - 1 : 0;  // loads past the run repeat its last unit (cache hits)
    const BpOff ofull = bp_off(15, K, lane), olast = bp_off(M - 1 - (tiles - 1) * 16, K, lane);
    auto issue = [&](BpSlot& sl, int uu) {
        const int t = t0 + uu / NPH;
        const bool last = t == tiles - 1;  // uniform
        BpOff o;
        o.c0 = last ? olast.c0 : ofull.c0; o.c1 = last ? olast.c1 : ofull.c1;
        o.wx = last ? olast.wx : ofull.wx; o.wy = last ? olast.wy : ofull.wy;
        bp_issue(sl, nib, cbs, t * 16, K, k0 + 256 * (uu % NPH), o);
    };
    BpSlot ring[kBpDepth];
#pragma unroll
    for (int s = 0; s < kBpDepth; ++s) issue(ring[s], min(u0 + s, ulast));
    __builtin_amdgcn_sched_barrier(0);

    // ---- B fragments of the slice (the conversion of oil4_gemv_bt)
#pragma unroll
    for (int e = 0; e < (conv ? XPH : 0); ++e) {
        const int ph = hp + 2 * e;
        uint8_t* bbuf = lds + ph * L::bphase;
        float xv[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xv[4 * i] = tok ? xq[e][i].x : 0.0f; xv[4 * i + 1] = tok ? xq[e][i].y : 0.0f;
            xv[4 * i + 2] = tok ? xq[e][i].z : 0.0f; xv[4 * i + 3] = tok ? xq[e][i].w : 0.0f;
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(xv[i]));
        const int sh = fp16_scale_shift(row16_max(mx));  // the 16 threads of one (token, phase): one DPP row
        if (u == 0) shifts[ph * kBtTok + tt] = sh;
        const int qq = u >> 2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int m = 2 * (u & 3) + h;
            half8 vh, vl;
#pragma unroll
            for (int e2 = 0; e2 < 8; ++e2) {
                const float xs = ldexpf(xv[8 * h + oil4_elem_col(e2)], sh);
                const _Float16 hh = (_Float16)xs;
                vh[e2] = hh;
                vl[e2] = (_Float16)(xs - (float)hh);
            }
            *(half8*)(bbuf + bt_slot(m, qq, tt)) = vh;
            *(half8*)(bbuf + L::frag + bt_slot(m, qq, tt)) = vl;
        }
    }
    for (int i = tid; i < nt * 256; i += WV * 64) sums[(i >> 8) * 512 + 256 + (i & 255)] = 0.0f;  // slot 1
    __syncthreads();

    // ---- the run.  One unit: codebooks of the phase pair -> wave stage ->
    // the block of this lane's columns; 8 x (lookup8, hi and lo MFMA); the
    // phase's sum scaled back; at the end of a tile's part, the part to its
    // LDS slot (between tiles the store goes to the wave's dummy row, so the
    // loop body has no branch).
    uint8_t* stage = lds + L::stage + wave * 2048;
    constexpr int dummy_off = L::dummy / 4;  // in floats
    floatx4 ysum = {0.0f, 0.0f, 0.0f, 0.0f};
    int seg0 = u0 % NPH;  // phase at which the current tile's part began
    auto unit = [&](const BpSlot& sl, int uu) {
        const int ph = uu % NPH;
        *(uint4*)(stage + oil4_stage_off(lane >> 3, lane & 7)) = sl.c0;
        *(uint4*)(stage + oil4_stage_off(8 + (lane >> 3), lane & 7)) = sl.c1;
        const int bi = 2 * (ph & 1) + (q >> 1);
        const uint4 ca = *(const uint4*)(stage + oil4_stage_off(j, 2 * bi));
        const uint4 cb = *(const uint4*)(stage + oil4_stage_off(j, 2 * bi + 1));
        const CbPlanes pl = cb_planes(ca, cb);
        uint4 xa, yb;
        h3_exchange(sl.wx, sl.wy, lane, xa, yb);
        const uint8_t* bbuf = lds + ph * L::bphase;
        floatx4 acc_h = {0.0f, 0.0f, 0.0f, 0.0f}, acc_l = {0.0f, 0.0f, 0.0f, 0.0f};
        // the unit's 16 B fragments read before its lookups (the compiler otherwise reads each pair just
        // before its MFMAs and waits for the LDS round trip eight times per unit; 22016 x 4096 at 16
        // tokens 27.7 -> 26.9 us)
        half8 bh[8], bl[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            bh[m] = *(const half8*)(bbuf + bt_slot(m, q, j));
            bl[m] = *(const half8*)(bbuf + L::frag + bt_slot(m, q, j));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const half8 a = lookup8(m < 4 ? u4get(xa, m) : u4get(yb, m - 4), pl);
            acc_h = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh[m], acc_h, 0, 0, 0);
            acc_l = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl[m], acc_l, 0, 0, 0);
        }
        const int shn = shifts[ph * kBtTok + j];
#pragma unroll
        for (int i = 0; i < 4; ++i) ysum[i] += ldexpf(oil4_hi_lo(acc_h[i], acc_l[i]), -shn);
        // end of this tile's part (uniform); selects as arithmetic on masks so
        // that the compiler keeps the loop body one basic block
        const int bnd = (int)(ph == NPH - 1) | (int)(uu == u1 - 1);
        const int real = (int)(L::sums / 4) + (uu / NPH) * 512 + ((seg0 != 0) << 8);
        const int off = dummy_off + bnd * (real - dummy_off);
        *(floatx4*)((float*)lds + off + j * 16 + 4 * q) = ysum;
        const uint32_t keep = (uint32_t)bnd - 1u;  // 0 at a boundary, all ones otherwise
#pragma unroll
        for (int i = 0; i < 4; ++i) ysum[i] = __uint_as_float(__float_as_uint(ysum[i]) & keep);
        seg0 &= (int)keep;
    };
    const int nfull = (u1 - u0) / kBpDepth;
    int ub = u0;
    for (int it = 0; it < nfull; ++it, ub += kBpDepth) {
#pragma unroll
        for (int s = 0; s < kBpDepth; ++s) {
            unit(ring[s], ub + s);
            issue(ring[s], min(ub + s + kBpDepth, ulast));
        }
    }
    // the last (u1 - u0) % kBpDepth units sit in slots 0, 1, ...
#pragma unroll
    for (int s = 0; s < kBpDepth - 1; ++s)
        if (ub + s < u1) unit(ring[s], ub + s);
    __syncthreads();

    // ---- tile sums: rows (t0 + tile) 16 + r, token tk
    for (int i = tid; i < nt * 256; i += WV * 64) {
        const int tl = i >> 8, tk = (i >> 4) & 15, r = i & 15;
        const int row = (t0 + tl) * 16 + r;
        if (tk < batch && row < M) {
            const float v = sums[tl * 512 + tk * 16 + r] + sums[tl * 512 + 256 + tk * 16 + r];
            if (S == 1) y[(int64_t)tk * M + row] = v;
            else partial[((int64_t)z * kBtTok + tk) * M + row] = v;
        }
    }
}

template <int NPH, int WV = 8>
void run_bp(const uint8_t* nib, const uint16_t* cbs, const float* x, float* y, float* partial, int64_t M, int64_t K,
            int batch, bool reduce, hipStream_t s) {
    const int S = (int)(K / (256 * NPH));
    const int64_t tiles = (M + 15) / 16;
    int64_t per = std::max<int64_t>((kBpCUs + S - 1) / S, (tiles + kBpMaxTiles - 1) / kBpMaxTiles);
    per = std::min<int64_t>(per, tiles);
    oil4_gemv_bp<NPH, WV><<<(unsigned)(S * per), WV * 64, 0, s>>>(nib, cbs, x, y, partial, (int)M, (int)K, batch,
                                                                   (int)tiles, (int)per);
    if (S > 1 && reduce)
        oil4_bt_reduce<<<ceil_div_i((int64_t)batch * M, 256), 256, 0, s>>>(partial, y, (int)M, batch, S);
}

// phases of 256 columns per K slice: 4 (K a multiple of 1024, K >= 2048) or 2
inline int bt_nph(int64_t K) { return (K >= 2048 && K % 1024 == 0) ? 4 : 2; }

template <int NPH, bool SHARED>
void run_bt(const uint8_t* nib, const uint16_t* cbs, const float* x, float* y, float* partial, int64_t M, int64_t K,
            int batch, bool reduce, hipStream_t s) {
    const int nslice = (int)(K / (256 * NPH));
    const dim3 grid(ceil_div_i(M, kBtRows), (unsigned)nslice);
    oil4_gemv_bt<NPH, SHARED><<<grid, 256, 0, s>>>(nib, cbs, x, y, partial, (int)M, (int)K, batch);
    if (nslice > 1 && reduce)
        oil4_bt_reduce<<<ceil_div_i((int64_t)batch * M, 256), 256, 0, s>>>(partial, y, (int)M, batch, nslice);
}

void bt_dispatch(const uint8_t* nib, const uint16_t* cbs, bool sh, const float* x, float* y, float* partial,
                 int64_t M, int64_t K, int b, bool reduce, hipStream_t s) {
    if (bt_nph(K) == 4) {
        if (sh) run_bt<4, true>(nib, cbs, x, y, partial, M, K, b, reduce, s);
        else run_bp<4>(nib, cbs, x, y, partial, M, K, b, reduce, s);
    } else {
        if (sh) run_bt<2, true>(nib, cbs, x, y, partial, M, K, b, reduce, s);
        else run_bp<2>(nib, cbs, x, y, partial, M, K, b, reduce, s);
    }
}

}  // namespace

bool oil4_bt_swiglu_supported(int64_t F, int64_t K, int64_t cb_block, int64_t batch) {
    return batch <= kBtTok && F % 4 == 0 && oil4_bt_supported(2 * F, K, cb_block, batch);
}

int oil4_bt_swiglu_parts(int64_t F) { return ceil_div_i(F, 256); }

hipError_t launch_oil4_gemv_bt_swiglu(const uint8_t* nib, const uint16_t* cbs, int64_t cb_block, const float* x,
                                      const NormScale& ns, float* gu, float* amax, int64_t F, int64_t K,
                                      int64_t batch, float* partial, hipStream_t s) {
    if (!oil4_bt_swiglu_supported(F, K, cb_block, batch)) return hipErrorInvalidValue;
    const int64_t M = 2 * F;
    const int S = (int)(K / (256 * bt_nph(K)));
    bt_dispatch(nib, cbs, cb_block == 0, x, gu, partial, M, K, (int)batch, false, s);
    // one slice: the GEMV wrote gu itself, [token][2F] like a slice of
    // partial; act goes over gu's gate half either way
    oil4_bt_swiglu_reduce<<<dim3((unsigned)oil4_bt_swiglu_parts(F), (unsigned)batch), 256, 0, s>>>(
        S > 1 ? partial : gu, ns, gu, 2 * F, amax, (int)F, S);
    return hipGetLastError();
}

bool oil4_bt_supported(int64_t M, int64_t K, int64_t cb_block, int64_t batch) {
    // K <= 8192 keeps the slice count <= 16 (the reduction kernel's limit)
    // (M * K / 2 < 2^32: the tile loads use 32-bit byte offsets into the nibbles)
    return batch >= 2 && (cb_block == 0 || cb_block == 128) && K >= 512 && K <= 8192 && K % 512 == 0 &&
           M < (1ll << 31) && M * (K / 2) < (1ll << 32);
}

size_t oil4_bt_partial_bytes(int64_t M, int64_t K) {
    const int64_t S = K / (256 * bt_nph(K));
    return S > 1 ? (size_t)(S * kBtTok * M * 4) : 0;
}

bool oil8_bt_supported(int64_t M, int64_t K, int64_t batch) {
    // the kernel takes K, rows and the concatenated row index as int
    return batch >= 2 && K >= 128 && K % 128 == 0 && K < (1ll << 31) && M < (1ll << 31) && M * K < (1ll << 40);
}

size_t oil8_bt_partial_bytes(int64_t M, int64_t K) {
    const int64_t S = K / (128 * h3_phases(K));
    return S > 1 ? (size_t)(S * kH3Tok * M * 4) : 0;
}

bool oil8_bt_segs_fusable(const Oil8Seg* seg, int nseg, int64_t K, int64_t batch) {
    if (nseg < 1 || nseg > kOil8MaxSegs) return false;
    int64_t total = 0;
    for (int i = 0; i < nseg; ++i) {
        if (seg[i].rows < 1 || ((uintptr_t)seg[i].idx & 15u) != 0) return false;
        total += seg[i].rows;
    }
    return oil8_bt_supported(total, K, batch);
}

hipError_t launch_oil8_gemv_bt_segs(const Oil8Seg* seg, int nseg, const float* x, int64_t K, int64_t batch,
                                    float* partial, hipStream_t s) {
    // groups of 16 tokens, one launch each (the weights are read per group)
    for (int64_t t0 = 0; t0 < batch; t0 += kH3Tok) {
        const int b = (int)(batch - t0 < kH3Tok ? batch - t0 : kH3Tok);
        Oil8Seg g[kOil8MaxSegs];
        for (int i = 0; i < nseg; ++i) {
            g[i] = seg[i];
            g[i].y = seg[i].y + t0 * seg[i].rows;
        }
        const float* xg = x + t0 * K;
        h3_dispatch(g, nseg, xg, K, b, partial, true, s);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

int oil8_bt_slices(int64_t K) { return (int)(K / (128 * h3_phases(K))); }

hipError_t launch_oil8_gemv_bt_segs_slices(const Oil8Seg* seg, int nseg, const float* x, int64_t K, int64_t batch,
                                           float* partial, Slices* out, hipStream_t s) {
    h3_dispatch(seg, nseg, x, K, (int)batch, partial, false, s);
    const int S = oil8_bt_slices(K);
    int64_t mtot = 0;
    for (int i = 0; i < nseg; ++i) mtot += seg[i].rows;
    for (int i = 0, off = 0; i < nseg; off += (int)seg[i].rows, ++i)
        out[i] = S == 1 ? plain_slices(seg[i].y, seg[i].rows)
                        : Slices{partial + off, mtot, kH3Tok * mtot, S, 1.0f, nullptr};
    return hipGetLastError();
}

hipError_t launch_oil8_gemv_bt(const uint8_t* idx, const float* cb, const float* x, float* y, int64_t M, int64_t K,
                               int64_t batch, float* partial, hipStream_t s) {
    const Oil8Seg seg{idx, cb, y, M};
    return launch_oil8_gemv_bt_segs(&seg, 1, x, K, batch, partial, s);
}

hipError_t launch_oil4_gemv_bt(const uint8_t* nib, const uint16_t* cbs, int64_t cb_block, const float* x, float* y,
                               int64_t M, int64_t K, int64_t batch, float* partial, hipStream_t s) {
    const bool sh = cb_block == 0;
    // groups of 16 tokens, one launch each (the weights are read per group)
    for (int64_t t0 = 0; t0 < batch; t0 += kBtTok) {
        const int b = (int)(batch - t0 < kBtTok ? batch - t0 : kBtTok);
        bt_dispatch(nib, cbs, sh, x + t0 * K, y + t0 * M, partial, M, K, b, true, s);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace mth
