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


inline int ceil_div_i(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// ===================================================================
// OIL8, batch 2..16, on FP32 MFMA (v_mfma_f32_16x16x4_f32)
// ===================================================================
//   y[t][m] = sum_k cb[idx[m][k]] * x[t][k]
// Workgroup = 4 waves x 16 rows and one K slice of ks columns (a multiple of
// 64); grid = (ceil(M / 64), K / ks).  Per 64-column chunk, lane l (row
// r = l % 16, k group g = l / 16) loads the 16 index bytes of its row at
// chunk columns 16g .. 16g + 15 (one 128-bit load), gathers their FP32
// codebook values from LDS and feeds them to 16 MFMAs: in MFMA j the lane's
// A element is W[r][16g + j] and its B element x[t = r][16g + j], i.e. the k
// order inside the chunk is permuted alike on both operands.  Products and
// sums are FP32.  The chunk's x for 16 tokens ([16][64] floats, rows padded
// to 68 floats against bank conflicts) is staged in LDS once per workgroup
// (double buffered) and read by all four waves.  Slices are added by
// oil4_bt_reduce (same [slice][16][M] partial layout).
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kO8Pad = 68;

__global__ __launch_bounds__(256) void oil8_gemv_bt(const uint8_t* idx, const float* __restrict__ cb, const float* x,
                                                    float* __restrict__ y, float* __restrict__ partial, int M, int K,
                                                    int batch, int ks) {
    __shared__ float tab[256];
    __shared__ __align__(16) float xs[2][kBtTok * kO8Pad];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.x * kBtRows + wave * 16;
    const int k0 = blockIdx.y * ks;
    const int nch = ks / 64;
    const uint8_t* wrow = idx + (int64_t)min(m0 + r, M - 1) * K + k0 + 16 * g;  // clamped rows
    const int xt = tid >> 4, xc = (tid & 15) * 4;  // staging: token xt, 4 columns at xc
    const bool xv = xt < batch;
    const float* xrow = x + (int64_t)(xv ? xt : 0) * K + k0 + xc;
    float4 xn = xv ? ldf4(xrow) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    tab[tid] = cb[tid];
    uint4 wn = ld_stream(wrow);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = 0; c < nch; ++c) {
        float* xb = xs[c & 1];
        *(float4*)(xb + xt * kO8Pad + xc) = xn;
        __syncthreads();  // the buffer written two chunks ago has been read by all
        const uint4 w = wn;
        if (c + 1 < nch) {
            wn = ld_stream(wrow + (c + 1) * 64);
            if (xv) xn = ldf4(xrow + (c + 1) * 64);
        }
        const float* xp = xb + r * kO8Pad + 16 * g;
        float4 xb4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) xb4[q] = *(const float4*)(xp + 4 * q);
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float xq[4] = {xb4[q].x, xb4[q].y, xb4[q].z, xb4[q].w};
#pragma unroll
            for (int b = 0; b < 4; ++b)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(tab[(wd[q] >> (8 * b)) & 0xffu], xq[b], acc, 0, 0, 0);
        }
    }
    // D: lane l holds rows 4g + i, token r
    const int t = r;
    if (t >= batch) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * g + i;
        if (m >= M) continue;
        if (gridDim.y == 1)
            y[(int64_t)t * M + m] = acc[i];
        else
            partial[((int64_t)blockIdx.y * kBtTok + t) * M + m] = acc[i];
    }
}

// K slices for the OIL8 batched GEMV: enough workgroups to cover the CUs,
// at most 16, each a multiple of 64 columns.
inline int o8_slices(int64_t M, int64_t K) {
    const int64_t groups = (M + kBtRows - 1) / kBtRows;
    int S = 1;
    while (S < 16 && groups * S < 256 && K % (64 * S * 2) == 0) S *= 2;
    return S;
}

// phases of 256 columns per K slice: 4 (K a multiple of 1024, K >= 2048) or 2
inline int bt_nph(int64_t K) { return (K >= 2048 && K % 1024 == 0) ? 4 : 2; }

template <int NPH, bool SHARED>
void run_bt(const uint8_t* nib, const uint16_t* cbs, const float* x, float* y, float* partial, int64_t M, int64_t K,
            int batch, hipStream_t s) {
    const int nslice = (int)(K / (256 * NPH));
    const dim3 grid(ceil_div_i(M, kBtRows), (unsigned)nslice);
    oil4_gemv_bt<NPH, SHARED><<<grid, 256, 0, s>>>(nib, cbs, x, y, partial, (int)M, (int)K, batch);
    if (nslice > 1)
        oil4_bt_reduce<<<ceil_div_i((int64_t)batch * M, 256), 256, 0, s>>>(partial, y, (int)M, batch, nslice);
}

}  // namespace

bool oil4_bt_supported(int64_t M, int64_t K, int64_t cb_block, int64_t batch) {
    // K <= 8192 keeps the slice count <= 16 (the reduction kernel's limit)
    return batch >= 2 && (cb_block == 0 || cb_block == 128) && K >= 512 && K <= 8192 && K % 512 == 0 &&
           M < (1ll << 31) && M * K < (1ll << 40);
}

size_t oil4_bt_partial_bytes(int64_t M, int64_t K) {
    const int64_t S = K / (256 * bt_nph(K));
    return S > 1 ? (size_t)(S * kBtTok * M * 4) : 0;
}

bool oil8_bt_supported(int64_t M, int64_t K, int64_t batch) {
    // the kernel takes K and its slice width as int
    return batch >= 2 && K >= 64 && K % 64 == 0 && K < (1ll << 31) && M < (1ll << 31) && M * K < (1ll << 40);
}

size_t oil8_bt_partial_bytes(int64_t M, int64_t K) {
    const int S = o8_slices(M, K);
    return S > 1 ? (size_t)(S * kBtTok * M * 4) : 0;
}

hipError_t launch_oil8_gemv_bt(const uint8_t* idx, const float* cb, const float* x, float* y, int64_t M, int64_t K,
                               int64_t batch, float* partial, hipStream_t s) {
    const int S = o8_slices(M, K);
    const dim3 grid(ceil_div_i(M, kBtRows), (unsigned)S);
    for (int64_t t0 = 0; t0 < batch; t0 += kBtTok) {
        const int b = (int)(batch - t0 < kBtTok ? batch - t0 : kBtTok);
        oil8_gemv_bt<<<grid, 256, 0, s>>>(idx, cb, x + t0 * K, y + t0 * M, partial, (int)M, (int)K, b,
                                          (int)(K / S));
        if (S > 1)
            oil4_bt_reduce<<<ceil_div_i((int64_t)b * M, 256), 256, 0, s>>>(partial, y + t0 * M, (int)M, b, S);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_oil4_gemv_bt(const uint8_t* nib, const uint16_t* cbs, int64_t cb_block, const float* x, float* y,
                               int64_t M, int64_t K, int64_t batch, float* partial, hipStream_t s) {
    const bool sh = cb_block == 0;
    // groups of 16 tokens, one launch each (the weights are read per group)
    for (int64_t t0 = 0; t0 < batch; t0 += kBtTok) {
        const int b = (int)(batch - t0 < kBtTok ? batch - t0 : kBtTok);
        const float* xg = x + t0 * K;
        float* yg = y + t0 * M;
        if (bt_nph(K) == 4) {
            if (sh) run_bt<4, true>(nib, cbs, xg, yg, partial, M, K, b, s);
            else run_bt<4, false>(nib, cbs, xg, yg, partial, M, K, b, s);
        } else {
            if (sh) run_bt<2, true>(nib, cbs, xg, yg, partial, M, K, b, s);
            else run_bt<2, false>(nib, cbs, xg, yg, partial, M, K, b, s);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace mth
