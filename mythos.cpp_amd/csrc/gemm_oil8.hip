// gemm_oil8.hip — the prompt prefill's OIL8 projections (Q, K, V and O) on
// gfx950 MFMA: FP32 rows in, FP32 rows out.
//
//   y_s[m][n] = sum_k cb_s[idx_s[n][k]] * a[m][k]    (m < Mr, segment s)
//
// per row m the reference's oil8_gemm with N = 1 (src/kernel_oil8.cpp:14-27,
// 63-71), as the decode GEMVs compute it, for every row of a prompt chunk at
// once (the prompt as one forward pass, src/generator.cpp:36), so each weight
// is read once per 128 rows instead of once per 16 (the batched GEMV).
// Up to three weights (Q, K, V), each with its own 256-entry FP32 codebook and
// output, run in one launch.
//
// Arithmetic: the batched OIL8 GEMV's FP16 hi / lo scheme.  Rows of a arrive
// as FP16 hi / lo virtual rows after a per-row power-of-two scale
// (oil4_prefill_a16x: 2^r a = hi + lo); the codebook is scaled by 2^w
// (max |cb| 2^w in [2^14, 2^15)) and each entry split the same way into a
// 256-entry LDS table of (hi, lo) pairs.  Three products per weight and row,
// a_hi w_hi + a_hi w_lo + a_lo w_hi (a_lo w_lo is below FP32's rounding),
// each exact in FP32 on v_mfma_f32_16x16x32_f16, summed in FP32; the result is
// scaled back by 2^-(r + w), exactly.  A workgroup whose codebook or rows
// hold a non-finite value (Inf cannot be split: Inf - Inf is NaN) computes its
// tile with FP32 FMAs over the reference's products in column order instead,
// so Inf and NaN propagate as in the reference.
//
// Tiling.  A workgroup computes 128 rows x BN columns of one segment: 8 waves,
// two per SIMD.  Waves 4-7 (producers) stream the index bytes of BN weight
// rows (4 K steps of 64 ahead), look every byte up in the table (one
// ds_read_b32 gives both FP16 parts) and write the hi and lo tiles of each
// K step into a ring of 2 BS steps in LDS, BS steps ahead of the consumers;
// one barrier per BS steps hands the tiles over.  Waves 0-3 (consumers) hold
// the accumulators of 32 real rows each — their hi rows (two groups of 16)
// and the same rows' lo parts (two groups) — so the three products per
// weight are balanced across the waves and an output's hi and lo sums meet in
// one lane; A fragments come from L2 into a ring of PA register sets.
// Workgroups on one XCD share an M tile (WG i runs on XCD i % 8), so the
// XCD's L2 holds that tile's A (256 virtual rows x K FP16).  C is staged
// through LDS and written in 16-byte pieces.
#include "common.h"
#include "launch.h"
#include "oil4_common.h"

#include <type_traits>

namespace mth {
namespace {

constexpr int QBK = 64;  // K step

// (row r, 16-byte piece c) of a W tile (rows of 128 bytes): lanes 0-15
// reading 16 rows of one piece hit distinct bank groups
__device__ __forceinline__ int q_off(int r, int c) { return r * 128 + 16 * (c ^ ((r & 7) ^ ((r >> 3) & 1))); }

__device__ __forceinline__ uint32_t hl_pair(float c) {
    const _Float16 h = (_Float16)c;
    const _Float16 l = (_Float16)(c - (float)h);
    return (uint32_t)__builtin_bit_cast(uint16_t, h) | ((uint32_t)__builtin_bit_cast(uint16_t, l) << 16);
}

struct Oil8GemmSegs {
    const uint8_t* idx[3];
    const float* cb[3];
    float* y[3];
    int rows[3];
    int t0[4];  // first N tile of each segment; t0[nseg] = all tiles
};

template <int BN, int BS, int CW>
struct Q8Lds {
    static constexpr int hdr = 1024 + 64;                  // table, producer wave maxima
    static constexpr int tile = BN * 256;                  // one K step: hi tile, then lo tile
    static constexpr int ring = 2 * BS * tile;
    static constexpr int stage = 32 * CW * (BN + 4) * 4;  // C (FP32, rows padded by 4)
    static constexpr int bytes = hdr + (ring > stage ? ring : stage);
};

// CW consumer waves of 32 real rows each (4: tiles of 128 rows, two waves per
// SIMD; 8: tiles of 256 rows, three waves per SIMD, so each SIMD has a second
// consumer to issue MFMAs while one waits for LDS, and each W tile serves
// twice the rows), then 4 producer waves.
template <int BN, int PA, int BS, int CW>
__global__ __launch_bounds__(64 * (CW + 4)) void oil8_prefill_ws(const uint16_t* __restrict__ A16,
                                                                 const float* __restrict__ a32, Oil8GemmSegs sg,
                                                                 int Mr, int K, const int* __restrict__ rsh,
                                                                 int ntiles) {
    using L = Q8Lds<BN, BS, CW>;
    constexpr int NT = BN / 16, TPR = 256 / BN, BPT = QBK / TPR, NV = BPT / 16, PW = 4;
    constexpr int MT = 32 * CW, NTH = 64 * (CW + 4);  // real rows per tile, threads
    static_assert(PA == 2 || PA == 4, "A ring index");
    static_assert(BS == 1 || BS == 2 || BS == 4, "barrier interval");
    static_assert(BPT % 16 == 0, "producer piece");
    __shared__ __align__(16) uint8_t lds[L::bytes];
    uint32_t* tab = (uint32_t*)lds;
    float* wred = (float*)(lds + 1024);
    uint8_t* ring = lds + L::hdr;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tm = (Mr + MT - 1) / MT;
    int mt, nt;
    {
        const int id = blockIdx.x, total = tm * ntiles;
        if (total % 8 == 0 && tm % 8 == 0) {
            const int xcd = id % 8, slot = id / 8;
            mt = 8 * (slot / ntiles) + xcd;
            nt = slot % ntiles;
        } else if (total % 8 == 0 && 8 % tm == 0) {
            const int grp = 8 / tm, xcd = id % 8, slot = id / 8;
            mt = xcd / grp;
            nt = slot * grp + xcd % grp;
        } else {
            mt = id / ntiles;
            nt = id % ntiles;
        }
    }
    const int s = (nt >= sg.t0[1]) + (nt >= sg.t0[2]);
    const int N = sg.rows[s], n0 = (nt - sg.t0[s]) * BN;
    const uint8_t* idx = sg.idx[s];
    const float* cb = sg.cb[s];
    float* y = sg.y[s];
    const int steps = K / QBK;

    // ---- codebook scale and the non-finite check (codebook entries, rows of the tile)
    float cbv = 0.0f;
    bool fin = true;
    if (wave >= CW) {
        cbv = cb[tid - 64 * CW];
        fin = __builtin_isfinite(cbv);
        const float m = wave_max(fabsf(cbv));
        if (lane == 0) wred[wave - CW] = m;
    } else if (tid < MT) {
        const int row = MT * mt + tid;
        fin = !(row < Mr && rsh[row] == kRowNonFinite);
    }
    if (__syncthreads_or(!fin)) {
        // FP32 FMAs over the reference's products in column order
        for (int o = tid; o < MT * BN; o += NTH) {
            const int r = o / BN, n = o % BN, row = MT * mt + r;
            if (row >= Mr) continue;
            const uint8_t* w = idx + (int64_t)(n0 + n) * K;
            const float* a = a32 + (int64_t)row * K;
            float sum = 0.0f;
            for (int k = 0; k < K; ++k) sum = fmaf(cb[w[k]], a[k], sum);
            y[(int64_t)row * N + n0 + n] = sum;
        }
        return;
    }
    const int sw = fp16_scale_shift(fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3])));

    if (wave >= CW) {
        // ---------------- producers ----------------
        const int t = tid - 64 * CW;
        tab[t] = hl_pair(ldexpf(cbv, sw));
        const int wn = t / TPR, wh = t % TPR;
        const uint8_t* wrow = idx + (int64_t)(n0 + wn) * K + BPT * wh;
        uint4 nv[PW][NV];
        auto load_n = [&](int step, int slot) {
#pragma unroll
            for (int v = 0; v < NV; ++v) nv[slot][v] = ld_stream(wrow + step * QBK + 16 * v);
        };
#pragma unroll
        for (int u = 0; u < PW; ++u) load_n(min(u, steps - 1), u);
        __syncthreads();  // the table
        // Look K step x (x % 4 == XM) up into its ring tile, then refill x's slot with step x + 4.
        auto produce = [&](int x, auto xm) {
            constexpr int XM = decltype(xm)::value;
            uint8_t* wb = ring + (x % (2 * BS)) * L::tile;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    const uint32_t w0 = h2 ? nv[XM][v].z : nv[XM][v].x, w1 = h2 ? nv[XM][v].w : nv[XM][v].y;
                    uint32_t gv[8];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        gv[e] = tab[(w0 >> (8 * e)) & 0xffu];
                        gv[4 + e] = tab[(w1 >> (8 * e)) & 0xffu];
                    }
                    u32x4 hv, lv;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        hv[d] = __builtin_amdgcn_perm(gv[2 * d + 1], gv[2 * d], 0x05040100u);
                        lv[d] = __builtin_amdgcn_perm(gv[2 * d + 1], gv[2 * d], 0x07060302u);
                    }
                    const int c = (BPT * wh + 16 * v) / 8 + h2;  // 16-byte piece (8 k) of the step
                    *(u32x4*)(wb + q_off(wn, c)) = hv;
                    *(u32x4*)(wb + BN * 128 + q_off(wn, c)) = lv;
                }
            }
            load_n(min(x + PW, steps - 1), XM);
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
        produce(0, I0{});
        if constexpr (BS >= 2) produce(1, I1{});
        if constexpr (BS >= 4) {
            produce(2, I2{});
            produce(3, I3{});
        }
        __syncthreads();
        for (int s0 = 0; s0 < steps; s0 += 4) {
            // steps s0 + BS .. s0 + 3 + BS while the consumers run s0 .. s0 + 3 (tiles of steps >= steps unused)
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
        __syncthreads();
    } else {
        // ---------------- consumers ----------------
        // virtual 16-row groups: 128 real rows are 16 groups, the hi parts in the first 8;
        // wave w: hi groups 2w', 2w' + 1 (w' = w % 4) of the 128-row block w / 4 of the tile (real rows
        // 32w .. 32w + 31 of the tile) and their lo groups
        const int kc32 = K / 32;
        const int gb = 16 * (MT / 128 * mt + wave / 4) + 2 * (wave % 4);
        const half8* af16 = (const half8*)A16 + lane;
        half8 af[PA][4][2];
        auto load_a = [&](int step, int b) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int g = gb + (i & 1) + 8 * (i >> 1);
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) af[b][i][kk] = af16[((int64_t)g * kc32 + 2 * step + kk) * 64];
            }
        };
        floatx4 acc[4][NT];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < PA - 1; ++u) load_a(min(u, steps - 1), u);
        __syncthreads();  // the table
        __syncthreads();  // the first BS tiles
        for (int s0 = 0; s0 < steps; s0 += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int step = s0 + u;
                const uint8_t* cur = ring + (step % (2 * BS)) * L::tile;
                load_a(min(step + PA - 1, steps - 1), (u + PA - 1) % PA);  // into the set of A(step - 1)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    half8 bh[NT], bl[NT];
#pragma unroll
                    for (int j = 0; j < NT; ++j) {
                        const int o = q_off(16 * j + (lane & 15), 4 * kk + (lane >> 4));
                        bh[j] = *(const half8*)(cur + o);
                        bl[j] = *(const half8*)(cur + BN * 128 + o);
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < NT; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[u % PA][i][kk], bh[j], acc[i][j], 0,
                                                                               0, 0);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < NT; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[u % PA][i][kk], bl[j], acc[i][j], 0,
                                                                               0, 0);
                }
                if ((u + 1) % BS == 0) __syncthreads();
            }
        }
        __syncthreads();
        // real row 32w + 16i + 4(lane / 16) + r of the tile: hi sum + lo sum, times 2^-(shift + sw)
        float* st = (float*)ring;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int rr = 32 * wave + 16 * i + 4 * (lane >> 4) + r;
                const int sh = rsh[min(MT * mt + rr, Mr - 1)] + sw;
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    st[rr * (BN + 4) + 16 * j + (lane & 15)] = ldexpf(acc[i][j][r] + acc[i + 2][j][r], -sh);
            }
        __syncthreads();
    }
    constexpr int CPR = BN / 4;
    const float* st = (const float*)ring;
    for (int c = tid; c < MT * CPR; c += NTH) {
        const int r = c / CPR, q = c % CPR, row = MT * mt + r;
        if (row < Mr) *(float4*)(y + (int64_t)row * N + n0 + 4 * q) = *(const float4*)(st + r * (BN + 4) + 4 * q);
    }
}

}  // namespace

bool oil8_gemm_x32_supported(const Oil8Seg* seg, int nseg, int64_t Mr, int64_t K) {
    if (nseg < 1 || nseg > 3 || Mr < 1 || Mr > (1 << 24) || K < 256 || K % 256 != 0 || K > (1 << 20)) return false;
    int64_t tiles = 0;
    for (int i = 0; i < nseg; ++i) {
        const Oil8Seg& g = seg[i];
        if (!g.idx || !g.cb || !g.y || g.rows < 64 || g.rows % 64 != 0 || g.rows >= (1ll << 31)) return false;
        if ((((uintptr_t)g.idx | (uintptr_t)g.y) & 15u) != 0) return false;
        tiles += g.rows / 64;
    }
    return tiles * ((Mr + 127) / 128) < (1ll << 31) && Mr * K < (1ll << 40);
}

// the row shifts, then the hi / lo fragments of Mr rows rounded up to 256
// (the tiles of 256 rows read both 128-row blocks)
size_t oil8_gemm_x32_workspace_bytes(int64_t Mr, int64_t K) {
    return oil4_prefill_shift_bytes(Mr) + (size_t)(2 * ((Mr + 255) / 256 * 256) * K * 2);
}

hipError_t launch_oil8_gemm_x32(const float* a, const Oil8Seg* seg, int nseg, int64_t Mr, int64_t K, void* ws,
                                hipStream_t s) {
    if (!oil8_gemm_x32_supported(seg, nseg, Mr, K)) return hipErrorInvalidValue;
    constexpr int BN = 64;
    Oil8GemmSegs g{};
    int t = 0;
    for (int i = 0; i < 3; ++i) {
        g.t0[i] = t;
        if (i < nseg) {
            g.idx[i] = seg[i].idx;
            g.cb[i] = seg[i].cb;
            g.y[i] = seg[i].y;
            g.rows[i] = (int)seg[i].rows;
            t += (int)(seg[i].rows / BN);
        } else {
            g.idx[i] = seg[0].idx;
            g.cb[i] = seg[0].cb;
            g.y[i] = seg[0].y;
            g.rows[i] = (int)seg[0].rows;
        }
    }
    g.t0[3] = t;
    for (int i = nseg; i < 3; ++i) g.t0[i] = t + 1;  // never selected
    const int* rsh = (const int*)ws;
    const uint16_t* a16 = (const uint16_t*)((const char*)ws + oil4_prefill_shift_bytes(Mr));
    // tiles of 256 rows (8 consumer waves) when they fill a round of 256 CUs, else of 128
    const int64_t t256 = (Mr + 255) / 256, t128 = (Mr + 127) / 128;
    const bool wide = t256 * t >= 256;
    hipError_t e = launch_prefill_a16x(a, Mr, K, ws, s, wide ? 256 * t256 : 128 * t128);
    if (e != hipSuccess) return e;
    if (wide)
        oil8_prefill_ws<BN, 2, 1, 8><<<(unsigned)(t256 * t), 768, 0, s>>>(a16, a, g, (int)Mr, (int)K, rsh, t);
    else
        oil8_prefill_ws<BN, 4, 2, 4><<<(unsigned)(t128 * t), 512, 0, s>>>(a16, a, g, (int)Mr, (int)K, rsh, t);
    return hipGetLastError();
}

}  // namespace mth
