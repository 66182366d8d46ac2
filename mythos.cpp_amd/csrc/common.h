// common.h — device helpers shared by the gfx950 kernels of libmythos_oil.
//
// Wave64 only (CDNA4).  Nothing here allocates; every helper is header-only
// and inlined into the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MTH_WAVE 64

namespace mth {

// ---- rounded FP32 products ---------------------------------------------------
// x * y rounded to FP32 on its own.  hipcc's __fmul_rn is a plain multiply,
// which the compiler may fuse with a following add into one FMA (one rounding
// instead of two) depending on the surrounding code; the reference rounds the
// product first (e.g. an I2_S row's (sum * w_scale) * act_scale, then the
// residual add), so these products are kept out of contraction.
__device__ __forceinline__ float fmul_rn(float x, float y) {
#pragma clang fp contract(off)
    return x * y;
}

// ---- cross-lane reductions over aligned groups of G lanes (G | 64) -------
// In VALU only, with no LDS round trip: lanes l and l ^ 32 by
// v_permlane32_swap and l and l ^ 16 by v_permlane16_swap (each swaps one
// half of its two operands, so with both operands v its two results are v
// and the partner in every lane), 16-lane rows by DPP row rotations, groups
// of 8 / 4 / 2 by DPP half-mirror and quad permutations.  Every lane of a
// group ends with the group's reduction (each step combines two equal-rank
// values, so all lanes add the same operands).  The empty asm keeps each
// cross-lane read out of partial-exec code.
__device__ __forceinline__ uint32_t lane_pin(uint32_t r) {
    asm volatile("" : "+v"(r));
    return r;
}
// (v_mov_b32_dpp without an "old" operand: every pattern used here gives each
// lane a source lane inside its row, so there is nothing to initialise)
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return lane_pin((uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true));
}
template <typename T>
__device__ __forceinline__ uint32_t lane_bits(T v) { return __builtin_bit_cast(uint32_t, v); }
template <typename T>
__device__ __forceinline__ T lane_val(uint32_t b) { return __builtin_bit_cast(T, b); }

template <int G, typename T, typename Op>
__device__ __forceinline__ T group_reduce(T v, Op op) {
    static_assert(sizeof(T) == 4 && G >= 1 && G <= 64 && (G & (G - 1)) == 0, "32-bit lanes, G a power of two");
    if constexpr (G >= 64) {
        const auto r = __builtin_amdgcn_permlane32_swap(lane_bits(v), lane_bits(v), false, false);
        v = op(lane_val<T>(lane_pin(r[0])), lane_val<T>(lane_pin(r[1])));
    }
    if constexpr (G >= 32) {
        const auto r = __builtin_amdgcn_permlane16_swap(lane_bits(v), lane_bits(v), false, false);
        v = op(lane_val<T>(lane_pin(r[0])), lane_val<T>(lane_pin(r[1])));
    }
    if constexpr (G >= 16) {
        v = op(v, lane_val<T>(dpp_u<0x128>(lane_bits(v))));  // row_ror:8
        v = op(v, lane_val<T>(dpp_u<0x124>(lane_bits(v))));  // row_ror:4
        v = op(v, lane_val<T>(dpp_u<0x122>(lane_bits(v))));  // row_ror:2
        v = op(v, lane_val<T>(dpp_u<0x121>(lane_bits(v))));  // row_ror:1
    } else {
        if constexpr (G >= 8) v = op(v, lane_val<T>(dpp_u<0x141>(lane_bits(v))));  // row_half_mirror
        if constexpr (G >= 4) v = op(v, lane_val<T>(dpp_u<0x4E>(lane_bits(v))));   // quad_perm [2,3,0,1]
        if constexpr (G >= 2) v = op(v, lane_val<T>(dpp_u<0xB1>(lane_bits(v))));   // quad_perm [1,0,3,2]
    }
    return v;
}
// The value of lane l ^ 1 (DPP quad_perm [1,0,3,2]).
__device__ __forceinline__ float lane_xor1(float v) { return lane_val<float>(dpp_u<0xB1>(lane_bits(v))); }
struct AddOp {
    template <typename T>
    __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct MaxOp {
    __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
// Maximum of unsigned values (e.g. the bit patterns of magnitudes).
struct UMaxOp {
    __device__ __forceinline__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
};

// Transposed reduction of R per-lane values over the 64 lanes: halving
// exchanges (lanes l ^ 32, l ^ 16, l ^ 8: each lane keeps the rows of its
// half and adds its partner's values of them) and then a sum over groups of
// 64 / R lanes.  After it every lane holds the wave total of row lane /
// (64 / R).  R <= 8.
template <int R, typename T>
__device__ __forceinline__ T transposed_reduce(T (&v)[R], int lane) {
    static_assert(R == 1 || R == 2 || R == 4 || R == 8, "R in 1, 2, 4, 8");
    if constexpr (R >= 2) {  // lanes l ^ 32: lanes < 32 keep v[j], the rest v[j + R/2]
#pragma unroll
        for (int j = 0; j < R / 2; ++j) {
            const auto r = __builtin_amdgcn_permlane32_swap(lane_bits(v[j]), lane_bits(v[j + R / 2]), false, false);
            v[j] = lane_val<T>(lane_pin(r[0])) + lane_val<T>(lane_pin(r[1]));
        }
    }
    if constexpr (R >= 4) {  // lanes l ^ 16
#pragma unroll
        for (int j = 0; j < R / 4; ++j) {
            const auto r = __builtin_amdgcn_permlane16_swap(lane_bits(v[j]), lane_bits(v[j + R / 4]), false, false);
            v[j] = lane_val<T>(lane_pin(r[0])) + lane_val<T>(lane_pin(r[1]));
        }
    }
    if constexpr (R >= 8) {  // lanes l ^ 8 (row_ror:8)
        const bool hi = (lane & 8) != 0;
        const T send = hi ? v[0] : v[1], keep = hi ? v[1] : v[0];
        v[0] = keep + lane_val<T>(dpp_u<0x128>(lane_bits(send)));
    }
    return group_reduce<64 / R>(v[0], AddOp{});
}

// Sums over groups of G consecutive lanes; every lane of a group gets it.
template <int G>
__device__ __forceinline__ float group_sum(float v) { return group_reduce<G>(v, AddOp{}); }
template <int G>
__device__ __forceinline__ int group_sum_i(int v) { return group_reduce<G>(v, AddOp{}); }
template <int N>
__device__ __forceinline__ float lanes_sum(float v) { return group_reduce<N>(v, AddOp{}); }
__device__ __forceinline__ float wave_max(float v) { return group_reduce<64>(v, MaxOp{}); }

// ---- fp16 bits -> f32 (hardware v_cvt_f32_f16: exact for normals and
// subnormals, the same values as src/kernel_oil4.cpp:15-29; NaNs stay NaN) ----
__device__ __forceinline__ float h2f(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}
__device__ __forceinline__ float h2f_lo(uint32_t w) { return h2f(w & 0xffffu); }
__device__ __forceinline__ float h2f_hi(uint32_t w) { return h2f(w >> 16); }

// ---- 128-bit loads ------------------------------------------------------
// Streaming weight loads: each weight byte is read once per launch.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const void* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ld16(const void* p) { return *(const uint4*)p; }
__device__ __forceinline__ float4 ldf4(const float* p) { return *(const float4*)p; }

__device__ __forceinline__ uint32_t u4get(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// ---- row segments: one launch over up to three matrices with the same K --
// Segment s covers workgroups [g0[s], g0[s+1]) and rows [off[s], off[s] +
// rows[s]) of the concatenated row space (g0, off: INT_MAX past the last).
struct Oil8SegArgs {
    const uint8_t* idx[3];
    const float* cb[3];
    float* y[3];
    int rows[3];
    int g0[3];
    int off[3];
    int mtot;
};
// Host-side description of one segment.
struct Oil8Seg {
    const uint8_t* idx;
    const float* cb;
    float* y;
    int64_t rows;
};
constexpr int kOil8MaxSegs = 3;

// Segment table for workgroups of `per_group` rows (nseg <= 3, rows < 2^31).
inline Oil8SegArgs make_seg_args(const Oil8Seg* seg, int nseg, int per_group) {
    Oil8SegArgs a{};
    int g = 0, r = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < nseg) {
            a.idx[i] = seg[i].idx;
            a.cb[i] = seg[i].cb;
            a.y[i] = seg[i].y;
            a.rows[i] = (int)seg[i].rows;
            a.g0[i] = g;
            a.off[i] = r;
            g += (int)((seg[i].rows + per_group - 1) / per_group);
            r += (int)seg[i].rows;
        } else {
            a.idx[i] = seg[0].idx;
            a.cb[i] = seg[0].cb;
            a.y[i] = seg[0].y;
            a.rows[i] = 1;
            a.g0[i] = 0x7fffffff;
            a.off[i] = 0x7fffffff;
        }
    }
    a.mtot = r;
    return a;
}
// Workgroups of a segment table (blockIdx.x range).
inline int seg_groups(const Oil8Seg* seg, int nseg, int per_group) {
    int g = 0;
    for (int i = 0; i < nseg; ++i) g += (int)((seg[i].rows + per_group - 1) / per_group);
    return g;
}

__device__ __forceinline__ int seg_of_group(const Oil8SegArgs& a, int g) { return (g >= a.g0[1]) + (g >= a.g0[2]); }
__device__ __forceinline__ int seg_of_row(const Oil8SegArgs& a, int r) { return (r >= a.off[1]) + (r >= a.off[2]); }

// ---- a batched GEMV's output as its K-slice partial sums ------------------
// value(t, m) = epi(sum over z < n of p[z*zs + t*ts + m]) with the slices
// added in the order 0, 1, ... (the order of the GEMVs' own reduction
// kernels) and epi(v) = (v * scale) * tscale[t] where tscale is set (the
// I2_S epilogue), else v.  n == 1: the finished output.  A consumer that
// reads it in place of a reduced array saves the reduction launch.
struct Slices {
    const float* p;
    int64_t ts, zs;
    int n;
    float scale;
    const float* tscale;
};
constexpr int kMaxSlices = 16;
inline Slices plain_slices(const float* y, int64_t ts) { return Slices{y, ts, 0, 1, 1.0f, nullptr}; }

// slice_value in two steps, so that a consumer can put the loads of several
// values (and of its other operands) in flight before it waits for any:
// slice_issue loads the n partials of value (t, m) into v (the rest are 0),
// slice_sum adds them in the order above and applies the epilogue.
__device__ __forceinline__ void slice_issue(const Slices& s, int t, int64_t m, float (&v)[kMaxSlices]) {
    const float* q = s.p + (int64_t)t * s.ts + m;
#pragma unroll
    for (int z = 0; z < kMaxSlices; ++z) v[z] = z < s.n ? q[z * s.zs] : 0.0f;
}
// slice_issue with every load unconditional (n >= 1; slices z >= n re-read
// slice n - 1, in bounds and from cache): no branch between the loads, so
// the loads of several values stay in flight together.  slice_sum ignores
// v[z] for z >= n.
__device__ __forceinline__ void slice_issue_all(const Slices& s, int t, int64_t m, float (&v)[kMaxSlices]) {
    const float* q = s.p + (int64_t)t * s.ts + m;
    const int last = s.n - 1;
#pragma unroll
    for (int z = 0; z < kMaxSlices; ++z) v[z] = q[(int64_t)min(z, last) * s.zs];
}
__device__ __forceinline__ float slice_sum(const Slices& s, int t, const float (&v)[kMaxSlices]) {
    float sum = v[0];
#pragma unroll
    for (int z = 1; z < kMaxSlices; ++z)
        if (z < s.n) sum += v[z];
    if (s.tscale) sum = fmul_rn(fmul_rn(sum, s.scale), s.tscale[t]);
    return sum;
}
__device__ __forceinline__ float slice_value(const Slices& s, int t, int64_t m) {
    float v[kMaxSlices];
    slice_issue(s, t, m, v);  // every load before the first add
    return slice_sum(s, t, v);
}
// Four consecutive m (m % 4 == 0; 16-byte aligned rows).
__device__ __forceinline__ float4 slice_value4(const Slices& s, int t, int64_t m) {
    const float* q = s.p + (int64_t)t * s.ts + m;
    float4 v[kMaxSlices];
#pragma unroll
    for (int z = 0; z < kMaxSlices; ++z)
        v[z] = z < s.n ? *(const float4*)(q + z * s.zs) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 sum = v[0];
#pragma unroll
    for (int z = 1; z < kMaxSlices; ++z)
        if (z < s.n) {
            sum.x += v[z].x;
            sum.y += v[z].y;
            sum.z += v[z].z;
            sum.w += v[z].w;
        }
    if (s.tscale) {
        const float ts = s.tscale[t];
        sum = make_float4(fmul_rn(fmul_rn(sum.x, s.scale), ts), fmul_rn(fmul_rn(sum.y, s.scale), ts),
                          fmul_rn(fmul_rn(sum.z, s.scale), ts), fmul_rn(fmul_rn(sum.w, s.scale), ts));
    }
    return sum;
}

// ---- RMSNorm split over the launches around it ---------------------------
// y = W rms_norm(v) * gamma = inv * (W (v * gamma)), inv = 1 / sqrt(mean(v^2)
// + eps), so a GEMV can take xg = v * gamma and its consumer scale the output
// by inv.  The producer of the residual delta finishes the residual stream
// in its epilogue (ResidOut): x <- y + x (the norm's residual add), xg = x *
// gamma of the next norm, and per workgroup the sum of its rows' x^2 (double)
// in ssp[token][workgroup].  The next small consumer (attention, SwiGLU)
// reads NormScale: the sum over the nparts partials, in order.
struct ResidOut {
    float* x;             // null: off (plain output)
    const float* gamma;
    float* xg;
    double* ssp;
};
struct NormScale {
    const double* ssp;    // null: off
    int nparts;
    float dim, eps;
};
// Sum over the 64 lanes in FP64, the same steps as group_reduce<64> on both
// halves of each value.
__device__ __forceinline__ double wave_sum_dbl(double v) {
    auto part = [](double x, int step) -> double {
        const uint64_t b = __builtin_bit_cast(uint64_t, x);
        const uint32_t lo = (uint32_t)b, hi = (uint32_t)(b >> 32);
        uint32_t l2, h2;
        if (step == 0 || step == 1) {
            const auto rl = step == 0 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                                      : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
            const auto rh = step == 0 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                                      : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
            const double a = __builtin_bit_cast(double, (uint64_t)lane_pin(rl[0]) | ((uint64_t)lane_pin(rh[0]) << 32));
            const double c = __builtin_bit_cast(double, (uint64_t)lane_pin(rl[1]) | ((uint64_t)lane_pin(rh[1]) << 32));
            return a + c;
        }
        switch (step) {
            case 2: l2 = dpp_u<0x128>(lo), h2 = dpp_u<0x128>(hi); break;
            case 3: l2 = dpp_u<0x124>(lo), h2 = dpp_u<0x124>(hi); break;
            case 4: l2 = dpp_u<0x122>(lo), h2 = dpp_u<0x122>(hi); break;
            default: l2 = dpp_u<0x121>(lo), h2 = dpp_u<0x121>(hi); break;
        }
        return x + __builtin_bit_cast(double, (uint64_t)l2 | ((uint64_t)h2 << 32));
    };
#pragma unroll
    for (int step = 0; step < 6; ++step) v = part(v, step);
    return v;
}
// This thread's share of token t's NormScale sum: partials i = i0, i0 +
// stride, ... added in order.  norm_issue loads the first kNormBatch of them
// (clamped to the last partial, so every load is in bounds and none waits
// on a branch) and norm_finish adds them, then any further ones.
constexpr int kNormBatch = 4;
__device__ __forceinline__ void norm_issue(const NormScale& ns, int t, int i0, int stride,
                                           double (&v)[kNormBatch]) {
    const double* p = ns.ssp + (int64_t)t * ns.nparts;
    const int last = ns.nparts - 1;
#pragma unroll
    for (int j = 0; j < kNormBatch; ++j) v[j] = last >= 0 ? p[min(i0 + j * stride, last)] : 0.0;
}
__device__ __forceinline__ double norm_finish(const NormScale& ns, int t, int i0, int stride,
                                              const double (&v)[kNormBatch]) {
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kNormBatch; ++j)
        if (i0 + j * stride < ns.nparts) s += v[j];
    for (int i = i0 + kNormBatch * stride; i < ns.nparts; i += stride) s += ns.ssp[(int64_t)t * ns.nparts + i];
    return s;
}
// 1 / sqrt(sum / dim + eps) of token t, computed by a whole workgroup of
// NW waves (red: NW doubles of LDS); every thread gets it.
// norm_scale_issued: the same from partials this thread loaded with
// norm_issue(ns, t, threadIdx.x, NW * 64, v) earlier (ahead of other loads).
template <int NW>
__device__ __forceinline__ float norm_scale_issued(const NormScale& ns, int t, const double (&v)[kNormBatch],
                                                   double* red) {
    double s = wave_sum_dbl(norm_finish(ns, t, threadIdx.x, NW * 64, v));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = 0.0;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += red[w];
    return (float)(1.0 / sqrt(s / (double)ns.dim + (double)ns.eps));
}
template <int NW>
__device__ __forceinline__ float norm_scale(const NormScale& ns, int t, double* red) {
    double v[kNormBatch];
    norm_issue(ns, t, threadIdx.x, NW * 64, v);
    return norm_scale_issued<NW>(ns, t, v, red);
}

// silu(g) = g / (1 + e^-g), in FP32 with expf and an IEEE division (the
// SwiGLU of every decoder path uses this one definition).
__device__ __forceinline__ float silu1(float g) { return (g / (1.0f + expf(-g))); }

// ---- int8 helpers ---------------------------------------------------------
// sum_{i<4} (int8)a.byte[i] * (int8)b.byte[i] + c   (v_dot4_i32_i8)
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Reference int8 quantisation of one value (src/int8_quant.cpp:19):
// (int8_t)std::round(v * scale) — round half away from zero, then truncate.
__device__ __forceinline__ int quant_i8(float v, float scale) {
    return (int)(int8_t)(int)__builtin_roundf(fmul_rn(v, scale));
}

}  // namespace mth
