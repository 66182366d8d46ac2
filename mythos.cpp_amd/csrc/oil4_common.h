// oil4_common.h — the OIL4 weight path shared by the decode kernels
// (oil4_gemv_v2 for batch 1, oil4_gemv_bt for batches up to 16).
//
// Weight layout (the reference's, src/kernel_oil4.cpp:45-48): row m is K/2
// bytes, element k is the low nibble of byte k/2 for even k and the high
// nibble for odd k; codebooks cb[m][K/128][16] FP16.
//
// Loads.  A wave instruction that reads 64-byte runs of 16 rows reaches only
// ~4.2 TB/s on MI355X; runs of 128 bytes or more reach the streaming rate.  So
// for a 16-row tile every nibble load reads 8 rows x 128 contiguous bytes
// (lane 16q + jj: row jj % 8 (+8 for the second load), 16-byte piece
// 2q + (jj >= 8) of a 256-column phase), and one DPP row rotation by 8 plus a
// select hands each lane (j = l % 16, q = l / 16) the 32 bytes of row j it
// feeds to the MFMA: pieces 2q, 2q+1, i.e. columns [64q, 64q + 64) of the
// phase.  Codebooks (4 blocks = 128 bytes per row per phase pair) load the
// same way into a 2 KB wave-private LDS stage (XOR-swizzled: conflict-free for
// the writes and for the reads) and each lane reads back the 32-byte block of
// its columns.
//
// Dequantisation.  The block's 16 FP16 entries become 8 byte-plane VGPRs and
// v_perm_b32 is a four-wide 8-entry byte lookup (lookup8): no LDS on the
// weight path.  MFMA m of phase p then covers columns 256p + 64q + 8m + v of
// the tile for lane group q, with the 8 elements of a lane in the order
// v = 0, 2, 4, 6, 1, 3, 5, 7.
#pragma once

#include "common.h"

namespace mth {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Compiler-level ordering point for wave-private LDS traffic.  LDS operations
// of one wave execute in program order, so no wait is needed, only that the
// compiler keeps the order.
__device__ __forceinline__ void wave_lds_order() { asm volatile("" ::: "memory"); }

// Element e of an A/B fragment holds column offset kOrder[e] of its 8.
__device__ __forceinline__ int oil4_elem_col(int e) { return (e < 4) ? 2 * e : 2 * (e - 4) + 1; }

struct CbPlanes {
    uint32_t l[4], h[4];
};

// entries 2i (low half) and 2i+1 (high half) in dword i of a (i < 4) / b
__device__ __forceinline__ CbPlanes cb_planes(const uint4& a, const uint4& b) {
    CbPlanes p;
    p.l[0] = __builtin_amdgcn_perm(a.y, a.x, 0x06040200u);
    p.h[0] = __builtin_amdgcn_perm(a.y, a.x, 0x07050301u);
    p.l[1] = __builtin_amdgcn_perm(a.w, a.z, 0x06040200u);
    p.h[1] = __builtin_amdgcn_perm(a.w, a.z, 0x07050301u);
    p.l[2] = __builtin_amdgcn_perm(b.y, b.x, 0x06040200u);
    p.h[2] = __builtin_amdgcn_perm(b.y, b.x, 0x07050301u);
    p.l[3] = __builtin_amdgcn_perm(b.w, b.z, 0x06040200u);
    p.h[3] = __builtin_amdgcn_perm(b.w, b.z, 0x07050301u);
    return p;
}

// (a & m) | (b & ~m) in one v_bfi_b32: the compiler otherwise spends an AND
// and an OR on the pick selectors below (VOP3 takes no literal on gfx9, so it
// cannot fold both constants into one v_and_or_b32).
__device__ __forceinline__ uint32_t bit_select(uint32_t m, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(m), "v"(a), "v"(b));
    return r;
}

// Pick-selector base: byte j holds j.  Kept in a VGPR (loop-invariant) so
// that bit_select reads only one scalar operand.
__device__ __forceinline__ uint32_t pick_base() {
    uint32_t c = 0x03020100u;
    asm("" : "+v"(c));
    return c;
}

// Weights 0..7 of d (weight v = low nibble of byte v/2 for even v, high for
// odd v) -> FP16 pairs {0,2}, {4,6}, {1,3}, {5,7}.  The low 3 bits of each
// nibble select within entries 0-7 and 8-15, a second v_perm picks by bit 3,
// a third interleaves lo and hi bytes into FP16 pairs (23 VALU per 8 weights).
__device__ __forceinline__ half8 lookup8(uint32_t d, const CbPlanes& p) {
    const uint32_t sE = d & 0x07070707u;
    const uint32_t dO = d >> 4;
    const uint32_t sO = dO & 0x07070707u;
    // byte j of the pick selector: j (entries 0-7) or 4 + j (entries 8-15)
    const uint32_t base = pick_base();
    const uint32_t pE = bit_select(0x04040404u, d >> 1, base);
    const uint32_t pO = bit_select(0x04040404u, d >> 5, base);
    const uint32_t loE = __builtin_amdgcn_perm(__builtin_amdgcn_perm(p.l[3], p.l[2], sE),
                                               __builtin_amdgcn_perm(p.l[1], p.l[0], sE), pE);
    const uint32_t hiE = __builtin_amdgcn_perm(__builtin_amdgcn_perm(p.h[3], p.h[2], sE),
                                               __builtin_amdgcn_perm(p.h[1], p.h[0], sE), pE);
    const uint32_t loO = __builtin_amdgcn_perm(__builtin_amdgcn_perm(p.l[3], p.l[2], sO),
                                               __builtin_amdgcn_perm(p.l[1], p.l[0], sO), pO);
    const uint32_t hiO = __builtin_amdgcn_perm(__builtin_amdgcn_perm(p.h[3], p.h[2], sO),
                                               __builtin_amdgcn_perm(p.h[1], p.h[0], sO), pO);
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v r = {__builtin_amdgcn_perm(hiE, loE, 0x05010400u), __builtin_amdgcn_perm(hiE, loE, 0x07030602u),
                      __builtin_amdgcn_perm(hiO, loO, 0x05010400u), __builtin_amdgcn_perm(hiO, loO, 0x07030602u)};
    return __builtin_bit_cast(half8, r);
}

// As lookup8, but in natural order: FP16/BF16 pairs {0,1}, {2,3}, {4,5},
// {6,7} (for operands whose other side is stored in column order).
__device__ __forceinline__ half8 lookup8_natural(uint32_t d, const CbPlanes& p) {
    const uint32_t sE = d & 0x07070707u;
    const uint32_t dO = d >> 4;
    const uint32_t sO = dO & 0x07070707u;
    const uint32_t base = pick_base();
    const uint32_t pE = bit_select(0x04040404u, d >> 1, base);
    const uint32_t pO = bit_select(0x04040404u, d >> 5, base);
    const uint32_t loE = __builtin_amdgcn_perm(__builtin_amdgcn_perm(p.l[3], p.l[2], sE),
                                               __builtin_amdgcn_perm(p.l[1], p.l[0], sE), pE);
    const uint32_t hiE = __builtin_amdgcn_perm(__builtin_amdgcn_perm(p.h[3], p.h[2], sE),
                                               __builtin_amdgcn_perm(p.h[1], p.h[0], sE), pE);
    const uint32_t loO = __builtin_amdgcn_perm(__builtin_amdgcn_perm(p.l[3], p.l[2], sO),
                                               __builtin_amdgcn_perm(p.l[1], p.l[0], sO), pO);
    const uint32_t hiO = __builtin_amdgcn_perm(__builtin_amdgcn_perm(p.h[3], p.h[2], sO),
                                               __builtin_amdgcn_perm(p.h[1], p.h[0], sO), pO);
    // lo / hi bytes of weights 0-3 and 4-7 in order, then byte pairs
    const uint32_t l03 = __builtin_amdgcn_perm(loO, loE, 0x05010400u), h03 = __builtin_amdgcn_perm(hiO, hiE, 0x05010400u);
    const uint32_t l47 = __builtin_amdgcn_perm(loO, loE, 0x07030602u), h47 = __builtin_amdgcn_perm(hiO, hiE, 0x07030602u);
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v r = {__builtin_amdgcn_perm(h03, l03, 0x05010400u), __builtin_amdgcn_perm(h03, l03, 0x07030602u),
                      __builtin_amdgcn_perm(h47, l47, 0x05010400u), __builtin_amdgcn_perm(h47, l47, 0x07030602u)};
    return __builtin_bit_cast(half8, r);
}

// DPP row rotation inside each 16-lane row (CTRL 0x121..0x12F = row_ror:1..15).
// The empty asm pins the read in the convergent code: a DPP read sunk under a
// partial exec mask would see its source lane disabled.  mov_dpp has no
// "old" operand (a rotation gives every lane a source), so the compiler
// emits no initialising move per read.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_row(uint32_t v) {
    uint32_t r = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true);
    asm volatile("" : "+v"(r));
    return r;
}
__device__ __forceinline__ uint32_t dpp_ror8(uint32_t v) { return dpp_row<0x128>(v); }
// keep, with the lanes of the DPP banks in BANKS (4 lanes each within a 16-lane row) replaced by moved of the
// lane 8 places along the row (row_ror:8): one v_mov_b32_dpp with a bank mask
template <int BANKS>
__device__ __forceinline__ uint32_t dpp_mix(uint32_t keep, uint32_t moved) {
    uint32_t r = (uint32_t)__builtin_amdgcn_update_dpp((int)keep, (int)moved, 0x128, 0xf, BANKS, false);
    asm volatile("" : "+v"(r));
    return r;
}

// Max over the 16 lanes of each DPP row (every lane gets the row's max).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __uint_as_float(dpp_row<0x128>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_row<0x124>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_row<0x122>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp_row<0x121>(__float_as_uint(v))));
    return v;
}

// Sum of the hi-part and lo-part dot products of an FP16 hi/lo split of x
// (x*2^s = hi + lo).  An infinite codebook entry w meets both parts: w*hi is
// +-Inf, but w*lo is NaN where lo is exactly 0, which the reference's single
// product w*x (src/kernel_oil4.cpp:50) never gives.  So an infinite hi sum is
// the result: the reference's sum is then that infinity too (a NaN in its sum
// needs Inf*0, a NaN entry or infinities of both signs, each of which makes
// the hi sum NaN as well), except where x_k is so small relative to max|x|
// that hi_k underflows to 0 (|x_k| < max|x| * 2^-39).
__device__ __forceinline__ float oil4_hi_lo(float hi, float lo) { return __builtin_isinf(hi) ? hi : hi + lo; }

// Power-of-two exponent s with max|x| * 2^s < 2^15 (0 for zero / non-finite).
__device__ __forceinline__ int fp16_scale_shift(float mx) {
    int e = 0;
    if (mx > 0.0f && mx <= 3.40282347e38f) {
        (void)frexpf(mx, &e);
        return 15 - e;
    }
    return 0;
}

// Codebook stage (2 KB, wave-private): (row r, 16-byte piece c) at
// r*128 + 16*(c ^ s(r)).  Lanes 0-7 / 0-15 of a wave access distinct banks
// both when 8 lanes write one row and when 16 lanes read 16 rows.
__device__ __forceinline__ int oil4_stage_off(int r, int c) {
    return r * 128 + 16 * (c ^ ((r & 7) ^ ((r >> 3) & 1)));
}

// All weight loads of one wave for a 16-row tile and NPH phases of 256
// columns starting at column k0, issued in consumption order.
template <int NPH, bool SHARED>
struct Oil4TileLoads {
    static_assert(SHARED || NPH % 2 == 0, "codebooks load per phase pair");
    uint4 wx[NPH], wy[NPH], c0[NPH / 2 + 1], c1[NPH / 2 + 1];

    __device__ __forceinline__ void issue(const uint8_t* nib, const uint16_t* cbs, int row0, int M, int K, int k0,
                                          int lane) {
        issue_rows(nib, cbs, row0, row0 + 8, M, K, k0, lane);
    }
    // Tile rows 0-7 are weight rows rowA.., tile rows 8-15 rows rowB.. (rows
    // past M - 1 read row M - 1).
    __device__ __forceinline__ void issue_rows(const uint8_t* nib, const uint16_t* cbs, int rowA, int rowB, int M,
                                               int K, int k0, int lane) {
        issue_phases<0, NPH>(nib, cbs, rowA, rowB, M, K, k0, lane);
    }
    // Phases P0 .. P1 - 1 only (P0 even: a phase pair's codebooks load with its first phase).
    template <int P0, int P1>
    __device__ __forceinline__ void issue_phases(const uint8_t* nib, const uint16_t* cbs, int rowA, int rowB, int M,
                                                 int K, int k0, int lane) {
        const int j = lane & 15, q = lane >> 4, jj8 = j & 7, hi8 = j >> 3;
        const uint32_t nbr = (uint32_t)K >> 7;  // codebook blocks per row
        // 32-bit byte offsets from the uniform bases (the callers keep M * K / 2 below 2^32), so the loads take a
        // scalar base and a lane offset instead of 64-bit address arithmetic per lane
        const uint32_t hb = (uint32_t)K >> 1, col = (uint32_t)(k0 >> 1) + 16 * (2 * q + hi8);
        const uint32_t ox = (uint32_t)min(rowA + jj8, M - 1) * hb + col, oy = (uint32_t)min(rowB + jj8, M - 1) * hb + col;
        // codebook loads: lane l -> row 8u + l/8, 16-byte piece l % 8 of the
        // 4 blocks of a phase pair
        const uint32_t cpiece = ((uint32_t)(k0 >> 7) * 16 + 8 * (lane & 7)) * 2;
        const uint32_t oc0 = (uint32_t)min(rowA + (lane >> 3), M - 1) * nbr * 32 + cpiece;
        const uint32_t oc1 = (uint32_t)min(rowB + (lane >> 3), M - 1) * nbr * 32 + cpiece;
        const uint8_t* cb8 = (const uint8_t*)cbs;
#pragma unroll
        for (int p = P0; p < P1; ++p) {
            if (!SHARED && p % 2 == 0) {
                c0[p / 2] = ld16(cb8 + oc0 + (p / 2) * 128);
                c1[p / 2] = ld16(cb8 + oc1 + (p / 2) * 128);
            }
            wx[p] = ld_stream(nib + ox + 128 * p);
            wy[p] = ld_stream(nib + oy + 128 * p);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // The 16 FP16 entries (entries 2i, 2i+1 in dword i of a, then b) of the
    // codebook block behind this lane's columns of phase p (stage: the wave's
    // 2 KB codebook stage).
    __device__ __forceinline__ void block(int p, uint8_t* stage, int lane, uint4& a, uint4& b) {
        const int j = lane & 15, q = lane >> 4;
        if (p % 2 == 0) {
            *(uint4*)(stage + oil4_stage_off(lane >> 3, lane & 7)) = c0[p / 2];
            *(uint4*)(stage + oil4_stage_off(8 + (lane >> 3), lane & 7)) = c1[p / 2];
            wave_lds_order();
        }
        const int bi = 2 * (p & 1) + (q >> 1);  // block of this lane's columns
        a = *(const uint4*)(stage + oil4_stage_off(j, 2 * bi));
        b = *(const uint4*)(stage + oil4_stage_off(j, 2 * bi + 1));
        wave_lds_order();
    }

    // Byte planes of that block (lookup8).
    __device__ __forceinline__ CbPlanes planes(int p, uint8_t* stage, int lane) {
        uint4 a, b;
        block(p, stage, lane, a, b);
        return cb_planes(a, b);
    }

    // Rows 0-7 / 8-15 -> lane (j, q): a = piece 2q, b = piece 2q+1 of row j.
    __device__ __forceinline__ void exchange(int p, int lane, uint4& a, uint4& b) const {
        // a: wx in lanes 0-7 of each 16-lane row, wy of lanes 0-7 (row_ror:8) in lanes 8-15 (DPP writes of banks
        // 2-3 only); b: wx of lanes 8-15 in lanes 0-7 (banks 0-1), wy in lanes 8-15
        a = make_uint4(dpp_mix<0xc>(wx[p].x, wy[p].x), dpp_mix<0xc>(wx[p].y, wy[p].y),
                       dpp_mix<0xc>(wx[p].z, wy[p].z), dpp_mix<0xc>(wx[p].w, wy[p].w));
        b = make_uint4(dpp_mix<0x3>(wy[p].x, wx[p].x), dpp_mix<0x3>(wy[p].y, wx[p].y),
                       dpp_mix<0x3>(wy[p].z, wx[p].z), dpp_mix<0x3>(wy[p].w, wx[p].w));
    }
};

}  // namespace mth
