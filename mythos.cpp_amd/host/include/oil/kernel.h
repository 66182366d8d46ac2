// oil/kernel.h — drop-in replacement for MYTHOS.cpp's include/oil/kernel.h
// (lines 13-65): the same namespace, names and signatures, backed by the
// gfx950 kernels of libmythos_oil.so (include/mythos_oil.h).
//
// Contract kept from the reference: host pointers, synchronous return,
// outputs overwritten, the reference's per-(m,n) weight indexing for
// oil8_gemm / oil4_gemm / tl1_gemm / tl2_gemm, weights shared over n for the
// i2s_gemm family.  Differences (all documented at the definitions):
//   * failures throw oil::Error (the reference has no checks; UB instead);
//   * oil4_gemm computes the scalar definition (src/kernel_oil4.cpp:31-54),
//     not the AVX2 build's extra codebook[0]*sum(act) term;
//   * i2s_gemv always sees an initialised decode table (the reference returns
//     0 until some i2s_gemm* call has run);
//   * i2s_gemm_vnni computes its documented body (the as-built reference
//     compiles an empty stub);
//   * tl2_gemm requires K % 3 == 0 (the reference reads out of bounds else);
//   * the dense FP32 helpers (scalar_gemm, tiled_gemm, avx2_gemm,
//     avx2_tiled_gemm) all run one rocBLAS SGEMM, for any N (the reference's
//     avx2_gemm needs N % 8 == 0).
// Weight operands registered with oil::mi355x::register_weights
// (oil/mi355x.h) stay resident on the device.
#pragma once

#include <cstdint>

#include "oil/tensor.h"
#include "oil/types.h"

namespace oil {
namespace kernel {

void i2s_gemm(const Tensor& weights, const Tensor& activations, Tensor& output, int M, int N, int K);
void i2s_gemv(const uint8_t* packed_w, float w_scale, const int8_t* act, float act_scale, float* output, int K);

void tl1_gemm(const Tensor& weights, const Tensor& activations, Tensor& output, int M, int N, int K);
void tl1_precompute_lut(const int8_t* activations, int8_t* lut, int K, float scales);

void tl2_gemm(const Tensor& weights, const Tensor& activations, Tensor& output, int M, int N, int K);
void tl2_precompute_lut(const int8_t* activations, int8_t* lut, int K, float scales);

void oil8_gemm(const uint8_t* indices, const float* codebook, const float* activations, float* output,
               int M, int N, int K);

void oil4_gemm(const uint8_t* packed_indices, const uint16_t* codebook, const float* activations,
               float* output, int M, int N, int K);

void i2s_gemm_avx2(const Tensor& weights, const Tensor& activations, Tensor& output, int M, int N, int K);

void i2s_gemm_vnni(const uint8_t* packed_w, const int8_t* activations, float* output, int M, int N, int K);

// Dense FP32: C[M][N] = A[M][K] * B[K][N], row-major, C overwritten.
void scalar_gemm(const float* A, const float* B, float* C, int M, int N, int K);
void tiled_gemm(const float* A, const float* B, float* C, int M, int N, int K);
void avx2_gemm(const float* A, const float* B, float* C, int M, int N, int K);
void avx2_tiled_gemm(const float* A, const float* B, float* C, int M, int N, int K);

// ---- extensions (no reference counterpart): the decode formats of the
// BASELINE configs, host-pointer + synchronous like the functions above ----

// y[t*M + m] = sum_k codebooks[(m*(K/cb_block) + k/cb_block)*16 + nib] * x[t*K + k]
void oil4_gemv_blocked(const uint8_t* packed, const uint16_t* codebooks, int cb_block, const float* x,
                       float* y, int M, int K, int batch);
// quantize_per_token(x_t) then i2s_gemv per row: y[t*M + m]
void i2s_gemv_f32(const uint8_t* packed, float w_scale, const float* x, float* y, int M, int K, int batch);

}  // namespace kernel
}  // namespace oil
