// kernel.cpp — host-pointer, synchronous drop-ins for MYTHOS.cpp's
// oil::kernel::* and oil::quantize_* (include/oil/kernel.h:13-65,
// include/oil/int8_quant.h:7-28), running on the gfx950 kernels through the
// C ABI of libmythos_oil.so.
//
// Each call stages its operands in a per-thread device arena (grown on
// demand, never shrunk), copies inputs host->device, launches on the
// thread's stream, copies outputs back and synchronises.  Weight operands
// that lie inside a range registered with oil::mi355x::register_weights are
// read from their resident device copy instead of being copied.  There is no
// CPU code path: a missing or failing GPU raises oil::Error.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "mythos_oil.h"
#include "oil/int8_quant.h"
#include "oil/kernel.h"
#include "oil/mi355x.h"
#include "staging.h"

namespace oil {
using namespace detail;

namespace kernel {

void oil8_gemm(const uint8_t* indices, const float* codebook, const float* activations, float* output,
               int M, int N, int K) {
    check_dims(M, N, K, "oil8_gemm");
    const size_t R = (size_t)M * N, nw = R * K, na = (size_t)N * K;
    Arena& a = arena();
    a.begin(P(nw) + P(256 * 4) + P(na * 4) + P(R * 4));
    const uint8_t* di = a.weights(indices, nw);
    const float* dc = a.weights(codebook, 256);
    const float* dx = a.upload(activations, na);
    float* dy = (float*)a.carve(R * 4);
    mth_check(mth_oil8_gemm(di, dc, dx, dy, M, N, K, a.stream()), "oil8_gemm");
    a.download(output, dy, R);
    a.sync();
}

void oil4_gemm(const uint8_t* packed_indices, const uint16_t* codebook, const float* activations,
               float* output, int M, int N, int K) {
    check_dims(M, N, K, "oil4_gemm");
    const size_t R = (size_t)M * N, nb = (R * (size_t)K + 1) / 2, na = (size_t)N * K;
    Arena& a = arena();
    a.begin(P(nb) + P(32) + P(na * 4) + P(R * 4));
    const uint8_t* dp = a.weights(packed_indices, nb);
    const uint16_t* dc = a.weights(codebook, 16);
    const float* dx = a.upload(activations, na);
    float* dy = (float*)a.carve(R * 4);
    mth_check(mth_oil4_gemm(dp, dc, dx, dy, M, N, K, a.stream()), "oil4_gemm");
    a.download(output, dy, R);
    a.sync();
}

void i2s_gemv(const uint8_t* packed_w, float w_scale, const int8_t* act, float act_scale, float* output, int K) {
    if (K <= 0 || K % 4) throw Error("i2s_gemv: K must be a positive multiple of 4");
    Arena& a = arena();
    a.begin(P(K / 4) + P(K) + P(4) + P(4));
    const uint8_t* dw = a.weights(packed_w, (size_t)K / 4);
    const int8_t* dq = a.upload(act, (size_t)K);
    const float* ds = a.upload(&act_scale, 1);
    float* dy = (float*)a.carve(4);
    mth_check(mth_i2s_gemv(dw, w_scale, dq, ds, dy, 1, K, 1, a.stream()), "i2s_gemv");
    a.download(output, dy, 1);
    a.sync();
}

void i2s_gemm(const Tensor& weights, const Tensor& activations, Tensor& output, int M, int N, int K) {
    check_dims(M, N, K, "i2s_gemm");
    const size_t nw = (size_t)M * (K / 4) + (K % 4 ? 1 : 0), na = (size_t)N * K, R = (size_t)M * N;
    OIL_CHECK(weights.size_bytes() >= nw && activations.numel() >= (int64_t)na && output.numel() >= (int64_t)R,
              "i2s_gemm: tensor too small");
    Arena& a = arena();
    a.begin(P(nw) + P(na * 4) + P(R * 4));
    const uint8_t* dw = a.weights(weights.data<uint8_t>(), nw);
    const float* dx = a.upload(activations.data<float>(), na);
    float* dy = (float*)a.carve(R * 4);
    mth_check(mth_i2s_gemm(dw, dx, dy, M, N, K, a.stream()), "i2s_gemm");
    a.download(output.data<float>(), dy, R);
    a.sync();
}

// Same contract as i2s_gemm (the reference's AVX2 variant differs only in
// summation order, src/kernel_i2s.cpp:156-199).
void i2s_gemm_avx2(const Tensor& weights, const Tensor& activations, Tensor& output, int M, int N, int K) {
    i2s_gemm(weights, activations, output, M, N, K);
}

void i2s_gemm_vnni(const uint8_t* packed_w, const int8_t* activations, float* output, int M, int N, int K) {
    check_dims(M, N, K, "i2s_gemm_vnni");
    const size_t nw = (size_t)M * (K / 4) + (K % 4 ? 1 : 0), na = (size_t)N * K, R = (size_t)M * N;
    Arena& a = arena();
    a.begin(P(nw) + P(na) + P(R * 4));
    const uint8_t* dw = a.weights(packed_w, nw);
    const int8_t* dx = a.upload(activations, na);
    float* dy = (float*)a.carve(R * 4);
    mth_check(mth_i2s_gemm_vnni(dw, dx, dy, M, N, K, a.stream()), "i2s_gemm_vnni");
    a.download(output, dy, R);
    a.sync();
}

void tl1_gemm(const Tensor& weights, const Tensor& activations, Tensor& output, int M, int N, int K) {
    check_dims(M, N, K, "tl1_gemm");
    const size_t R = (size_t)M * N, nw = (R * (size_t)K) / 4 + 1, na = (size_t)N * K;
    OIL_CHECK(weights.size_bytes() + 1 >= nw && activations.numel() >= (int64_t)na && output.numel() >= (int64_t)R,
              "tl1_gemm: tensor too small");
    Arena& a = arena();
    a.begin(P(nw) + P(na * 4) + P(R * 4));
    uint8_t* dw = (uint8_t*)a.carve(nw);
    hip_check(hipMemsetAsync(dw, 0, nw, (hipStream_t)a.stream()), "hipMemset");
    hip_check(hipMemcpyAsync(dw, weights.data(), std::min(nw, weights.size_bytes()), hipMemcpyHostToDevice,
                             (hipStream_t)a.stream()),
              "hipMemcpy H2D");
    const float* dx = a.upload(activations.data<float>(), na);
    float* dy = (float*)a.carve(R * 4);
    mth_check(mth_tl1_gemm(dw, dx, dy, M, N, K, a.stream()), "tl1_gemm");
    a.download(output.data<float>(), dy, R);
    a.sync();
}

void tl2_gemm(const Tensor& weights, const Tensor& activations, Tensor& output, int M, int N, int K) {
    check_dims(M, N, K, "tl2_gemm");
    const size_t R = (size_t)M * N, bpr = ((size_t)K * 2 + 7) / 8, nw = R * bpr, na = (size_t)N * K;
    OIL_CHECK(weights.size_bytes() >= nw && activations.numel() >= (int64_t)na && output.numel() >= (int64_t)R,
              "tl2_gemm: tensor too small");
    Arena& a = arena();
    a.begin(P(nw) + P(na * 4) + P(R * 4));
    const uint8_t* dw = a.weights(weights.data<uint8_t>(), nw);
    const float* dx = a.upload(activations.data<float>(), na);
    float* dy = (float*)a.carve(R * 4);
    mth_check(mth_tl2_gemm(dw, dx, dy, M, N, K, a.stream()), "tl2_gemm");
    a.download(output.data<float>(), dy, R);
    a.sync();
}

void tl1_precompute_lut(const int8_t* activations, int8_t* lut, int K, float scales) {
    (void)scales;  // unused by the reference as well (src/kernel_tl.cpp:15)
    if (K < 2) return;
    Arena& a = arena();
    const size_t nl = (size_t)(K / 2) * 9;
    a.begin(P(K) + P(nl));
    const int8_t* dx = a.upload(activations, (size_t)K);
    int8_t* dl = (int8_t*)a.carve(nl);
    mth_check(mth_tl_precompute_lut(dx, dl, K, 2, a.stream()), "tl1_precompute_lut");
    a.download(lut, dl, nl);
    a.sync();
}

void tl2_precompute_lut(const int8_t* activations, int8_t* lut, int K, float scales) {
    (void)scales;  // unused by the reference as well (src/kernel_tl.cpp:90)
    if (K <= 0) return;
    if (K % 3) throw Error("tl2_precompute_lut: K must be a multiple of 3");
    Arena& a = arena();
    const size_t nl = (size_t)(K / 3) * 27;
    a.begin(P(K) + P(nl));
    const int8_t* dx = a.upload(activations, (size_t)K);
    int8_t* dl = (int8_t*)a.carve(nl);
    mth_check(mth_tl_precompute_lut(dx, dl, K, 3, a.stream()), "tl2_precompute_lut");
    a.download(lut, dl, nl);
    a.sync();
}

void oil4_gemv_blocked(const uint8_t* packed, const uint16_t* codebooks, int cb_block, const float* x, float* y,
                       int M, int K, int batch) {
    check_dims(M, batch, K, "oil4_gemv_blocked");
    const size_t nb = (size_t)M * K / 2, nc = cb_block ? (size_t)M * (K / cb_block) * 16 : 16;
    Arena& a = arena();
    a.begin(P(nb) + P(nc * 2) + P((size_t)batch * K * 4) + P((size_t)batch * M * 4));
    const uint8_t* dp = a.weights(packed, nb);
    const uint16_t* dc = a.weights(codebooks, nc);
    const float* dx = a.upload(x, (size_t)batch * K);
    float* dy = (float*)a.carve((size_t)batch * M * 4);
    mth_check(mth_oil4_gemv(dp, dc, cb_block, dx, dy, M, K, batch, a.stream()), "oil4_gemv_blocked");
    a.download(y, dy, (size_t)batch * M);
    a.sync();
}

void i2s_gemv_f32(const uint8_t* packed, float w_scale, const float* x, float* y, int M, int K, int batch) {
    check_dims(M, batch, K, "i2s_gemv_f32");
    const size_t nw = (size_t)M * K / 4;
    Arena& a = arena();
    a.begin(P(nw) + P((size_t)batch * K * 4) + P((size_t)batch * M * 4));
    const uint8_t* dw = a.weights(packed, nw);
    const float* dx = a.upload(x, (size_t)batch * K);
    float* dy = (float*)a.carve((size_t)batch * M * 4);
    mth_check(mth_i2s_gemv_f32(dw, w_scale, dx, dy, M, K, batch, a.stream()), "i2s_gemv_f32");
    a.download(y, dy, (size_t)batch * M);
    a.sync();
}

// ---- dense FP32 GEMMs of the same header (src/kernel_i2s.cpp:67-154,236-246)
// C[M][N] = A[M][K] * B[K][N], row-major, C overwritten.  The reference keeps
// four loop orders of one product; all four run as one rocBLAS SGEMM here
// (row-major C = A*B is column-major C^T = B^T * A^T).
namespace {
void dense_gemm(const float* A, const float* B, float* C, int M, int N, int K, const char* what) {
    check_dims(M, N, K, what);
    const size_t na = (size_t)M * K, nb = (size_t)K * N, nc = (size_t)M * N;
    Arena& a = arena();
    a.begin(P(na * 4) + P(nb * 4) + P(nc * 4));
    const float* dA = a.weights(A, na);
    const float* dB = a.weights(B, nb);
    float* dC = (float*)a.carve(nc * 4);
    const float one = 1.0f, zero = 0.0f;
    if (rocblas_sgemm(a.blas(), rocblas_operation_none, rocblas_operation_none, N, M, K, &one, dB, N, dA, K, &zero,
                      dC, N) != rocblas_status_success)
        throw Error(std::string(what) + ": rocblas_sgemm failed");
    a.download(C, dC, nc);
    a.sync();
}
}  // namespace

void scalar_gemm(const float* A, const float* B, float* C, int M, int N, int K) {
    dense_gemm(A, B, C, M, N, K, "scalar_gemm");
}
void tiled_gemm(const float* A, const float* B, float* C, int M, int N, int K) {
    dense_gemm(A, B, C, M, N, K, "tiled_gemm");
}
void avx2_gemm(const float* A, const float* B, float* C, int M, int N, int K) {
    dense_gemm(A, B, C, M, N, K, "avx2_gemm");
}
void avx2_tiled_gemm(const float* A, const float* B, float* C, int M, int N, int K) {
    dense_gemm(A, B, C, M, N, K, "avx2_tiled_gemm");
}

}  // namespace kernel

// ---- weight residency (no reference counterpart) --------------------------
namespace mi355x {
void register_weights(const void* host, size_t bytes) { registry().add(host, bytes); }
bool unregister_weights(const void* host) { return registry().remove(host); }
size_t registered_bytes() { return registry().total(); }
}  // namespace mi355x

// ---- int8 quantisation (src/int8_quant.cpp:8-41) -------------------------

std::vector<Int8QuantParams> quantize_per_token(const float* src, int8_t* dst, int64_t rows, int64_t cols) {
    std::vector<Int8QuantParams> params((size_t)(rows > 0 ? rows : 0));
    if (rows <= 0 || cols <= 0) return params;
    const size_t n = (size_t)rows * (size_t)cols;
    Arena& a = arena();
    a.begin(P(n * 4) + P(n) + 2 * P((size_t)rows * 4));
    const float* dx = a.upload(src, n);
    int8_t* dq = (int8_t*)a.carve(n);
    float* ds = (float*)a.carve((size_t)rows * 4);
    float* di = (float*)a.carve((size_t)rows * 4);
    mth_check(mth_quantize_per_token(dx, dq, ds, di, rows, cols, a.stream()), "quantize_per_token");
    std::vector<float> s((size_t)rows), inv((size_t)rows);
    a.download(dst, dq, n);
    a.download(s.data(), ds, (size_t)rows);
    a.download(inv.data(), di, (size_t)rows);
    a.sync();
    for (int64_t r = 0; r < rows; r++) params[(size_t)r] = Int8QuantParams{s[(size_t)r], inv[(size_t)r]};
    return params;
}

Int8QuantParams quantize_per_tensor(const float* src, int8_t* dst, int64_t n) {
    if (n <= 0) {
        // the reference returns scale = 127/1e-10 for an empty tensor
        const float mx = 1e-10f;
        return Int8QuantParams{127.0f / mx, mx / 127.0f};
    }
    return quantize_per_token(src, dst, 1, n)[0];
}

void dequantize_per_tensor(const int8_t* src, float* dst, int64_t n, float inv_scale) {
    if (n <= 0) return;
    Arena& a = arena();
    a.begin(P((size_t)n) + P((size_t)n * 4));
    const int8_t* dq = a.upload(src, (size_t)n);
    float* dy = (float*)a.carve((size_t)n * 4);
    mth_check(mth_dequantize_per_tensor(dq, dy, n, inv_scale, a.stream()), "dequantize_per_tensor");
    a.download(dst, dy, (size_t)n);
    a.sync();
}

Int8QuantParams quantize_tensor(const Tensor& src, Tensor& dst) {
    return quantize_per_tensor(src.data<float>(), dst.data<int8_t>(), src.numel());
}

}  // namespace oil
