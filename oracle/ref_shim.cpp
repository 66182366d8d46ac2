// ref_shim.cpp — extern "C" entry points over the reference's own kernels,
// compiled together with the reference sources that lie under
// /root/reference/src by oracle/Makefile into oracle/_ref/ (never committed,
// never shipped as source).  TEST INFRASTRUCTURE ONLY: it is the checker that
// pins the oracle restatement (tests/golden/make_golden.py writes its outputs
// as fixtures) and, on the GPU box, the timed "reference" CPU baseline.
//
// Nothing here re-implements reference behaviour: each function only marshals
// plain pointers into the reference's Tensor / free-function API.
#include "oil/kernel.h"
#include "oil/int8_quant.h"
#include "oil/codebook.h"
#include "oil/random.h"
#include "oil/math.h"
#include "oil/tensor.h"
#include "oil/oil_format.h"

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

using namespace oil;

static Tensor make_u8(const uint8_t* p, int64_t n) {
    Tensor t(Shape{n}, DType::U8);
    std::memcpy(t.data(), p, (size_t)n);
    return t;
}
static Tensor make_f32(const float* p, int64_t n) {
    Tensor t(Shape{n}, DType::F32);
    std::memcpy(t.data(), p, (size_t)n * 4);
    return t;
}

extern "C" {

void ref_oil8_gemm(const uint8_t* idx, const float* cb, const float* act, float* out,
                   int M, int N, int K) {
    kernel::oil8_gemm(idx, cb, act, out, M, N, K);
}

// kernel::scalar_gemm (src/kernel_i2s.cpp:91-102): C[m][n] = sum_k A[m*K+k]*B[k*N+n],
// the product Linear::forward uses (src/transformer.cpp:62-70).
void ref_scalar_gemm(const float* A, const float* B, float* C, int M, int N, int K) {
    kernel::scalar_gemm(A, B, C, M, N, K);
}

void ref_oil4_gemm(const uint8_t* nib, const uint16_t* cb, const float* act, float* out,
                   int M, int N, int K) {
    kernel::oil4_gemm(nib, cb, act, out, M, N, K);
}

// Fills g_i2s_lut (kernel_i2s.cpp:24-30 is only reached through i2s_gemm*).
void ref_i2s_init(void) {
    Tensor w(Shape{1, 1}, DType::U8), a(Shape{4}, DType::F32), o(Shape{1}, DType::F32);
    kernel::i2s_gemm(w, a, o, 1, 1, 4);
}

void ref_i2s_gemv(const uint8_t* packed_w, float w_scale, const int8_t* act, float act_scale,
                  float* out, int K) {
    kernel::i2s_gemv(packed_w, w_scale, act, act_scale, out, K);
}

void ref_i2s_gemm(const uint8_t* w, const float* a, float* o, int M, int N, int K) {
    Tensor tw = make_u8(w, (int64_t)M * (K / 4));
    Tensor ta = make_f32(a, (int64_t)N * K);
    Tensor to(Shape{(int64_t)M * N}, DType::F32);
    kernel::i2s_gemm(tw, ta, to, M, N, K);
    std::memcpy(o, to.data(), (size_t)M * N * 4);
}

void ref_i2s_gemm_vnni(const uint8_t* w, const int8_t* a, float* o, int M, int N, int K) {
    kernel::i2s_gemm_vnni(w, a, o, M, N, K);
}

void ref_tl1_gemm(const uint8_t* w, const float* a, float* o, int M, int N, int K) {
    Tensor tw = make_u8(w, (int64_t)M * N * K / 4 + 64);
    Tensor ta = make_f32(a, (int64_t)N * K);
    Tensor to(Shape{(int64_t)M * N}, DType::F32);
    kernel::tl1_gemm(tw, ta, to, M, N, K);
    std::memcpy(o, to.data(), (size_t)M * N * 4);
}

void ref_tl2_gemm(const uint8_t* w, const float* a, float* o, int M, int N, int K) {
    const int64_t bpr = ((int64_t)K * 2 + 7) / 8;
    Tensor tw(Shape{(int64_t)M * N * bpr + 64}, DType::U8);   // zero padded past the rows
    std::memcpy(tw.data(), w, (size_t)(M * N * bpr));
    Tensor ta = make_f32(a, (int64_t)N * K);
    Tensor to(Shape{(int64_t)M * N}, DType::F32);
    kernel::tl2_gemm(tw, ta, to, M, N, K);
    std::memcpy(o, to.data(), (size_t)M * N * 4);
}

void ref_quantize_per_token(const float* src, int8_t* dst, int64_t rows, int64_t cols,
                            float* scale, float* inv_scale) {
    auto p = quantize_per_token(src, dst, rows, cols);
    for (int64_t r = 0; r < rows; r++) {
        scale[r] = p[(size_t)r].scale;
        inv_scale[r] = p[(size_t)r].inv_scale;
    }
}

uint16_t ref_float_to_half(float f) { return CodebookOIL4::float_to_half(f); }
float ref_half_to_float(uint16_t h) { return CodebookOIL4::half_to_float(h); }

void ref_rng_u64(uint64_t seed, uint64_t* out, int64_t n) {
    RNG r(seed);
    for (int64_t i = 0; i < n; i++) out[i] = r.next_u64();
}
void ref_rng_uniform(uint64_t seed, float* out, int64_t n) {
    RNG r(seed);
    for (int64_t i = 0; i < n; i++) out[i] = r.uniform();
}
void ref_rng_normal(uint64_t seed, float* out, int64_t n) {
    RNG r(seed);
    for (int64_t i = 0; i < n; i++) out[i] = r.normal();
}
void ref_rng_uniform_int(uint64_t seed, int lo, int hi, int32_t* out, int64_t n) {
    RNG r(seed);
    for (int64_t i = 0; i < n; i++) out[i] = r.uniform_int(lo, hi);
}

void ref_gemv(float alpha, const float* A, const float* x, float beta, float* y, int64_t M, int64_t N) {
    Tensor tA = make_f32(A, M * N).view(Shape{M, N});
    Tensor tx = make_f32(x, N);
    Tensor ty = make_f32(y, M);
    math::gemv(alpha, tA, tx, beta, ty);
    std::memcpy(y, ty.data(), (size_t)M * 4);
}

void ref_rms_norm(const float* x, const float* g, float eps, float* y, int64_t rows, int64_t dim) {
    Tensor tx = make_f32(x, rows * dim).view(Shape{rows, dim});
    Tensor tg = make_f32(g, dim);
    Tensor ty(Shape{rows, dim}, DType::F32);
    math::rms_norm(tx, tg, eps, ty);
    std::memcpy(y, ty.data(), (size_t)(rows * dim) * 4);
}

void ref_softmax(const float* x, float* y, int64_t rows, int64_t dim) {
    Tensor tx = make_f32(x, rows * dim).view(Shape{rows, dim});
    Tensor ty(Shape{rows, dim}, DType::F32);
    math::softmax(tx, ty, -1);
    std::memcpy(y, ty.data(), (size_t)(rows * dim) * 4);
}

void ref_silu(const float* x, float* y, int64_t n) {
    Tensor tx = make_f32(x, n);
    Tensor ty(Shape{n}, DType::F32);
    math::silu(tx, ty);
    std::memcpy(y, ty.data(), (size_t)n * 4);
}

// ---- .oil container (src/oil_format.cpp, src/codebook.cpp) ---------------
// Serialised codebooks exactly as CodebookOIL8/OIL4::serialize write them.
int64_t ref_serialize_oil8(const float* centroids, uint8_t* dst) {
    CodebookOIL8 cb;
    std::memcpy(cb.centroids, centroids, sizeof(cb.centroids));
    return (int64_t)cb.serialize(dst);
}
int64_t ref_serialize_oil4(const uint16_t* centroids, uint8_t* dst) {
    CodebookOIL4 cb;
    std::memcpy(cb.centroids, centroids, sizeof(cb.centroids));
    return (int64_t)cb.serialize(dst);
}

// Writes a .oil file with OILWriter: header (+ config), format table, tensor
// table, then every block.  Blocks are given in file order: formats[b],
// nweights[b], cb_sizes[b] bytes of codebook_data, idx_sizes[b] bytes of
// index_data (both concatenated).  Tensor t owns blocks
// [block_start[t], block_start[t] + num_blocks[t]).
void ref_oil_write(const char* path, const uint8_t* config, uint32_t config_size, int nblocks,
                   const uint8_t* formats, const uint32_t* nweights, const uint32_t* cb_sizes,
                   const uint8_t* codebook_data, const uint32_t* idx_sizes, const uint8_t* index_data,
                   int ntensors, const char* const* names, const uint32_t* block_start, const uint32_t* num_blocks) {
    OILWriter w(path);
    OILHeader h;
    std::memcpy(h.magic, "OIL1", 4);
    h.version = (1u << 22);
    h.flags = 0;
    h.config_size = config_size;
    w.write_header(h, config);
    std::vector<FormatBlockEntry> ft((size_t)nblocks);
    for (int b = 0; b < nblocks; b++) {
        ft[(size_t)b].block_id = (uint32_t)b;
        ft[(size_t)b].format = formats[b];
        ft[(size_t)b].cb_bytes = cb_sizes[b];
    }
    w.write_format_table(ft);
    std::vector<TensorEntry> te((size_t)ntensors);
    std::vector<std::string> nm((size_t)ntensors);
    for (int t = 0; t < ntensors; t++) {
        nm[(size_t)t] = names[t];
        te[(size_t)t].name_len = (uint16_t)nm[(size_t)t].size();
        te[(size_t)t].block_start = block_start[t];
        te[(size_t)t].num_blocks = num_blocks[t];
    }
    w.write_tensor_table(te, nm);
    size_t co = 0, io = 0;
    for (int b = 0; b < nblocks; b++) {
        BlockData bd;
        bd.num_weights = nweights[b];
        bd.codebook.assign(codebook_data + co, codebook_data + co + cb_sizes[b]);
        bd.indices.assign(index_data + io, index_data + io + idx_sizes[b]);
        co += cb_sizes[b];
        io += idx_sizes[b];
        w.write_block(bd);
    }
    w.close();
}

// OILReader::read_tensor: the reference's dequantised FP32 copy of a tensor.
// Returns the number of weights (0 if absent), writes at most cap floats.
int64_t ref_oil_read_tensor(const char* path, const char* name, float* out, int64_t cap) {
    OILReader r(path);
    if (!r.valid()) return -1;
    Tensor t = r.read_tensor(name);
    const int64_t n = t.numel();
    if (n > 0 && out) std::memcpy(out, t.data(), (size_t)(n < cap ? n : cap) * 4);
    return n;
}

}  // extern "C"
