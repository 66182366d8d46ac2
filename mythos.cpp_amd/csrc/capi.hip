// capi.hip — the extern "C" boundary of libmythos_oil.so (include/mythos_oil.h).
//
// Validates every argument, then hands the call to a launcher.  Errors are
// returned as negative codes with a thread-local message, mirroring the
// reference C API's thread_local g_last_error (src/production.cpp:206-217);
// nothing here throws across the C boundary.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

#include "launch.h"
#include "../../include/mythos_oil.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = '\0';
    return MTH_OK;
}

int check_launch(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(MTH_EDEVICE, "%s: launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

inline hipStream_t S(mth_stream_t s) { return (hipStream_t)s; }

// int32 row/column indices are used inside kernels for the fast paths; the
// generic kernels index with int64.  Reject sizes whose byte counts overflow.
constexpr int64_t kMaxDim = (int64_t)1 << 40;

// Device scratch of the batched OIL4 GEMV (partial sums of its K slices),
// one per (device, stream): calls on one stream are ordered and may share it;
// another stream gets its own.  Grown on demand, never shrunk.
struct Workspace {
    void* base = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

hipError_t bt_workspace(hipStream_t s, int64_t M, int64_t K, float** partial) {
    const size_t need = mth::oil4_bt_partial_bytes(M, K);
    *partial = nullptr;
    if (need == 0) return hipSuccess;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> g(g_ws_mu);
    Workspace& w = g_ws[{dev, s}];
    if (w.bytes < need) {
        void* p = nullptr;
        e = hipMalloc(&p, need);
        if (e != hipSuccess) return e;
        if (w.base) {
            (void)hipStreamSynchronize(s);  // earlier launches on s may still use it
            (void)hipFree(w.base);
        }
        w.base = p;
        w.bytes = need;
    }
    *partial = (float*)w.base;
    return hipSuccess;
}

#define REQUIRE(cond, ...) \
    do {                   \
        if (!(cond)) return fail(MTH_EINVAL, __VA_ARGS__); \
    } while (0)

}  // namespace

extern "C" {

const char* mth_last_error(void) { return g_err; }
int mth_version(void) { return (1 << 16) | 0; }

int mth_oil8_gemm(const uint8_t* indices, const float* codebook, const float* act, float* out,
                  int64_t M, int64_t N, int64_t K, mth_stream_t stream) {
    REQUIRE(indices && codebook && act && out, "mth_oil8_gemm: null pointer");
    REQUIRE(M > 0 && N > 0 && K > 0 && M < kMaxDim && N < kMaxDim && K < kMaxDim && M * N < kMaxDim,
            "mth_oil8_gemm: bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
    return check_launch(mth::launch_oil8_gemm_mn(indices, codebook, act, out, M, N, K, S(stream)), "mth_oil8_gemm");
}

int mth_oil8_gemv(const uint8_t* indices, const float* codebook, const float* x, float* y,
                  int64_t M, int64_t K, int64_t batch, mth_stream_t stream) {
    REQUIRE(indices && codebook && x && y, "mth_oil8_gemv: null pointer");
    REQUIRE(M > 0 && K > 0 && batch > 0 && M < kMaxDim && K < kMaxDim && batch <= 65536,
            "mth_oil8_gemv: bad sizes M=%lld K=%lld batch=%lld", (long long)M, (long long)K, (long long)batch);
    return check_launch(mth::launch_oil8_gemv(indices, codebook, x, y, M, K, batch, S(stream)), "mth_oil8_gemv");
}

int mth_oil4_gemm(const uint8_t* packed, const uint16_t* codebook, const float* act, float* out,
                  int64_t M, int64_t N, int64_t K, mth_stream_t stream) {
    REQUIRE(packed && codebook && act && out, "mth_oil4_gemm: null pointer");
    REQUIRE(M > 0 && N > 0 && K > 0 && M < kMaxDim && N < kMaxDim && K < kMaxDim && M * N < kMaxDim,
            "mth_oil4_gemm: bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
    return check_launch(mth::launch_oil4_gemm_mn(packed, codebook, act, out, M, N, K, S(stream)), "mth_oil4_gemm");
}

int mth_oil4_gemv(const uint8_t* packed, const uint16_t* codebooks, int64_t cb_block, const float* x,
                  float* y, int64_t M, int64_t K, int64_t batch, mth_stream_t stream) {
    REQUIRE(packed && codebooks && x && y, "mth_oil4_gemv: null pointer");
    REQUIRE(M > 0 && K > 0 && batch > 0 && M < kMaxDim && K < kMaxDim && batch <= 65536,
            "mth_oil4_gemv: bad sizes M=%lld K=%lld batch=%lld", (long long)M, (long long)K, (long long)batch);
    REQUIRE(K % 2 == 0, "mth_oil4_gemv: K=%lld must be even (two nibbles per byte)", (long long)K);
    REQUIRE(cb_block >= 0, "mth_oil4_gemv: cb_block=%lld < 0", (long long)cb_block);
    REQUIRE(cb_block == 0 || K % cb_block == 0, "mth_oil4_gemv: K=%lld not a multiple of cb_block=%lld",
            (long long)K, (long long)cb_block);
    const bool aligned = (((uintptr_t)packed | (uintptr_t)codebooks | (uintptr_t)x) & 15u) == 0;
    if (aligned && mth::oil4_bt_supported(M, K, cb_block, batch)) {
        float* partial = nullptr;
        const hipError_t e = bt_workspace(S(stream), M, K, &partial);
        if (e != hipSuccess)
            return fail(MTH_EDEVICE, "mth_oil4_gemv: workspace allocation failed: %s", hipGetErrorString(e));
        return check_launch(mth::launch_oil4_gemv_bt(packed, codebooks, cb_block, x, y, M, K, batch, partial, S(stream)),
                            "mth_oil4_gemv");
    }
    return check_launch(mth::launch_oil4_gemv(packed, codebooks, cb_block, x, y, M, K, batch, S(stream)),
                        "mth_oil4_gemv");
}

int mth_oil4_gemm_prefill(const uint16_t* a_bf16, const uint8_t* packed, const uint16_t* codebooks,
                          int64_t cb_block, uint16_t* c_bf16, int64_t M, int64_t N, int64_t K,
                          mth_stream_t stream) {
    REQUIRE(a_bf16 && packed && codebooks && c_bf16, "mth_oil4_gemm_prefill: null pointer");
    REQUIRE(M > 0 && N > 0 && K > 0 && M < kMaxDim && N < kMaxDim && K < kMaxDim,
            "mth_oil4_gemm_prefill: bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
    REQUIRE(K % 2 == 0, "mth_oil4_gemm_prefill: K=%lld must be even", (long long)K);
    REQUIRE(cb_block > 0 && K % cb_block == 0, "mth_oil4_gemm_prefill: K=%lld not a multiple of cb_block=%lld",
            (long long)K, (long long)cb_block);
    const bool aligned = (((uintptr_t)a_bf16 | (uintptr_t)packed | (uintptr_t)codebooks) & 15u) == 0;
    if (!aligned || !mth::oil4_gemm_prefill_supported(M, N, K, cb_block))
        return fail(MTH_EUNSUPPORTED,
                    "mth_oil4_gemm_prefill: M=%lld N=%lld K=%lld cb_block=%lld not supported "
                    "(needs K %% 32 == 0, cb_block %% 32 == 0, 16-byte aligned inputs)",
                    (long long)M, (long long)N, (long long)K, (long long)cb_block);
    return check_launch(mth::launch_oil4_gemm_prefill(a_bf16, packed, codebooks, cb_block, c_bf16, M, N, K, S(stream)),
                        "mth_oil4_gemm_prefill");
}

int mth_quantize_per_token(const float* src, int8_t* dst, float* scale, float* inv_scale, int64_t rows,
                           int64_t cols, mth_stream_t stream) {
    REQUIRE(src && dst, "mth_quantize_per_token: null pointer");
    REQUIRE(rows > 0 && cols > 0 && rows < (1ll << 31) && cols < kMaxDim,
            "mth_quantize_per_token: bad sizes rows=%lld cols=%lld", (long long)rows, (long long)cols);
    return check_launch(mth::launch_quantize_per_token(src, dst, scale, inv_scale, rows, cols, S(stream)),
                        "mth_quantize_per_token");
}

int mth_dequantize_per_tensor(const int8_t* src, float* dst, int64_t n, float inv_scale, mth_stream_t stream) {
    REQUIRE(src && dst, "mth_dequantize_per_tensor: null pointer");
    REQUIRE(n > 0 && n < kMaxDim, "mth_dequantize_per_tensor: bad size n=%lld", (long long)n);
    return check_launch(mth::launch_dequantize(src, dst, n, inv_scale, S(stream)), "mth_dequantize_per_tensor");
}

int mth_tl_precompute_lut(const int8_t* act, int8_t* lut, int64_t K, int group, mth_stream_t stream) {
    REQUIRE(act && lut, "mth_tl_precompute_lut: null pointer");
    REQUIRE(group == 2 || group == 3, "mth_tl_precompute_lut: group=%d must be 2 or 3", group);
    REQUIRE(K >= group && K < kMaxDim, "mth_tl_precompute_lut: bad K=%lld", (long long)K);
    REQUIRE(group == 2 || K % 3 == 0, "mth_tl_precompute_lut: K=%lld must be a multiple of 3", (long long)K);
    return check_launch(mth::launch_tl_precompute_lut(act, lut, K, group, S(stream)), "mth_tl_precompute_lut");
}

int mth_i2s_gemv(const uint8_t* packed, float w_scale, const int8_t* act, const float* act_scale, float* y,
                 int64_t M, int64_t K, int64_t batch, mth_stream_t stream) {
    REQUIRE(packed && act && act_scale && y, "mth_i2s_gemv: null pointer");
    REQUIRE(M > 0 && K > 0 && batch > 0 && M < kMaxDim && K < (1ll << 24) && batch <= 65536,
            "mth_i2s_gemv: bad sizes M=%lld K=%lld batch=%lld", (long long)M, (long long)K, (long long)batch);
    REQUIRE(K % 4 == 0, "mth_i2s_gemv: K=%lld must be a multiple of 4", (long long)K);
    return check_launch(mth::launch_i2s_gemv(packed, w_scale, nullptr, act, act_scale, y, M, K, batch, S(stream)),
                        "mth_i2s_gemv");
}

int mth_i2s_gemv_f32(const uint8_t* packed, float w_scale, const float* x, float* y, int64_t M, int64_t K,
                     int64_t batch, mth_stream_t stream) {
    REQUIRE(packed && x && y, "mth_i2s_gemv_f32: null pointer");
    REQUIRE(M > 0 && K > 0 && batch > 0 && M < kMaxDim && K < (1ll << 24) && batch <= 65536,
            "mth_i2s_gemv_f32: bad sizes M=%lld K=%lld batch=%lld", (long long)M, (long long)K, (long long)batch);
    REQUIRE(K % 4 == 0, "mth_i2s_gemv_f32: K=%lld must be a multiple of 4", (long long)K);
    return check_launch(mth::launch_i2s_gemv(packed, w_scale, x, nullptr, nullptr, y, M, K, batch, S(stream)),
                        "mth_i2s_gemv_f32");
}

int mth_i2s_gemm(const uint8_t* w, const float* act, float* out, int64_t M, int64_t N, int64_t K,
                 mth_stream_t stream) {
    REQUIRE(w && act && out, "mth_i2s_gemm: null pointer");
    REQUIRE(M > 0 && N > 0 && K > 0 && M * N < kMaxDim && K < kMaxDim, "mth_i2s_gemm: bad sizes");
    return check_launch(mth::launch_i2s_gemm(w, act, out, M, N, K, S(stream)), "mth_i2s_gemm");
}

int mth_i2s_gemm_vnni(const uint8_t* w, const int8_t* act, float* out, int64_t M, int64_t N, int64_t K,
                      mth_stream_t stream) {
    REQUIRE(w && act && out, "mth_i2s_gemm_vnni: null pointer");
    REQUIRE(M > 0 && N > 0 && K > 0 && M * N < kMaxDim && K < (1ll << 24), "mth_i2s_gemm_vnni: bad sizes");
    return check_launch(mth::launch_i2s_gemm_vnni(w, act, out, M, N, K, S(stream)), "mth_i2s_gemm_vnni");
}

int mth_tl1_gemm(const uint8_t* w, const float* act, float* out, int64_t M, int64_t N, int64_t K,
                 mth_stream_t stream) {
    REQUIRE(w && act && out, "mth_tl1_gemm: null pointer");
    REQUIRE(M > 0 && N > 0 && K > 0 && M * N < kMaxDim && K < (1ll << 24), "mth_tl1_gemm: bad sizes");
    return check_launch(mth::launch_tl1_gemm(w, act, out, M, N, K, S(stream)), "mth_tl1_gemm");
}

int mth_tl2_gemm(const uint8_t* w, const float* act, float* out, int64_t M, int64_t N, int64_t K,
                 mth_stream_t stream) {
    REQUIRE(w && act && out, "mth_tl2_gemm: null pointer");
    REQUIRE(M > 0 && N > 0 && K > 0 && M * N < kMaxDim && K < (1ll << 24), "mth_tl2_gemm: bad sizes");
    REQUIRE(K % 3 == 0, "mth_tl2_gemm: K=%lld must be a multiple of 3", (long long)K);
    return check_launch(mth::launch_tl2_gemm(w, act, out, M, N, K, S(stream)), "mth_tl2_gemm");
}

}  // extern "C"
