// capi.hip — the extern "C" boundary of libmythos_oil.so (include/mythos_oil.h).
//
// Validates every argument, then hands the call to a launcher.  Errors are
// returned as negative codes with a thread-local message, mirroring the
// reference C API's thread_local g_last_error (src/production.cpp:206-217);
// nothing here throws across the C boundary.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

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
// batches of at least this many tokens run the OIL8 / OIL4 GEMVs as MFMA GEMMs
constexpr int64_t kGemmRows = 128;

// Device scratch (partial sums of the batched GEMVs' K slices, argmax
// partials), one per (device, stream): calls on one stream are ordered and
// may share it; another stream gets its own.
//
// Growth allocates a new block (at least twice the old size) and RETIRES the
// old one without freeing it: launches already queued, and any HIP graph
// captured earlier from calls on that stream, keep using the old address, so
// it stays valid until the process ends.  Doubling bounds the retired memory
// by the final block's size.  Growth never happens inside a stream capture
// (hipMalloc is not capturable): such a call fails with MTH_EUNSUPPORTED and
// the caller reserves the size first (mth_workspace_reserve) or makes one
// uncaptured call of that shape.
struct Workspace {
    void* base = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
std::vector<void*> g_ws_retired;  // superseded blocks: valid until the process ends

// hipSuccess, or hipErrorStreamCaptureUnsupported when growing under capture
hipError_t workspace(hipStream_t s, size_t need, void** out) {
    *out = nullptr;
    if (need == 0) return hipSuccess;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> g(g_ws_mu);
    Workspace& w = g_ws[{dev, s}];
    if (w.bytes < need) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(s, &st);
        if (e != hipSuccess) return e;
        if (st != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        const size_t bytes = std::max(need, 2 * w.bytes);
        void* p = nullptr;
        e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return e;
        if (w.base) g_ws_retired.push_back(w.base);
        w.base = p;
        w.bytes = bytes;
    }
    *out = w.base;
    return hipSuccess;
}

int workspace_fail(const char* what, hipError_t e, size_t need) {
    if (e == hipErrorStreamCaptureUnsupported)
        return fail(MTH_EUNSUPPORTED,
                    "%s: needs %zu bytes of workspace on this stream, more than it holds, and the stream is "
                    "capturing; call mth_workspace_reserve (or this call uncaptured) before the capture",
                    what, need);
    return fail(MTH_EDEVICE, "%s: workspace allocation of %zu bytes failed: %s", what, need, hipGetErrorString(e));
}

#define REQUIRE(cond, ...) \
    do {                   \
        if (!(cond)) return fail(MTH_EINVAL, __VA_ARGS__); \
    } while (0)

// Scratch of mth_oil4_gemv_noalloc: the K-slice partial sums of the batched
// OIL4 GEMV, in a fixed device array instead of the allocated workspace.  The
// array's name is a host-side stand-in; the device address comes from
// hipGetSymbolAddress, once per device, with that device current.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the calling thread's current device's scratch.
hipError_t scratch_address(void** out) {
    *out = nullptr;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace

namespace mth {
int api_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}
int api_ok() { return ok(); }
}  // namespace mth

extern "C" {

const char* mth_last_error(void) { return g_err; }
// 2.0: mth_decoder_config gained struct_size (first member); 1.x callers of
// mth_decoder_create are rejected by its size check.
int mth_version(void) { return (2 << 16) | 0; }

int mth_workspace_reserve(int64_t bytes, mth_stream_t stream) {
    REQUIRE(bytes >= 0 && bytes < kMaxDim, "mth_workspace_reserve: bad size %lld", (long long)bytes);
    void* p = nullptr;
    const hipError_t e = workspace(S(stream), (size_t)bytes, &p);
    if (e != hipSuccess) return workspace_fail("mth_workspace_reserve", e, (size_t)bytes);
    return ok();
}

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
    const bool aligned = (((uintptr_t)indices | (uintptr_t)x) & 15u) == 0;
    const mth::Oil8Seg seg{indices, codebook, y, M};
    if (aligned && batch >= kGemmRows && mth::oil8_gemm_x32_supported(&seg, 1, batch, K)) {
        // >= 128 tokens: the MFMA GEMM (each weight read once per 128 tokens)
        void* ws = nullptr;
        const size_t need = mth::oil8_gemm_x32_workspace_bytes(batch, K);
        const hipError_t e = workspace(S(stream), need, &ws);
        if (e != hipSuccess) return workspace_fail("mth_oil8_gemv", e, need);
        return check_launch(mth::launch_oil8_gemm_x32(x, &seg, 1, batch, K, ws, S(stream)), "mth_oil8_gemv");
    }
    if (aligned && mth::oil8_bt_supported(M, K, batch)) {
        void* partial = nullptr;
        const size_t need = mth::oil8_bt_partial_bytes(M, K);
        const hipError_t e = workspace(S(stream), need, &partial);
        if (e != hipSuccess) return workspace_fail("mth_oil8_gemv", e, need);
        return check_launch(mth::launch_oil8_gemv_bt(indices, codebook, x, y, M, K, batch, (float*)partial, S(stream)),
                            "mth_oil8_gemv");
    }
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
    if (aligned && ((uintptr_t)y & 15u) == 0 && batch >= kGemmRows &&
        mth::oil4_gemm_x32_supported(batch, M, K, cb_block)) {
        // >= 128 tokens: the MFMA GEMM (each weight read once per 128 tokens)
        void* ws = nullptr;
        const size_t need = mth::oil4_gemm_x32_workspace_bytes(batch, K);
        const hipError_t e = workspace(S(stream), need, &ws);
        if (e != hipSuccess) return workspace_fail("mth_oil4_gemv", e, need);
        return check_launch(mth::launch_oil4_gemm_x32(x, packed, codebooks, cb_block, y, batch, M, K, ws, S(stream)),
                            "mth_oil4_gemv");
    }
    if (aligned && mth::oil4_bt_supported(M, K, cb_block, batch)) {
        void* partial = nullptr;
        const size_t need = mth::oil4_bt_partial_bytes(M, K);
        const hipError_t e = workspace(S(stream), need, &partial);
        if (e != hipSuccess) return workspace_fail("mth_oil4_gemv", e, need);
        return check_launch(mth::launch_oil4_gemv_bt(packed, codebooks, cb_block, x, y, M, K, batch, (float*)partial,
                                                     S(stream)),
                            "mth_oil4_gemv");
    }
    return check_launch(mth::launch_oil4_gemv(packed, codebooks, cb_block, x, y, M, K, batch, S(stream)),
                        "mth_oil4_gemv");
}

int mth_oil4_gemv_noalloc(const uint8_t* packed, const uint16_t* codebooks, int64_t cb_block, const float* x,
                          float* y, int64_t M, int64_t K, int64_t batch, mth_stream_t stream) {
    REQUIRE(packed && codebooks && x && y, "mth_oil4_gemv_noalloc: null pointer");
    REQUIRE(M > 0 && K > 0 && batch > 0 && M < kMaxDim && K < kMaxDim && batch <= 65536,
            "mth_oil4_gemv_noalloc: bad sizes M=%lld K=%lld batch=%lld", (long long)M, (long long)K,
            (long long)batch);
    REQUIRE(K % 2 == 0, "mth_oil4_gemv_noalloc: K=%lld must be even (two nibbles per byte)", (long long)K);
    REQUIRE(cb_block >= 0, "mth_oil4_gemv_noalloc: cb_block=%lld < 0", (long long)cb_block);
    REQUIRE(cb_block == 0 || K % cb_block == 0, "mth_oil4_gemv_noalloc: K=%lld not a multiple of cb_block=%lld",
            (long long)K, (long long)cb_block);
    const bool aligned = (((uintptr_t)packed | (uintptr_t)codebooks | (uintptr_t)x) & 15u) == 0;
    if (aligned && mth::oil4_bt_supported(M, K, cb_block, batch)) {
        const size_t need = mth::oil4_bt_partial_bytes(M, K);
        REQUIRE(need <= kNoAllocScratchBytes,
                "mth_oil4_gemv_noalloc: M=%lld K=%lld batch=%lld needs %zu bytes of scratch, more than the %zu "
                "this entry point holds; use mth_oil4_gemv",
                (long long)M, (long long)K, (long long)batch, need, kNoAllocScratchBytes);
        void* partial = nullptr;
        const hipError_t e = scratch_address(&partial);
        if (e != hipSuccess)
            return fail(MTH_EDEVICE, "mth_oil4_gemv_noalloc: scratch address: %s", hipGetErrorString(e));
        return check_launch(mth::launch_oil4_gemv_bt(packed, codebooks, cb_block, x, y, M, K, batch, (float*)partial,
                                                     S(stream)),
                            "mth_oil4_gemv_noalloc");
    }
    return check_launch(mth::launch_oil4_gemv(packed, codebooks, cb_block, x, y, M, K, batch, S(stream)),
                        "mth_oil4_gemv_noalloc");
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
    const bool aligned = (((uintptr_t)a_bf16 | (uintptr_t)packed | (uintptr_t)codebooks | (uintptr_t)c_bf16) & 15u) == 0;
    if (!aligned || !mth::oil4_gemm_prefill_supported(M, N, K, cb_block))
        return fail(MTH_EUNSUPPORTED,
                    "mth_oil4_gemm_prefill: M=%lld N=%lld K=%lld cb_block=%lld not supported "
                    "(needs K %% 32 == 0, cb_block %% 32 == 0, 16-byte aligned inputs)",
                    (long long)M, (long long)N, (long long)K, (long long)cb_block);
    // workspace: the per-row shifts of A, then (FP16-A kernels) A in FP16
    const size_t a16 = mth::oil4_prefill_workspace_bytes(M, N, K, cb_block);
    const size_t need = mth::oil4_prefill_shift_bytes(M) + a16;
    void* ws = nullptr;
    const hipError_t e = workspace(S(stream), need, &ws);
    if (e != hipSuccess) return workspace_fail("mth_oil4_gemm_prefill", e, need);
    if (a16)
        return check_launch(mth::launch_oil4_gemm_prefill_a16(a_bf16, packed, codebooks, cb_block, c_bf16, M, N, K, ws,
                                                             S(stream)),
                            "mth_oil4_gemm_prefill");
    return check_launch(mth::launch_oil4_gemm_prefill(a_bf16, packed, codebooks, cb_block, c_bf16, M, N, K, (int*)ws,
                                                      S(stream)),
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
    const bool aligned = (((uintptr_t)packed | (uintptr_t)act) & 15u) == 0;
    if (aligned && mth::i2s_bt_supported(M, K, batch)) {
        void* partial = nullptr;
        const size_t need = mth::i2s_bt_partial_bytes(M, K);
        const hipError_t e = workspace(S(stream), need, &partial);
        if (e != hipSuccess) return workspace_fail("mth_i2s_gemv", e, need);
        return check_launch(mth::launch_i2s_gemv_bt(packed, w_scale, act, act_scale, y, M, K, batch, (float*)partial,
                                                    S(stream)),
                            "mth_i2s_gemv");
    }
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
    const size_t need = mth::tl2_workspace_bytes(w, M, N, K);
    if (need) {
        void* ws = nullptr;
        const hipError_t e = workspace(S(stream), need, &ws);
        if (e != hipSuccess) return workspace_fail("mth_tl2_gemm", e, need);
        return check_launch(mth::launch_tl2_gemm_ws(w, act, out, M, N, K, ws, S(stream)), "mth_tl2_gemm");
    }
    return check_launch(mth::launch_tl2_gemm(w, act, out, M, N, K, S(stream)), "mth_tl2_gemm");
}

// ---- FP32 decode-step operators -------------------------------------------
int mth_rms_norm(const float* x, const float* gamma, float* y, int64_t rows, int64_t dim, float eps,
                 mth_stream_t stream) {
    REQUIRE(x && gamma && y, "mth_rms_norm: null pointer");
    REQUIRE(rows > 0 && rows < (1ll << 31) && dim > 0 && dim < kMaxDim, "mth_rms_norm: bad sizes");
    REQUIRE(eps >= 0.0f, "mth_rms_norm: eps < 0");
    return check_launch(mth::launch_rms_norm((float*)x, nullptr, gamma, y, rows, dim, eps, S(stream)),
                        "mth_rms_norm");
}

int mth_add_rms_norm(float* x, const float* t, const float* gamma, float* y, int64_t rows, int64_t dim, float eps,
                     mth_stream_t stream) {
    REQUIRE(x && t && gamma && y, "mth_add_rms_norm: null pointer");
    REQUIRE(rows > 0 && rows < (1ll << 31) && dim > 0 && dim < kMaxDim, "mth_add_rms_norm: bad sizes");
    REQUIRE(eps >= 0.0f, "mth_add_rms_norm: eps < 0");
    return check_launch(mth::launch_rms_norm(x, t, gamma, y, rows, dim, eps, S(stream)), "mth_add_rms_norm");
}

int mth_silu(const float* x, float* y, int64_t n, mth_stream_t stream) {
    REQUIRE(x && y, "mth_silu: null pointer");
    REQUIRE(n > 0 && n < kMaxDim, "mth_silu: bad size");
    return check_launch(mth::launch_silu(x, y, n, S(stream)), "mth_silu");
}

int mth_silu_mul(const float* g, const float* u, float* y, int64_t rows, int64_t n, int64_t gstride,
                 int64_t ustride, mth_stream_t stream) {
    REQUIRE(g && u && y, "mth_silu_mul: null pointer");
    REQUIRE(rows > 0 && rows <= 65535 && n > 0 && n < (1ll << 31) && gstride >= n && ustride >= n,
            "mth_silu_mul: bad sizes");
    return check_launch(mth::launch_silu_mul(g, u, y, rows, n, gstride, ustride, S(stream)), "mth_silu_mul");
}

int mth_silu_mul_quant(const float* g, const float* u, int8_t* q, float* inv_scale, int64_t rows, int64_t n,
                       int64_t gstride, int64_t ustride, mth_stream_t stream) {
    REQUIRE(g && u && q && inv_scale, "mth_silu_mul_quant: null pointer");
    REQUIRE(rows > 0 && rows <= 65535 && gstride >= n && ustride >= n, "mth_silu_mul_quant: bad sizes");
    REQUIRE(mth::silu_mul_quant_supported(n), "mth_silu_mul_quant: n=%lld outside 1..12288", (long long)n);
    return check_launch(mth::launch_silu_mul_quant(g, u, q, inv_scale, nullptr, rows, n, gstride, ustride, S(stream)),
                        "mth_silu_mul_quant");
}

int mth_oil4_gemv_swiglu(const uint8_t* packed, const uint16_t* codebooks, const float* x, float* act,
                         float* amax, int64_t F, int64_t K, mth_stream_t stream) {
    REQUIRE(packed && codebooks && x && act && amax, "mth_oil4_gemv_swiglu: null pointer");
    REQUIRE(mth::oil4_swiglu_supported(packed, codebooks, x, F, K),
            "mth_oil4_gemv_swiglu: F=%lld K=%lld not supported (F %% 8 == 0, K %% 512 == 0, 512 <= K <= 4096, "
            "16-byte aligned packed/codebooks/x)",
            (long long)F, (long long)K);
    return check_launch(mth::launch_oil4_swiglu(packed, codebooks, x, mth::NormScale{}, act, amax, F, K, S(stream)),
                        "mth_oil4_gemv_swiglu");
}

int mth_i2s_gemv_act(const uint8_t* packed, float w_scale, const float* act, const float* amax, float* y,
                     int64_t M, int64_t K, mth_stream_t stream) {
    REQUIRE(packed && act && amax && y, "mth_i2s_gemv_act: null pointer");
    REQUIRE(M > 0 && K > 0 && M < kMaxDim, "mth_i2s_gemv_act: bad sizes M=%lld K=%lld", (long long)M,
            (long long)K);
    REQUIRE(mth::i2s_swiglu_supported(packed, M, K) && (((uintptr_t)act & 15u) == 0),
            "mth_i2s_gemv_act: K=%lld not supported (K %% 64 == 0, K <= 12288, 16-byte aligned packed and act)",
            (long long)K);
    return check_launch(mth::launch_i2s_act(act, amax, packed, w_scale, y, M, K, mth::ResidOut{}, nullptr,
                                            S(stream)),
                        "mth_i2s_gemv_act");
}

int64_t mth_swiglu_batch_parts(int64_t F) { return F > 0 && F < kMaxDim ? mth::oil4_bt_swiglu_parts(F) : 0; }

int mth_oil4_gemv_swiglu_batch(const uint8_t* packed, const uint16_t* codebooks, int64_t cb_block, const float* x,
                               float* gu, float* amax, int64_t F, int64_t K, int64_t batch, mth_stream_t stream) {
    REQUIRE(packed && codebooks && x && gu && amax, "mth_oil4_gemv_swiglu_batch: null pointer");
    REQUIRE(F > 0 && K > 0 && F < kMaxDim && K < kMaxDim, "mth_oil4_gemv_swiglu_batch: bad sizes F=%lld K=%lld",
            (long long)F, (long long)K);
    REQUIRE(batch >= 2 && batch <= 16, "mth_oil4_gemv_swiglu_batch: batch=%lld outside 2..16", (long long)batch);
    REQUIRE((((uintptr_t)packed | (uintptr_t)codebooks | (uintptr_t)x) & 15u) == 0,
            "mth_oil4_gemv_swiglu_batch: packed, codebooks and x must be 16-byte aligned");
    REQUIRE(mth::oil4_bt_swiglu_supported(F, K, cb_block, batch),
            "mth_oil4_gemv_swiglu_batch: F=%lld K=%lld cb_block=%lld not supported (F %% 4 == 0, K %% 512 == 0, "
            "512 <= K <= 8192, cb_block 0 or 128)",
            (long long)F, (long long)K, (long long)cb_block);
    void* partial = nullptr;
    const size_t need = mth::oil4_bt_partial_bytes(2 * F, K);
    const hipError_t e = workspace(S(stream), need, &partial);
    if (e != hipSuccess) return workspace_fail("mth_oil4_gemv_swiglu_batch", e, need);
    return check_launch(mth::launch_oil4_gemv_bt_swiglu(packed, codebooks, cb_block, x, mth::NormScale{}, gu, amax, F,
                                                        K, batch, (float*)partial, S(stream)),
                        "mth_oil4_gemv_swiglu_batch");
}

int mth_i2s_gemv_act_batch(const uint8_t* packed, float w_scale, const float* act, int64_t lda, const float* amax,
                           float* inv_scale, float* y, int64_t M, int64_t K, int64_t batch, mth_stream_t stream) {
    REQUIRE(packed && act && amax && inv_scale && y, "mth_i2s_gemv_act_batch: null pointer");
    REQUIRE(M > 0 && K > 0 && M < (1ll << 31) && K <= 16384, "mth_i2s_gemv_act_batch: bad sizes M=%lld K=%lld",
            (long long)M, (long long)K);
    REQUIRE(batch >= 2 && batch <= 16, "mth_i2s_gemv_act_batch: batch=%lld outside 2..16", (long long)batch);
    REQUIRE(lda >= K && lda % 4 == 0 && lda < kMaxDim, "mth_i2s_gemv_act_batch: lda=%lld (>= K, multiple of 4)",
            (long long)lda);
    REQUIRE((((uintptr_t)packed | (uintptr_t)act) & 15u) == 0,
            "mth_i2s_gemv_act_batch: packed and act must be 16-byte aligned");
    REQUIRE(mth::i2s_bt_supported(M, K, batch), "mth_i2s_gemv_act_batch: K=%lld not a multiple of 256", (long long)K);
    void* partial = nullptr;
    const size_t need = mth::i2s_bt_partial_bytes(M, K);
    const hipError_t e = workspace(S(stream), need, &partial);
    if (e != hipSuccess) return workspace_fail("mth_i2s_gemv_act_batch", e, need);
    return check_launch(mth::launch_i2s_gemv_bt_f32act_y(packed, w_scale, act, lda, amax, mth::oil4_bt_swiglu_parts(K),
                                                         inv_scale, y, M, K, batch, (float*)partial, S(stream)),
                        "mth_i2s_gemv_act_batch");
}

int mth_add(const float* a, const float* b, float* c, int64_t n, mth_stream_t stream) {
    REQUIRE(a && b && c, "mth_add: null pointer");
    REQUIRE(n > 0 && n < kMaxDim, "mth_add: bad size");
    return check_launch(mth::launch_add(a, b, c, n, S(stream)), "mth_add");
}

int mth_mul(const float* a, const float* b, float* c, int64_t n, mth_stream_t stream) {
    REQUIRE(a && b && c, "mth_mul: null pointer");
    REQUIRE(n > 0 && n < kMaxDim, "mth_mul: bad size");
    return check_launch(mth::launch_mul(a, b, c, n, S(stream)), "mth_mul");
}

int mth_softmax(const float* x, float* y, int64_t rows, int64_t dim, mth_stream_t stream) {
    REQUIRE(x && y, "mth_softmax: null pointer");
    REQUIRE(rows > 0 && rows < (1ll << 31) && dim > 0 && dim < kMaxDim, "mth_softmax: bad sizes");
    return check_launch(mth::launch_softmax(x, y, rows, dim, S(stream)), "mth_softmax");
}

int mth_softmax_axis(const float* x, float* y, int64_t outer, int64_t dim, int64_t inner, mth_stream_t stream) {
    REQUIRE(x && y, "mth_softmax_axis: null pointer");
    REQUIRE(outer > 0 && dim > 0 && inner > 0 && outer < kMaxDim && dim < kMaxDim && inner < kMaxDim &&
                outer * inner < kMaxDim && dim * inner < kMaxDim && outer * dim * inner < kMaxDim,
            "mth_softmax_axis: bad sizes outer=%lld dim=%lld inner=%lld", (long long)outer, (long long)dim,
            (long long)inner);
    REQUIRE(inner > 1 || outer < (1ll << 31), "mth_softmax_axis: outer=%lld too large", (long long)outer);
    return check_launch(mth::launch_softmax_axis(x, y, outer, dim, inner, S(stream)), "mth_softmax_axis");
}

int mth_axpby(float alpha, const float* x, float beta, float* y, int64_t n, mth_stream_t stream) {
    REQUIRE(x && y, "mth_axpby: null pointer");
    REQUIRE(n > 0 && n < kMaxDim, "mth_axpby: bad size n=%lld", (long long)n);
    return check_launch(mth::launch_axpby(alpha, x, beta, y, n, S(stream)), "mth_axpby");
}

int mth_gemv_f32(float alpha, const float* A, const float* x, float beta, float* y, int64_t M, int64_t N,
                 mth_stream_t stream) {
    REQUIRE(A && x && y, "mth_gemv_f32: null pointer");
    REQUIRE(M > 0 && N > 0 && M < (1ll << 31) && N < kMaxDim && M * N < kMaxDim,
            "mth_gemv_f32: bad sizes M=%lld N=%lld", (long long)M, (long long)N);
    return check_launch(mth::launch_gemv_f32(alpha, A, x, beta, y, M, N, S(stream)), "mth_gemv_f32");
}

int mth_relu(const float* x, float* y, int64_t n, mth_stream_t stream) {
    REQUIRE(x && y, "mth_relu: null pointer");
    REQUIRE(n > 0 && n < kMaxDim, "mth_relu: bad size n=%lld", (long long)n);
    return check_launch(mth::launch_relu(x, y, n, S(stream)), "mth_relu");
}

int mth_gelu(const float* x, float* y, int64_t n, mth_stream_t stream) {
    REQUIRE(x && y, "mth_gelu: null pointer");
    REQUIRE(n > 0 && n < kMaxDim, "mth_gelu: bad size n=%lld", (long long)n);
    return check_launch(mth::launch_gelu(x, y, n, S(stream)), "mth_gelu");
}

int mth_scale(float s, const float* x, float* y, int64_t n, mth_stream_t stream) {
    REQUIRE(x && y, "mth_scale: null pointer");
    REQUIRE(n > 0 && n < kMaxDim, "mth_scale: bad size n=%lld", (long long)n);
    return check_launch(mth::launch_scale(s, x, y, n, S(stream)), "mth_scale");
}

int mth_layer_norm(const float* x, const float* gamma, const float* beta, float* y, int64_t rows, int64_t dim,
                   float eps, mth_stream_t stream) {
    REQUIRE(x && gamma && beta && y, "mth_layer_norm: null pointer");
    REQUIRE(rows > 0 && rows < (1ll << 31) && dim > 0 && dim < kMaxDim && rows * dim < kMaxDim,
            "mth_layer_norm: bad sizes rows=%lld dim=%lld", (long long)rows, (long long)dim);
    REQUIRE(eps >= 0.0f, "mth_layer_norm: eps < 0");
    return check_launch(mth::launch_layer_norm(x, gamma, beta, y, rows, dim, eps, S(stream)), "mth_layer_norm");
}

int mth_rope_tables(int64_t head_dim, int64_t max_seq, float theta, float* cos_t, float* sin_t) {
    REQUIRE(cos_t && sin_t, "mth_rope_tables: null pointer");
    REQUIRE(head_dim > 0 && head_dim % 2 == 0 && max_seq > 0 && head_dim * max_seq < kMaxDim,
            "mth_rope_tables: bad sizes");
    REQUIRE(theta > 0.0f, "mth_rope_tables: theta <= 0");
    const int64_t h2 = head_dim / 2;
    for (int64_t i = 0; i < max_seq; i++)
        for (int64_t j = 0; j < h2; j++) {
            const float inv_freq = 1.0f / std::pow(theta, (float)(2 * j) / (float)head_dim);
            const float val = (float)i * inv_freq;
            cos_t[i * h2 + j] = std::cos(val);
            sin_t[i * h2 + j] = std::sin(val);
        }
    return ok();
}

int mth_rope_kv(float* q, const float* k, const float* v, const float* cos_t, const float* sin_t, float* kcache,
                float* vcache, int64_t pos, int64_t batch, int64_t heads, int64_t kv_heads, int64_t head_dim,
                int64_t max_seq, mth_stream_t stream) {
    REQUIRE(q && k && v && cos_t && sin_t && kcache && vcache, "mth_rope_kv: null pointer");
    REQUIRE(batch > 0 && batch <= 65535 && heads > 0 && kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 &&
                heads * head_dim < (1ll << 24) && max_seq > 0 && max_seq < (1ll << 24),
            "mth_rope_kv: bad sizes");
    REQUIRE(pos >= 0 && pos < max_seq, "mth_rope_kv: pos=%lld outside 0..%lld", (long long)pos,
            (long long)max_seq - 1);
    return check_launch(mth::launch_rope_kv(q, k, v, cos_t, sin_t, kcache, vcache, nullptr, (int)pos, batch,
                                            (int)heads, (int)kv_heads, (int)head_dim, (int)max_seq, S(stream)),
                        "mth_rope_kv");
}

int mth_attention_decode(const float* q, const float* kcache, const float* vcache, float* out, int64_t batch,
                         int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t ctx, int64_t max_seq,
                         mth_stream_t stream) {
    REQUIRE(q && kcache && vcache && out, "mth_attention_decode: null pointer");
    REQUIRE(batch > 0 && batch <= 65535 && heads > 0 && heads <= 65535 && kv_heads > 0 && heads % kv_heads == 0,
            "mth_attention_decode: bad head counts");
    REQUIRE(max_seq > 0 && mth::attention_supported((int)head_dim, (int)max_seq),
            "mth_attention_decode: head_dim=%lld max_seq=%lld (head_dim 64/128/256, max_seq <= 16384)",
            (long long)head_dim, (long long)max_seq);
    REQUIRE(ctx >= 1 && ctx <= max_seq, "mth_attention_decode: ctx=%lld outside 1..%lld", (long long)ctx,
            (long long)max_seq);
    return check_launch(mth::launch_attention(q, kcache, vcache, out, nullptr, (int)ctx - 1, batch, (int)heads,
                                              (int)kv_heads, (int)head_dim, (int)max_seq, S(stream)),
                        "mth_attention_decode");
}

int mth_argmax(const float* logits, int32_t* ids, int64_t rows, int64_t n, mth_stream_t stream) {
    REQUIRE(logits && ids, "mth_argmax: null pointer");
    REQUIRE(rows > 0 && rows <= 65535 && n > 0 && n < (1ll << 31), "mth_argmax: bad sizes");
    void* ws = nullptr;
    const size_t nc = (size_t)mth::argmax_chunks(n) * (size_t)rows;
    const hipError_t e = workspace(S(stream), nc * 8, &ws);
    if (e != hipSuccess) return workspace_fail("mth_argmax", e, nc * 8);
    return check_launch(mth::launch_argmax(logits, rows, n, ids, nullptr, nullptr, 0, 0, (float*)ws,
                                           (int*)((char*)ws + nc * 4), S(stream)),
                        "mth_argmax");
}

}  // extern "C"
