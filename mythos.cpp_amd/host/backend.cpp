// backend.cpp — the HIP ComputeBackend (oil/backend.h): the reference's
// dispatch (include/oil/backend.h:49-80, src/backend.cpp:421-438) with the
// vtable's dense operators running on MI355X.
//
// Each call checks shapes as the reference's math:: function does (same
// conditions, oil::Error on failure), stages the host tensors in the
// backend's device arena, runs the libmythos_oil.so kernels (rocBLAS SGEMM
// for the product of gemm) on the backend's stream and copies the result
// back before returning.  Semantics per operator (src/math.cpp):
//   gemm   :74-97   C = alpha * (A B) + beta * C  (SGEMM into scratch, then
//                   mth_axpby: each product and the sum rounded, C read even
//                   when beta = 0, as the reference's loop reads it)
//   gemv   :52-72   mth_gemv_f32
//   softmax :207-249 over `axis` (negative counts from the end): mth_softmax_axis
//   layer_norm :148-180, rms_norm :182-205 over the last axis
//   relu, gelu, silu, add, mul, scale: elementwise over numel
// copy / fill / zero act on the host tensors (Tensor::copy_from / fill /
// zero_), as the reference's backends do.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <mutex>
#include <string>

#include "mythos_oil.h"
#include "oil/backend.h"
#include "oil/mi355x.h"
#include "staging.h"

namespace oil {
namespace backend {
namespace {

using detail::Arena;
using detail::hip_check;
using detail::mth_check;
using detail::P;

// Makes `dev` current for the scope and restores the caller's device.
class DeviceScope {
public:
    explicit DeviceScope(int dev) {
        hip_check(hipGetDevice(&prev_), "hipGetDevice");
        if (prev_ != dev) hip_check(hipSetDevice(dev), "hipSetDevice");
        set_ = prev_ != dev;
    }
    ~DeviceScope() {
        if (set_) (void)hipSetDevice(prev_);
    }

private:
    int prev_ = 0;
    bool set_ = false;
};

int64_t last_dim(const Tensor& x) { return x.rank() ? x.shape().dims[x.rank() - 1] : 1; }

class HIPBackend final : public ComputeBackend {
public:
    explicit HIPBackend(int device) : dev_(device) {}
    ~HIPBackend() override {
        // the arena's stream, buffer and rocBLAS handle belong to dev_
        int n = 0;
        if (hipGetDeviceCount(&n) == hipSuccess && dev_ < n) {
            int prev = 0;
            if (hipGetDevice(&prev) == hipSuccess) {
                (void)hipSetDevice(dev_);
                arena_.reset();
                (void)hipSetDevice(prev);
                return;
            }
        }
        arena_.reset();
    }

    BackendType type() const override { return BackendType::GPU_CUDA; }
    const char* name() const override { return "GPU_HIP_MI355X"; }

    void gemm(float alpha, const Tensor& A, const Tensor& B, float beta, Tensor& C) override {
        OIL_CHECK(A.shape().rank == 2, "gemm A must be 2D");
        OIL_CHECK(B.shape().rank == 2, "gemm B must be 2D");
        OIL_CHECK(C.shape().rank == 2, "gemm C must be 2D");
        const int64_t M = A.dim(0), K = A.dim(1), N = B.dim(1);
        OIL_CHECK(B.dim(0) == K, "gemm A cols != B rows");
        OIL_CHECK(C.dim(0) == M && C.dim(1) == N, "gemm C shape mismatch");
        if (M == 0 || N == 0) return;
        OIL_CHECK(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31), "gemm: dimension too large for SGEMM");
        Run r(*this, P(M * K * 4) + P(K * N * 4) + P(M * N * 4) * 2);
        const float* dA = r.a.upload(A.data<float>(), (size_t)(M * K));
        const float* dB = r.a.upload(B.data<float>(), (size_t)(K * N));
        float* dC = r.a.upload(C.data<float>(), (size_t)(M * N));
        float* dT = (float*)r.a.carve((size_t)(M * N) * 4);
        if (K == 0) {
            hip_check(hipMemsetAsync(dT, 0, (size_t)(M * N) * 4, (hipStream_t)r.a.stream()), "gemm: clear");
        } else {
            const float one = 1.0f, zero = 0.0f;  // row-major T = A B is column-major T^T = B^T A^T
            if (rocblas_sgemm(r.a.blas(), rocblas_operation_none, rocblas_operation_none, (int)N, (int)M, (int)K,
                              &one, dB, (int)N, dA, (int)K, &zero, dT, (int)N) != rocblas_status_success)
                throw Error("gemm: rocblas_sgemm failed");
        }
        mth_check(mth_axpby(alpha, dT, beta, dC, M * N, r.a.stream()), "gemm");
        r.a.download(C.data<float>(), dC, (size_t)(M * N));
        r.a.sync();
    }

    void gemv(float alpha, const Tensor& A, const Tensor& x, float beta, Tensor& y) override {
        OIL_CHECK(A.shape().rank == 2, "gemv A must be 2D");
        OIL_CHECK(x.shape().rank == 1, "gemv x must be 1D");
        OIL_CHECK(y.shape().rank == 1, "gemv y must be 1D");
        const int64_t M = A.dim(0), N = A.dim(1);
        OIL_CHECK(x.numel() == N, "gemv x size != A cols");
        OIL_CHECK(y.numel() == M, "gemv y size != A rows");
        if (M == 0) return;
        if (N == 0) {  // s = 0 for every row
            Run r(*this, P(M * 4) * 2);
            float* dy = r.a.upload(y.data<float>(), (size_t)M);
            float* dz = (float*)r.a.carve((size_t)M * 4);
            hip_check(hipMemsetAsync(dz, 0, (size_t)M * 4, (hipStream_t)r.a.stream()), "gemv: clear");
            mth_check(mth_axpby(alpha, dz, beta, dy, M, r.a.stream()), "gemv");
            r.a.download(y.data<float>(), dy, (size_t)M);
            r.a.sync();
            return;
        }
        Run r(*this, P(M * N * 4) + P(N * 4) + P(M * 4));
        const float* dA = r.a.upload(A.data<float>(), (size_t)(M * N));
        const float* dx = r.a.upload(x.data<float>(), (size_t)N);
        float* dy = r.a.upload(y.data<float>(), (size_t)M);
        mth_check(mth_gemv_f32(alpha, dA, dx, beta, dy, M, N, r.a.stream()), "gemv");
        r.a.download(y.data<float>(), dy, (size_t)M);
        r.a.sync();
    }

    void softmax(const Tensor& x, Tensor& y, int axis) override {
        OIL_CHECK(x.numel() == y.numel(), "softmax shape mismatch");
        const Shape& s = x.shape();
        if (axis < 0) axis += s.rank;
        OIL_CHECK(axis >= 0 && axis < s.rank, "softmax axis out of range");
        int64_t outer = 1, inner = 1;
        for (int i = 0; i < axis; i++) outer *= s.dims[i];
        for (int i = axis + 1; i < s.rank; i++) inner *= s.dims[i];
        const int64_t dim = s.dims[axis], n = x.numel();
        if (n == 0) return;
        Run r(*this, P(n * 4));
        float* d = r.a.upload(x.data<float>(), (size_t)n);
        mth_check(mth_softmax_axis(d, d, outer, dim, inner, r.a.stream()), "softmax");
        r.a.download(y.data<float>(), d, (size_t)n);
        r.a.sync();
    }

    void layer_norm(const Tensor& x, const Tensor& gamma, const Tensor& beta, float eps, Tensor& y) override {
        OIL_CHECK(x.numel() == y.numel(), "layer_norm shape mismatch");
        OIL_CHECK(gamma.numel() == last_dim(x), "layer_norm gamma dim mismatch");
        OIL_CHECK(beta.numel() == last_dim(x), "layer_norm beta dim mismatch");
        const int64_t dim = last_dim(x), n = x.numel();
        if (n == 0) return;
        Run r(*this, P(n * 4) * 2 + P(dim * 4) * 2);
        const float* dx = r.a.upload(x.data<float>(), (size_t)n);
        const float* dg = r.a.upload(gamma.data<float>(), (size_t)dim);
        const float* db = r.a.upload(beta.data<float>(), (size_t)dim);
        float* dy = (float*)r.a.carve((size_t)n * 4);
        mth_check(mth_layer_norm(dx, dg, db, dy, n / dim, dim, eps, r.a.stream()), "layer_norm");
        r.a.download(y.data<float>(), dy, (size_t)n);
        r.a.sync();
    }

    void rms_norm(const Tensor& x, const Tensor& gamma, float eps, Tensor& y) override {
        OIL_CHECK(x.numel() == y.numel(), "rms_norm shape mismatch");
        OIL_CHECK(gamma.numel() == last_dim(x), "rms_norm gamma dim mismatch");
        const int64_t dim = last_dim(x), n = x.numel();
        if (n == 0) return;
        Run r(*this, P(n * 4) + P(dim * 4));
        float* dx = r.a.upload(x.data<float>(), (size_t)n);
        const float* dg = r.a.upload(gamma.data<float>(), (size_t)dim);
        mth_check(mth_rms_norm(dx, dg, dx, n / dim, dim, eps, r.a.stream()), "rms_norm");
        r.a.download(y.data<float>(), dx, (size_t)n);
        r.a.sync();
    }

    void relu(const Tensor& x, Tensor& y) override { unary(x, y, "relu shape mismatch", mth_relu, "relu"); }
    void gelu(const Tensor& x, Tensor& y) override { unary(x, y, "gelu shape mismatch", mth_gelu, "gelu"); }
    void silu(const Tensor& x, Tensor& y) override { unary(x, y, "silu shape mismatch", mth_silu, "silu"); }
    void add(const Tensor& a, const Tensor& b, Tensor& c) override { binary(a, b, c, "add shape mismatch", mth_add, "add"); }
    void mul(const Tensor& a, const Tensor& b, Tensor& c) override { binary(a, b, c, "mul shape mismatch", mth_mul, "mul"); }

    void scale(float s, const Tensor& x, Tensor& y) override {
        OIL_CHECK(x.numel() == y.numel(), "scale shape mismatch");
        const int64_t n = x.numel();
        if (n == 0) return;
        Run r(*this, P(n * 4));
        float* d = r.a.upload(x.data<float>(), (size_t)n);
        mth_check(mth_scale(s, d, d, n, r.a.stream()), "scale");
        r.a.download(y.data<float>(), d, (size_t)n);
        r.a.sync();
    }

    void copy(const Tensor& src, Tensor& dst) override { dst.copy_from(src); }
    void fill(Tensor& t, float val) override { t.fill(val); }
    void zero(Tensor& t) override { t.zero_(); }

    bool is_available() const override {
        int n = 0;
        return hipGetDeviceCount(&n) == hipSuccess && dev_ >= 0 && dev_ < n;
    }
    int64_t memory_free() const override { return mem_info(true); }
    int64_t memory_total() const override { return mem_info(false); }
    void synchronize() override {
        if (!is_available()) return;
        DeviceScope ds(dev_);
        hip_check(hipDeviceSynchronize(), "synchronize");
    }

private:
    // One operator's use of the arena: the backend's device current and the
    // arena held for the call.
    struct Run {
        Run(HIPBackend& b, size_t bytes) : lock(b.mu_), dev((b.require(), b.dev_)), a(*b.arena_) { a.begin(bytes); }
        std::lock_guard<std::mutex> lock;
        DeviceScope dev;
        Arena& a;
    };

    void require() {
        if (!is_available()) throw Error(std::string("GPU_CUDA backend: no HIP device ") + std::to_string(dev_));
    }

    int64_t mem_info(bool free) const {
        if (!is_available()) return 0;
        DeviceScope ds(dev_);
        size_t f = 0, t = 0;
        hip_check(hipMemGetInfo(&f, &t), "hipMemGetInfo");
        return (int64_t)(free ? f : t);
    }

    void unary(const Tensor& x, Tensor& y, const char* shape_msg, int (*op)(const float*, float*, int64_t, mth_stream_t),
               const char* what) {
        OIL_CHECK(x.numel() == y.numel(), shape_msg);
        const int64_t n = x.numel();
        if (n == 0) return;
        Run r(*this, P(n * 4));
        float* d = r.a.upload(x.data<float>(), (size_t)n);
        mth_check(op(d, d, n, r.a.stream()), what);
        r.a.download(y.data<float>(), d, (size_t)n);
        r.a.sync();
    }

    void binary(const Tensor& a, const Tensor& b, Tensor& c, const char* shape_msg,
                int (*op)(const float*, const float*, float*, int64_t, mth_stream_t), const char* what) {
        OIL_CHECK(a.numel() == b.numel() && b.numel() == c.numel(), shape_msg);
        const int64_t n = a.numel();
        if (n == 0) return;
        Run r(*this, P(n * 4) * 2);
        float* da = r.a.upload(a.data<float>(), (size_t)n);
        const float* db = r.a.upload(b.data<float>(), (size_t)n);
        mth_check(op(da, db, da, n, r.a.stream()), what);
        r.a.download(c.data<float>(), da, (size_t)n);
        r.a.sync();
    }

    const int dev_;
    std::mutex mu_;
    std::unique_ptr<Arena> arena_ = std::make_unique<Arena>();
};

}  // namespace
}  // namespace backend

backend::ComputeBackend* mi355x::make_hip_backend(int64_t device_id) {
    OIL_CHECK(device_id >= 0 && device_id < (1 << 30), "make_hip_backend: bad device_id");
    return new backend::HIPBackend((int)device_id);
}

namespace backend {
// Standalone library: the factory and the probes.  Compiled into the
// reference's tree (OIL_HAS_MI355X), its src/backend.cpp keeps its own and
// calls mi355x::make_hip_backend from the GPU_CUDA case.
#if !defined(OIL_HAS_MI355X)
ComputeBackend* ComputeBackend::create(const BackendConfig& cfg) {
    switch (cfg.type) {
        case BackendType::GPU_CUDA: return mi355x::make_hip_backend(cfg.device_id);
        default: return nullptr;  // not built here: see oil/backend.h
    }
}

bool is_cuda_available() {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess && n > 0;
}

int64_t gpu_memory_free(int64_t device_id) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device_id < 0 || device_id >= n) return 0;
    DeviceScope ds((int)device_id);
    size_t f = 0, t = 0;
    if (hipMemGetInfo(&f, &t) != hipSuccess) return 0;
    return (int64_t)f;
}
#endif

}  // namespace backend
}  // namespace oil
