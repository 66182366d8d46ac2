// backend_test.cpp — the HIP ComputeBackend (oil/backend.h of
// libmythos_host.so) driven the way the reference's tests drive a backend
// (tests/test_all.cpp:244-336: create, the add / gemm / relu / scale checks,
// memory), then every vtable operator against closed forms that hold exactly
// (small-integer operands make gemm / gemv sums exact; relu, add, mul, scale
// by powers of two are exact in FP32) or against float64 evaluations of the
// reference's formulas (src/math.cpp) with FP32 bounds.  Needs a GPU; run by
// tests/test_gpu_backend.py.  One line per check; non-zero exit on failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <random>
#include <vector>

#include "oil/backend.h"

using namespace oil;
using namespace oil::backend;

static int g_fail = 0;
#define CHECK(name, cond)                                   \
    do {                                                    \
        bool ok_ = (cond);                                  \
        std::printf("%s %s\n", ok_ ? "PASS" : "FAIL", name); \
        if (!ok_) ++g_fail;                                 \
    } while (0)

static float* F(Tensor& t) { return t.data<float>(); }

int main() {
    std::mt19937 rng(20261201);
    auto uni = [&](int lo, int hi) { return (float)std::uniform_int_distribution<int>(lo, hi)(rng); };
    auto nrm = [&](double s) { return (float)(std::normal_distribution<double>(0.0, s)(rng)); };

    std::unique_ptr<ComputeBackend> be(ComputeBackend::create(BackendConfig{BackendType::GPU_CUDA}));
    CHECK("GPU_CUDA created", be != nullptr);
    if (!be) return 1;
    CHECK("type and name", be->type() == BackendType::GPU_CUDA && std::strlen(be->name()) > 0);
    CHECK("is_available", be->is_available() && is_cuda_available());
    CHECK("memory", be->memory_free() > 0 && be->memory_total() >= be->memory_free() && gpu_memory_free(0) > 0);
    CHECK("types not built here give nullptr",
          ComputeBackend::create(BackendConfig{BackendType::CPU_SCALAR}) == nullptr &&
              ComputeBackend::create(BackendConfig{BackendType::DISTRIBUTED}) == nullptr);

    // ---- the reference's test_backend_ops (tests/test_all.cpp:244-276) ----
    {
        Tensor a({2, 3}), b({2, 3}), c({2, 3});
        a.fill(2.0f);
        b.fill(3.0f);
        be->add(a, b, c);
        CHECK("add (reference check)", std::fabs(F(c)[0] - 5.0f) < 1e-5f);
        Tensor A({2, 3}), B({3, 4}), C({2, 4});
        A.fill(1.0f);
        B.fill(2.0f);
        be->gemm(1.0f, A, B, 0.0f, C);
        CHECK("gemm (reference check)", std::fabs(F(C)[0] - 6.0f) < 1e-5f);
        Tensor rx({2, 4}), ry({2, 4});
        rx.fill(-1.0f);
        be->relu(rx, ry);
        bool ok = F(ry)[0] == 0.0f;
        rx.fill(3.0f);
        be->relu(rx, ry);
        CHECK("relu (reference check)", ok && F(ry)[0] == 3.0f);
        Tensor sx({2, 3}), sy({2, 3});
        sx.fill(2.0f);
        be->scale(3.0f, sx, sy);
        CHECK("scale (reference check)", std::fabs(F(sy)[0] - 6.0f) < 1e-5f);
    }

    // ---- gemm: integer operands, alpha/beta, C read when beta = 0 ----------
    {
        const int M = 67, N = 45, K = 129;
        Tensor A({M, K}), B({K, N}), C({M, N});
        for (int i = 0; i < M * K; i++) F(A)[i] = uni(-8, 8);
        for (int i = 0; i < K * N; i++) F(B)[i] = uni(-8, 8);
        for (int i = 0; i < M * N; i++) F(C)[i] = uni(-8, 8);
        std::vector<float> want(M * N);
        for (int i = 0; i < M; i++)
            for (int j = 0; j < N; j++) {
                int64_t s = 0;
                for (int k = 0; k < K; k++) s += (int64_t)F(A)[i * K + k] * (int64_t)F(B)[k * N + j];
                want[i * N + j] = 2.0f * (float)s + -0.5f * F(C)[i * N + j];
            }
        be->gemm(2.0f, A, B, -0.5f, C);
        CHECK("gemm integer exact, alpha/beta", std::memcmp(F(C), want.data(), want.size() * 4) == 0);
        Tensor C2({M, N});
        C2.fill(0.0f);
        F(C2)[7] = NAN;
        F(C2)[11] = INFINITY;
        be->gemm(1.0f, A, B, 0.0f, C2);
        CHECK("gemm beta=0 still reads C (0*NaN, 0*Inf)", std::isnan(F(C2)[7]) && std::isnan(F(C2)[11]) &&
                                                             std::isfinite(F(C2)[8]));
        bool threw = false;
        Tensor Bad({K + 1, N});
        try {
            be->gemm(1.0f, A, Bad, 0.0f, C);
        } catch (const Error&) {
            threw = true;
        }
        CHECK("gemm shape mismatch throws oil::Error", threw);
    }

    // ---- gemv: integers exact, float within FP32 reordering ----------------
    {
        const int M = 513, N = 1025;
        Tensor A({M, N}), x{Shape(N)}, y{Shape(M)};
        for (int i = 0; i < M * N; i++) F(A)[i] = uni(-8, 8);
        for (int i = 0; i < N; i++) F(x)[i] = uni(-8, 8);
        for (int i = 0; i < M; i++) F(y)[i] = uni(-8, 8);
        std::vector<float> want(M);
        for (int i = 0; i < M; i++) {
            int64_t s = 0;
            for (int j = 0; j < N; j++) s += (int64_t)F(A)[i * N + j] * (int64_t)F(x)[j];
            want[i] = 0.75f * (float)s + 1.5f * F(y)[i];
        }
        be->gemv(0.75f, A, x, 1.5f, y);
        CHECK("gemv integer exact", std::memcmp(F(y), want.data(), M * 4) == 0);
        for (int i = 0; i < M * N; i++) F(A)[i] = nrm(1.0);
        for (int i = 0; i < N; i++) F(x)[i] = nrm(1.0);
        be->gemv(1.0f, A, x, 0.0f, y);
        bool ok = true;
        for (int i = 0; i < M; i++) {
            double s = 0, a = 0;
            for (int j = 0; j < N; j++) {
                s += (double)F(A)[i * N + j] * F(x)[j];
                a += std::fabs((double)F(A)[i * N + j] * F(x)[j]);
            }
            ok &= std::fabs(F(y)[i] - s) <= 1e-5 * a;
        }
        CHECK("gemv float within 1e-5 sum|a x|", ok);
    }

    // ---- softmax along each axis -------------------------------------------
    {
        const int D0 = 3, D1 = 17, D2 = 9;
        Tensor x({D0, D1, D2}), y({D0, D1, D2});
        for (int i = 0; i < D0 * D1 * D2; i++) F(x)[i] = nrm(4.0);
        for (int axis : {0, 1, 2, -1}) {
            be->softmax(x, y, axis);
            const int ax = axis < 0 ? axis + 3 : axis;
            const int dims[3] = {D0, D1, D2};
            int outer = 1, inner = 1;
            for (int i = 0; i < ax; i++) outer *= dims[i];
            for (int i = ax + 1; i < 3; i++) inner *= dims[i];
            const int dim = dims[ax];
            bool ok = true;
            for (int o = 0; o < outer; o++)
                for (int in = 0; in < inner; in++) {
                    double mx = -INFINITY, sum = 0;
                    for (int d = 0; d < dim; d++) mx = std::fmax(mx, F(x)[(o * dim + d) * inner + in]);
                    for (int d = 0; d < dim; d++) sum += std::exp((double)F(x)[(o * dim + d) * inner + in] - mx);
                    for (int d = 0; d < dim; d++) {
                        const int idx = (o * dim + d) * inner + in;
                        const double w = std::exp((double)F(x)[idx] - mx) / sum;
                        // FP32 x - max is rounded before expf: the exponential
                        // carries |x - max| ulps of that argument
                        const double arg = std::fabs((double)F(x)[idx] - mx);
                        ok &= std::fabs(F(y)[idx] - w) <= (4e-7 + 1.2e-7 * arg) * w + 1e-30;
                    }
                }
            char name[64];
            std::snprintf(name, sizeof name, "softmax axis %d vs float64", axis);
            CHECK(name, ok);
        }
    }

    // ---- layer_norm / rms_norm over the last axis ----------------------------
    {
        const int R = 4, D = 1000;
        Tensor x({R, D}), g{Shape(D)}, b{Shape(D)}, y({R, D});
        for (int i = 0; i < R * D; i++) F(x)[i] = nrm(2.0) + (float)(i / D) * 5.0f;
        for (int i = 0; i < D; i++) F(g)[i] = 0.5f + (float)(i % 7) * 0.125f, F(b)[i] = nrm(1.0);
        be->layer_norm(x, g, b, 1e-5f, y);
        bool ok = true;
        for (int r = 0; r < R; r++) {
            double mu = 0, var = 0;
            for (int j = 0; j < D; j++) mu += F(x)[r * D + j];
            mu /= D;
            for (int j = 0; j < D; j++) var += ((double)F(x)[r * D + j] - mu) * ((double)F(x)[r * D + j] - mu);
            var /= D;
            for (int j = 0; j < D; j++) {
                const double z = ((double)F(x)[r * D + j] - mu) / std::sqrt(var + 1e-5);
                const double w = z * F(g)[j] + F(b)[j];
                ok &= std::fabs(F(y)[r * D + j] - w) <= 4e-7 * (std::fabs(z * F(g)[j]) + std::fabs(w)) + 1e-30;
            }
        }
        CHECK("layer_norm vs float64", ok);
        be->rms_norm(x, g, 1e-5f, y);
        ok = true;
        for (int r = 0; r < R; r++) {
            double ss = 0;
            for (int j = 0; j < D; j++) ss += (double)F(x)[r * D + j] * F(x)[r * D + j];
            const double inv = 1.0 / std::sqrt(ss / D + 1e-5);
            for (int j = 0; j < D; j++) {
                const double w = F(x)[r * D + j] * inv * F(g)[j];
                ok &= std::fabs(F(y)[r * D + j] - w) <= 3e-7 * std::fabs(w) + 1e-30;
            }
        }
        CHECK("rms_norm vs float64", ok);
    }

    // ---- elementwise ----------------------------------------------------------
    {
        const int n = 70001;
        Tensor a{Shape(n)}, b{Shape(n)}, c{Shape(n)};
        for (int i = 0; i < n; i++) F(a)[i] = uni(-1000, 1000), F(b)[i] = uni(-1000, 1000);
        be->add(a, b, c);
        bool ok = true;
        for (int i = 0; i < n; i++) ok &= F(c)[i] == F(a)[i] + F(b)[i];
        CHECK("add exact", ok);
        be->mul(a, b, c);
        ok = true;
        for (int i = 0; i < n; i++) ok &= F(c)[i] == F(a)[i] * F(b)[i];
        CHECK("mul exact", ok);
        be->scale(-0.25f, a, c);
        ok = true;
        for (int i = 0; i < n; i++) ok &= F(c)[i] == -0.25f * F(a)[i];
        CHECK("scale exact", ok);
        for (int i = 0; i < n; i++) F(a)[i] = nrm(3.0);
        be->silu(a, c);
        ok = true;
        for (int i = 0; i < n; i++) {
            const double v = F(a)[i], w = v / (1.0 + std::exp(-v));
            ok &= std::fabs(F(c)[i] - w) <= 4e-7 * std::fabs(w) + 1e-30;
        }
        CHECK("silu vs float64", ok);
        be->gelu(a, c);
        ok = true;
        for (int i = 0; i < n; i++) {
            const double v = F(a)[i], w = 0.5 * v * (1.0 + std::erf(v / std::sqrt(2.0)));
            ok &= std::fabs(F(c)[i] - w) <= 4e-7 * std::fabs(w) + 2.5e-7 * std::fabs(0.5 * v) + 1e-37;
        }
        CHECK("gelu vs float64", ok);
        be->relu(a, c);
        ok = true;
        for (int i = 0; i < n; i++) ok &= F(c)[i] == (F(a)[i] > 0.0f ? F(a)[i] : 0.0f);
        CHECK("relu exact", ok);
    }

    // ---- copy / fill / zero, synchronize, empty tensors ----------------------
    {
        Tensor a({3, 5}), b({5, 3});
        for (int i = 0; i < 15; i++) F(a)[i] = (float)i;
        be->copy(a, b);
        bool ok = std::memcmp(F(a), F(b), 60) == 0;
        be->fill(b, 2.5f);
        for (int i = 0; i < 15; i++) ok &= F(b)[i] == 2.5f;
        be->zero(b);
        for (int i = 0; i < 15; i++) ok &= F(b)[i] == 0.0f;
        be->synchronize();
        Tensor e0(Shape(0)), e1(Shape(0));
        be->relu(e0, e1);
        CHECK("copy / fill / zero / synchronize / empty", ok);
    }

    std::printf("%d failures\n", g_fail);
    return g_fail ? 1 : 0;
}
