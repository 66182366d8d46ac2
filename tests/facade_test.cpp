// facade_test.cpp — the C++ drop-in (libmythos_host.so) called the way the
// reference's own code calls oil::kernel::* (host pointers, oil::Tensor,
// synchronous), checked against closed forms that hold exactly: integer
// codebooks and integer activations make every FP32 sum exact, ternary and
// int8 results are integers by definition.  Needs a GPU; run by
// tests/test_gpu_facade.py.  Prints one line per check, exits non-zero on any
// failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "oil/int8_quant.h"
#include "oil/kernel.h"
#include "oil/mi355x.h"

static int g_fail = 0;
#define CHECK(name, cond)                                   \
    do {                                                    \
        bool ok_ = (cond);                                  \
        std::printf("%s %s\n", ok_ ? "PASS" : "FAIL", name); \
        if (!ok_) ++g_fail;                                 \
    } while (0)

template <typename T> static bool same(const std::vector<T>& a, const std::vector<T>& b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(T)) == 0;
}

static uint16_t half_bits(int v) {  // small integers are exact in FP16
    _Float16 h = (_Float16)v;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

int main() {
    std::mt19937 rng(20260601);
    auto uni = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };

    // ---- OIL8: src/kernel_oil8.cpp:14-71, per-(m,n) weight rows ----------
    for (int N : {1, 3}) {
        const int M = 37, K = 301;
        std::vector<uint8_t> idx((size_t)M * N * K);
        std::vector<float> cb(256), x((size_t)N * K), y((size_t)M * N), want((size_t)M * N);
        for (auto& v : idx) v = (uint8_t)uni(0, 255);
        for (int i = 0; i < 256; i++) cb[i] = (float)(i - 128);
        for (auto& v : x) v = (float)uni(-8, 8);
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++) {
                int64_t s = 0;
                for (int k = 0; k < K; k++) s += (int64_t)(idx[((size_t)m * N + n) * K + k] - 128) * (int64_t)x[n * K + k];
                want[m * N + n] = (float)s;
            }
        oil::kernel::oil8_gemm(idx.data(), cb.data(), x.data(), y.data(), M, N, K);
        CHECK(N == 1 ? "oil8_gemm N=1 exact" : "oil8_gemm N=3 exact", same(y, want));
    }

    // ---- OIL4: src/kernel_oil4.cpp:31-54 (scalar definition) -------------
    {
        const int M = 21, N = 2, K = 258;
        std::vector<uint8_t> nib((size_t)M * N * K / 2);
        std::vector<uint16_t> cb(16);
        std::vector<float> x((size_t)N * K), y((size_t)M * N), want((size_t)M * N);
        for (auto& v : nib) v = (uint8_t)uni(0, 255);
        for (int i = 0; i < 16; i++) cb[i] = half_bits(i - 8);
        for (auto& v : x) v = (float)uni(-4, 4);
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++) {
                int64_t s = 0;
                for (int k = 0; k < K; k++) {
                    const size_t e = ((size_t)m * N + n) * K + k;
                    const int code = (e % 2 == 0) ? (nib[e / 2] & 15) : (nib[e / 2] >> 4);
                    s += (int64_t)(code - 8) * (int64_t)x[n * K + k];
                }
                want[m * N + n] = (float)s;
            }
        oil::kernel::oil4_gemm(nib.data(), cb.data(), x.data(), y.data(), M, N, K);
        CHECK("oil4_gemm exact", same(y, want));
    }

    // ---- I2_S: src/kernel_i2s.cpp:13-65,201-235 ---------------------------
    {
        const int M = 9, N = 4, K = 512;
        std::vector<int> t((size_t)M * K);
        std::vector<uint8_t> w((size_t)M * K / 4, 0);
        for (size_t i = 0; i < t.size(); i++) {
            t[i] = uni(-1, 1);
            w[i / 4] |= (uint8_t)((t[i] + 1) << (2 * (i % 4)));
        }
        std::vector<int8_t> ai((size_t)N * K);
        for (auto& v : ai) v = (int8_t)uni(-128, 127);
        std::vector<float> af((size_t)N * K);
        for (size_t i = 0; i < af.size(); i++) af[i] = (float)ai[i];
        std::vector<float> want((size_t)M * N), y((size_t)M * N);
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++) {
                int64_t s = 0;
                for (int k = 0; k < K; k++) s += (int64_t)t[(size_t)m * K + k] * ai[(size_t)n * K + k];
                want[m * N + n] = (float)s;
            }
        oil::kernel::i2s_gemm_vnni(w.data(), ai.data(), y.data(), M, N, K);
        CHECK("i2s_gemm_vnni exact", same(y, want));

        oil::Tensor tw(oil::Shape{(int64_t)w.size()}, oil::DType::U8), ta(oil::Shape{(int64_t)N * K}),
            to(oil::Shape{(int64_t)M * N});
        std::memcpy(tw.data(), w.data(), w.size());
        std::memcpy(ta.data(), af.data(), af.size() * 4);
        oil::kernel::i2s_gemm(tw, ta, to, M, N, K);
        CHECK("i2s_gemm (Tensor) exact", std::memcmp(to.data(), want.data(), want.size() * 4) == 0);
        oil::kernel::i2s_gemm_avx2(tw, ta, to, M, N, K);
        CHECK("i2s_gemm_avx2 (Tensor) exact", std::memcmp(to.data(), want.data(), want.size() * 4) == 0);

        float out = 0.0f;
        const float ws = 0.5f, as = 0.25f;   // powers of two: the epilogue is exact
        oil::kernel::i2s_gemv(w.data(), ws, ai.data(), as, &out, K);
        CHECK("i2s_gemv row 0", out == (float)((double)want[0] * ws * as));
    }

    // ---- int8 quantisation: src/int8_quant.cpp:8-31 ----------------------
    {
        const float xr[8] = {127.0f, 63.5f, -63.5f, 0.5f, -0.5f, 1.5f, -2.5f, -127.0f};
        int8_t q[16];
        float both[16];
        std::memcpy(both, xr, sizeof xr);
        std::memset(both + 8, 0, 8 * sizeof(float));
        auto p = oil::quantize_per_token(both, q, 2, 8);
        const int8_t want[8] = {127, 64, -64, 1, -1, 2, -3, -127};
        bool ok = p.size() == 2 && p[0].scale == 1.0f && p[0].inv_scale == 1.0f && std::memcmp(q, want, 8) == 0;
        for (int i = 8; i < 16; i++) ok = ok && q[i] == 0;
        ok = ok && p[1].inv_scale == 1e-10f / 127.0f;
        CHECK("quantize_per_token ties + zero row", ok);
    }

    // ---- TL2 with integer activations whose max is 127 (scale 1) -----------
    {
        const int M = 3, N = 2, K = 48;
        const size_t bpr = ((size_t)K * 2 + 7) / 8;
        std::vector<int> t((size_t)M * N * K);
        std::vector<uint8_t> w((size_t)M * N * bpr, 0);
        for (int r = 0; r < M * N; r++)
            for (int k = 0; k < K; k++) {
                const int v = uni(-1, 1);
                t[(size_t)r * K + k] = v;
                w[(size_t)r * bpr + k / 4] |= (uint8_t)((v + 1) << (2 * (k % 4)));
            }
        oil::Tensor tw(oil::Shape{(int64_t)w.size()}, oil::DType::U8), ta(oil::Shape{(int64_t)N * K}),
            to(oil::Shape{(int64_t)M * N});
        std::memcpy(tw.data(), w.data(), w.size());
        float* a = ta.data<float>();
        for (int i = 0; i < N * K; i++) a[i] = (float)uni(-100, 100);
        a[0] = 127.0f;
        a[K] = -127.0f;
        oil::kernel::tl2_gemm(tw, ta, to, M, N, K);
        bool ok = true;
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++) {
                int64_t s = 0;
                for (int k = 0; k < K; k++) s += (int64_t)t[((size_t)m * N + n) * K + k] * (int64_t)a[n * K + k];
                ok = ok && to.data<float>()[m * N + n] == (float)s;
            }
        CHECK("tl2_gemm exact", ok);
    }

    // ---- dense FP32 helpers: tests/test_math.cpp:45-72 known answer --------
    {
        const float A[6] = {1, 2, 3, 4, 5, 6}, B[6] = {7, 8, 9, 10, 11, 12};
        const float want[9] = {27, 30, 33, 61, 68, 75, 95, 106, 117};
        float C[9];
        bool ok = true;
        oil::kernel::scalar_gemm(A, B, C, 3, 3, 2);
        ok = ok && std::memcmp(C, want, sizeof C) == 0;
        oil::kernel::tiled_gemm(A, B, C, 3, 3, 2);
        ok = ok && std::memcmp(C, want, sizeof C) == 0;
        oil::kernel::avx2_gemm(A, B, C, 3, 3, 2);
        ok = ok && std::memcmp(C, want, sizeof C) == 0;
        oil::kernel::avx2_tiled_gemm(A, B, C, 3, 3, 2);
        ok = ok && std::memcmp(C, want, sizeof C) == 0;
        CHECK("dense gemm known answer", ok);
    }

    // ---- weight residency ------------------------------------------------
    {
        const int M = 64, K = 256;
        std::vector<uint8_t> idx((size_t)M * K);
        std::vector<float> cb(256), x(K), y0(M), y1(M), y2(M), y3(M);
        for (auto& v : idx) v = (uint8_t)uni(0, 255);
        for (int i = 0; i < 256; i++) cb[i] = (float)(i - 128);
        for (auto& v : x) v = (float)uni(-8, 8);
        oil::kernel::oil8_gemm(idx.data(), cb.data(), x.data(), y0.data(), M, 1, K);
        oil::mi355x::register_weights(idx.data(), idx.size());
        const bool held = oil::mi355x::registered_bytes() == idx.size();
        // a row slice inside the registered range reads the resident copy
        oil::kernel::oil8_gemm(idx.data(), cb.data(), x.data(), y1.data(), M, 1, K);
        std::vector<float> yr(M - 8);
        oil::kernel::oil8_gemm(idx.data() + 8 * K, cb.data(), x.data(), yr.data(), M - 8, 1, K);
        // the resident copy is a snapshot until registered again
        for (auto& v : idx) v = (uint8_t)(255 - v);
        oil::kernel::oil8_gemm(idx.data(), cb.data(), x.data(), y2.data(), M, 1, K);
        const bool dropped = oil::mi355x::unregister_weights(idx.data());
        oil::kernel::oil8_gemm(idx.data(), cb.data(), x.data(), y3.data(), M, 1, K);
        bool ok = held && dropped && same(y0, y1) && same(y0, y2) && !same(y0, y3) &&
                  oil::mi355x::registered_bytes() == 0;
        ok = ok && std::memcmp(yr.data(), y0.data() + 8, yr.size() * 4) == 0;
        CHECK("register_weights snapshot / slice / unregister", ok);
    }

    // ---- errors surface as oil::Error -------------------------------------
    {
        bool threw = false;
        try {
            oil::kernel::oil8_gemm(nullptr, nullptr, nullptr, nullptr, 0, 1, 1);
        } catch (const oil::Error&) {
            threw = true;
        }
        CHECK("invalid sizes throw oil::Error", threw);
    }

    std::printf("%s: %d failure(s)\n", g_fail ? "FAILED" : "OK", g_fail);
    return g_fail ? 1 : 0;
}
