// synth.cpp — seeded synthetic inputs for the benchmark configurations
// (libmythos_synth.so, host only, used by synth.py).
//
// The stream is MYTHOS.cpp's RNG: xoroshiro128+ seeded by two splitmix64
// draws (src/random.cpp:7-30), one stream per configuration with seed
// 0x5EED0000 + config.  From it:
//   * indices: the top `bits` bits of successive next_u64() (8 for OIL8
//     indices, 4 for OIL4 nibbles);
//   * ternary codes: uniform_int(lo, hi) by rejection (src/random.cpp:45-51);
//   * normals: a double-precision Box–Muller over next_u64() >> 11 (both
//     values of each pair are used), rounded to float.
// The caller owns the 2-word state and passes it to every call, so arrays
// drawn one after another continue a single stream.
#include <cmath>
#include <cstdint>
#include <cstring>

namespace {

inline uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

inline uint64_t next_u64(uint64_t* st) {
    const uint64_t s0 = st[0];
    uint64_t s1 = st[1];
    const uint64_t r = s0 + s1;
    s1 ^= s0;
    st[0] = rotl(s0, 24) ^ s1 ^ (s1 << 16);
    st[1] = rotl(s1, 37);
    return r;
}

// FP32 -> FP16 bits, rounding toward zero (the reference's float_to_half,
// src/codebook.cpp:16-34): exponent rebias, mantissa truncated; values past
// the FP16 range become infinity, NaN stays NaN; subnormal results keep the
// shifted mantissa, smaller magnitudes flush to a signed zero.
inline uint16_t f32_to_f16_trunc(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int e = (int)((u >> 23) & 0xFF) - 127 + 15;
    const uint32_t mant = u & 0x007FFFFFu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        return (uint16_t)(sign | (((mant | 0x00800000u) >> (1 - e)) >> 13));
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u | (mant ? 0x0200u : 0u));
    return (uint16_t)(sign | ((uint32_t)e << 10) | (mant >> 13));
}

}  // namespace

extern "C" {

void mth_synth_seed(uint64_t seed, uint64_t* st) {
    uint64_t t = seed;
    st[0] = splitmix64(t);
    st[1] = splitmix64(t);
}

void mth_synth_u64(uint64_t* st, uint64_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = next_u64(st);
}

void mth_synth_bits(uint64_t* st, uint8_t* out, int64_t n, int bits) {
    const int sh = 64 - bits;
    for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)(next_u64(st) >> sh);
}

void mth_synth_uniform_int(uint64_t* st, int8_t* out, int64_t n, int lo, int hi) {
    const uint64_t range = (uint64_t)(hi - lo + 1);
    const uint64_t limit = UINT64_MAX - (UINT64_MAX % range);
    for (int64_t i = 0; i < n; ++i) {
        uint64_t v;
        do {
            v = next_u64(st);
        } while (v >= limit);
        out[i] = (int8_t)(lo + (int)(v % range));
    }
}

// OIL4 nibbles packed two per byte: element 2i (low nibble) then 2i+1, each
// the top 4 bits of one next_u64() (the same draws as mth_synth_bits(.., 4)
// followed by packing).
void mth_synth_nibbles(uint64_t* st, uint8_t* out, int64_t nbytes) {
    for (int64_t i = 0; i < nbytes; ++i) {
        const uint8_t lo = (uint8_t)(next_u64(st) >> 60);
        const uint8_t hi = (uint8_t)(next_u64(st) >> 60);
        out[i] = (uint8_t)(lo | (hi << 4));
    }
}

// Ternary codes t+1 = uniform_int(0, 2) packed four per byte, element 4i+j
// in bits 2j (the same draws as mth_synth_uniform_int(.., 0, 2) + packing).
void mth_synth_ternary(uint64_t* st, uint8_t* out, int64_t nbytes) {
    const uint64_t limit = UINT64_MAX - (UINT64_MAX % 3);
    for (int64_t i = 0; i < nbytes; ++i) {
        uint32_t b = 0;
        for (int j = 0; j < 4; ++j) {
            uint64_t v;
            do {
                v = next_u64(st);
            } while (v >= limit);
            b |= (uint32_t)(v % 3) << (2 * j);
        }
        out[i] = (uint8_t)b;
    }
}

void mth_synth_uniform_i32(uint64_t* st, int32_t* out, int64_t n, int lo, int hi) {
    const uint64_t range = (uint64_t)((int64_t)hi - lo + 1);
    const uint64_t limit = UINT64_MAX - (UINT64_MAX % range);
    for (int64_t i = 0; i < n; ++i) {
        uint64_t v;
        do {
            v = next_u64(st);
        } while (v >= limit);
        out[i] = (int32_t)(lo + (int64_t)(v % range));
    }
}

void mth_synth_normal(uint64_t* st, float* out, int64_t n, double mean, double stddev) {
    const double two_pi = 6.283185307179586476925286766559;
    const double inv53 = 1.0 / 9007199254740992.0;  // 2^-53
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = (double)(next_u64(st) >> 11) * inv53;
        const double u2 = (double)(next_u64(st) >> 11) * inv53;
        if (u1 <= 0.0) u1 = inv53;
        const double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = (float)(mean + stddev * r * std::cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(mean + stddev * r * std::sin(two_pi * u2));
    }
}

// normals as mth_synth_normal draws them, stored as truncated FP16 bits
void mth_synth_normal_f16(uint64_t* st, uint16_t* out, int64_t n, double mean, double stddev) {
    float buf[256];
    for (int64_t i = 0; i < n; i += 256) {
        const int64_t m = n - i < 256 ? n - i : 256;
        mth_synth_normal(st, buf, m, mean, stddev);
        for (int64_t j = 0; j < m; ++j) out[i + j] = f32_to_f16_trunc(buf[j]);
    }
}

}  // extern "C"
