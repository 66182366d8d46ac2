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

}  // extern "C"
