// stream_probe.hip — the measured streaming floor used as the second roofline
// denominator in bench.py (libmythos_probe.so; not part of the C ABI of the
// quantized path, and no counterpart in the reference).
//
// A pure read of `bytes` bytes: 16-byte non-temporal loads, grid-strided,
// UNROLL loads in flight per thread, XOR-folded so that the loads cannot be
// removed; one store in the whole launch, and only if the fold hits a value
// the caller's data never produces.  Its time for the same byte count as a
// GEMV's weights is what one launch of any kernel that reads those bytes once
// can reach on this device (launch cost, ramp-up and drain included).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int UNROLL>
__global__ __launch_bounds__(256) void stream_read_k(const u32x4* __restrict__ p, int64_t n16,
                                                      uint32_t* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    uint32_t acc = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride * UNROLL) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int64_t j = i + (int64_t)u * stride;
            v[u] = j < n16 ? __builtin_nontemporal_load(p + j) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) out[0] = acc;
}

extern "C" {

// Reads bytes / 16 16-byte words of p (16-byte aligned) on `grid`
// workgroups of 256 threads, unroll 1 or 4.  Returns 0, or -1 for bad
// arguments, -2 when the launch fails.
int mth_probe_stream_read(const void* p, int64_t bytes, int grid, int unroll, uint32_t* out, void* stream) {
    if (!p || !out || bytes < 16 || grid < 1 || grid > 65535 || ((uintptr_t)p & 15u) != 0) return -1;
    const hipStream_t s = (hipStream_t)stream;
    const int64_t n16 = bytes / 16;
    if (unroll == 4)
        stream_read_k<4><<<grid, 256, 0, s>>>((const u32x4*)p, n16, out);
    else if (unroll == 1)
        stream_read_k<1><<<grid, 256, 0, s>>>((const u32x4*)p, n16, out);
    else
        return -1;
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
