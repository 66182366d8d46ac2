// oil/mi355x.h — device residency for the weight operands of the oil::kernel
// drop-ins.  No counterpart in MYTHOS.cpp, whose kernels read host memory in
// place; without registration every call copies its operands over PCIe.
#pragma once

#include <cstddef>
#include <cstdint>

namespace oil {
namespace backend {
class ComputeBackend;
}
namespace mi355x {

// The HIP ComputeBackend (oil/backend.h) on HIP device device_id; the caller
// owns it.  This is what ComputeBackend::create(GPU_CUDA) returns; the
// reference's factory calls it from its GPU_CUDA case when built with
// OIL_HAS_MI355X.
backend::ComputeBackend* make_hip_backend(int64_t device_id);

// Uploads [host, host + bytes) to device memory once.  Afterwards every
// oil::kernel call whose weight operand (indices, packed weights, codebooks,
// dense A/B) lies inside the range reads the resident copy.  A new range
// replaces the registered ranges it overlaps.  The copy is a snapshot: after
// changing the host bytes, register the range again.  Thread-safe; a call in
// flight keeps the copy it uses alive.  Throws oil::Error on failure.
void register_weights(const void* host, size_t bytes);

// Drops the range registered at exactly `host`; false if there is none.
bool unregister_weights(const void* host);

// Device bytes held by registered ranges.
size_t registered_bytes();

}  // namespace mi355x
}  // namespace oil
