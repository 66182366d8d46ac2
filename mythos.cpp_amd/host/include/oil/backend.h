// oil/backend.h — the compute-backend dispatch of MYTHOS.cpp
// (include/oil/backend.h:9-80 there), with an MI355X backend behind it.
//
// BackendType, backend_name, BackendConfig and the ComputeBackend vtable keep
// the reference's names, values and signatures, so code written against the
// reference's dispatch compiles and means the same.  ComputeBackend::create
// returns the HIP backend for BackendType::GPU_CUDA (the reference's GPU
// slot; its enum has no ROCm value) and nullptr for every type this build
// does not provide (the CPU, DirectX, Vulkan, RAM-swap and distributed
// backends).  Tensors are host tensors, as in the reference: every operator
// stages its operands on the GPU, runs there and copies the result back
// before it returns.  copy, fill and zero act on the host tensors directly
// (the reference's backends do the same).  Errors raise oil::Error.
#pragma once

#include <cstdint>
#include <string>

#include "oil/tensor.h"
#include "oil/types.h"

namespace oil {
namespace backend {

enum class BackendType {
    CPU_SCALAR = 0,
    CPU_AVX2,
    CPU_AVX512,
    CPU_NEON,
    GPU_CUDA,
    GPU_DIRECTX,
    GPU_VULKAN,
    IGPU_SHARED,
    RAM_SWAP,
    DISTRIBUTED
};

inline const char* backend_name(BackendType t) {
    switch (t) {
        case BackendType::CPU_SCALAR: return "CPU_SCALAR";
        case BackendType::CPU_AVX2: return "CPU_AVX2";
        case BackendType::CPU_AVX512: return "CPU_AVX512";
        case BackendType::CPU_NEON: return "CPU_NEON";
        case BackendType::GPU_CUDA: return "GPU_CUDA";
        case BackendType::GPU_DIRECTX: return "GPU_DIRECTX";
        case BackendType::GPU_VULKAN: return "GPU_VULKAN";
        case BackendType::IGPU_SHARED: return "IGPU_SHARED";
        case BackendType::RAM_SWAP: return "RAM_SWAP";
        case BackendType::DISTRIBUTED: return "DISTRIBUTED";
    }
    return "UNKNOWN";
}

struct BackendConfig {
    BackendType type = BackendType::CPU_SCALAR;
    int64_t device_id = 0;
    int64_t num_devices = 1;
    int64_t threads = 0;
    bool enable_fp16 = false;
    bool enable_mixed_precision = false;
    float memory_fraction = 0.9f;
    std::string device_name;
};

class ComputeBackend {
public:
    virtual ~ComputeBackend() = default;
    virtual BackendType type() const = 0;
    virtual const char* name() const = 0;

    virtual void gemm(float alpha, const Tensor& A, const Tensor& B, float beta, Tensor& C) = 0;
    virtual void gemv(float alpha, const Tensor& A, const Tensor& x, float beta, Tensor& y) = 0;

    virtual void softmax(const Tensor& x, Tensor& y, int axis) = 0;
    virtual void layer_norm(const Tensor& x, const Tensor& gamma, const Tensor& beta, float eps, Tensor& y) = 0;
    virtual void rms_norm(const Tensor& x, const Tensor& gamma, float eps, Tensor& y) = 0;

    virtual void relu(const Tensor& x, Tensor& y) = 0;
    virtual void gelu(const Tensor& x, Tensor& y) = 0;
    virtual void silu(const Tensor& x, Tensor& y) = 0;

    virtual void add(const Tensor& a, const Tensor& b, Tensor& c) = 0;
    virtual void mul(const Tensor& a, const Tensor& b, Tensor& c) = 0;
    virtual void scale(float s, const Tensor& x, Tensor& y) = 0;

    virtual void copy(const Tensor& src, Tensor& dst) = 0;
    virtual void fill(Tensor& t, float val) = 0;
    virtual void zero(Tensor& t) = 0;

    virtual bool is_available() const = 0;
    virtual int64_t memory_free() const = 0;
    virtual int64_t memory_total() const = 0;
    virtual void synchronize() = 0;

    // The caller owns the result (delete it), as with the reference's.
    static ComputeBackend* create(const BackendConfig& cfg);
};

// A HIP device is present (the reference's probe for its GPU slot).
bool is_cuda_available();
// Free device memory of device_id in bytes (0 when there is none).
int64_t gpu_memory_free(int64_t device_id);

}  // namespace backend
}  // namespace oil
