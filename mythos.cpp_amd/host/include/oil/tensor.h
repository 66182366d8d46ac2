// oil/tensor.h — minimal host Tensor for the operator signatures that take
// tensors (i2s_gemm, tl1_gemm, tl2_gemm, i2s_gemm_avx2, the ComputeBackend
// vtable).  Matches the reference's observable contract
// (include/oil/tensor.h:15-94, src/tensor.cpp:74-82,233-246): Tensor(Shape,
// DType) owns numel*dtype_size bytes, zero-filled and 64-byte aligned;
// data()/data<T>()/numel()/shape()/dtype(); fill (every element as float),
// zero_ (every byte), copy_from (equal numel, size_bytes copied).
#pragma once

#include <cstdlib>
#include <cstring>
#include <memory>

#include "oil/types.h"

namespace oil {

class Tensor {
public:
    Tensor() = default;
    explicit Tensor(Shape shape, DType dtype = DType::F32) : shape_(shape), dtype_(dtype) {
        const size_t bytes = (size_t)shape.numel() * dtype_size(dtype);
        const size_t alloc = ((bytes + 63) / 64) * 64;
        void* p = alloc ? std::aligned_alloc(64, alloc) : nullptr;
        if (alloc && !p) throw Error("Tensor: out of host memory");
        if (p) std::memset(p, 0, alloc);
        buf_ = std::shared_ptr<void>(p, [](void* q) { std::free(q); });
    }
    const Shape& shape() const { return shape_; }
    int64_t dim(int i) const { return shape_.dims[i]; }
    int rank() const { return shape_.rank; }
    int64_t numel() const { return shape_.numel(); }
    DType dtype() const { return dtype_; }
    size_t size_bytes() const { return (size_t)numel() * dtype_size(dtype_); }
    void* data() { return buf_.get(); }
    const void* data() const { return buf_.get(); }
    template <typename T> T* data() { return static_cast<T*>(data()); }
    template <typename T> const T* data() const { return static_cast<const T*>(data()); }

    void fill(float val) {
        float* d = data<float>();
        for (int64_t i = 0; i < numel(); i++) d[i] = val;
    }
    void zero_() {
        if (data()) std::memset(data(), 0, size_bytes());
    }
    void copy_from(const Tensor& src) {
        OIL_CHECK(numel() == src.numel(), "copy_from: size mismatch");
        if (size_bytes()) std::memcpy(data(), src.data(), size_bytes());
    }

private:
    Shape shape_;
    DType dtype_ = DType::F32;
    std::shared_ptr<void> buf_;
};

}  // namespace oil
