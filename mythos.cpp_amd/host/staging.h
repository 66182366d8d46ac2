// staging.h — internal to libmythos_host.so: the per-thread device arena
// that stages host operands, the resident-weight registry, and error
// helpers, shared by kernel.cpp (oil::kernel drop-ins) and backend.cpp (the
// HIP ComputeBackend).  The accessors are inline functions with static
// storage, so the library holds one registry and one arena per thread.
#pragma once

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "mythos_oil.h"
#include "oil/types.h"

namespace oil {
namespace detail {


inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}
inline void mth_check(int rc, const char* what) {
    if (rc != MTH_OK) throw Error(std::string(what) + ": " + mth_last_error());
}

// Resident weights: host range -> device copy.  Entries are shared_ptr so a
// call that is using a copy keeps it alive across a concurrent unregister.
struct Resident {
    void* dev = nullptr;
    size_t bytes = 0;
    ~Resident() {
        if (dev) (void)hipFree(dev);
    }
};

class Registry {
public:
    void add(const void* host, size_t bytes) {
        if (!host || !bytes) throw Error("register_weights: empty range");
        auto r = std::make_shared<Resident>();
        hip_check(hipMalloc(&r->dev, bytes), "register_weights: hipMalloc");
        r->bytes = bytes;
        hip_check(hipMemcpy(r->dev, host, bytes, hipMemcpyHostToDevice), "register_weights: hipMemcpy");
        std::lock_guard<std::mutex> g(mu_);
        const uintptr_t b = (uintptr_t)host;
        // a new range replaces every registered range it overlaps
        for (auto it = map_.begin(); it != map_.end();) {
            const uintptr_t ob = it->first, oe = ob + it->second->bytes;
            if (ob < b + bytes && b < oe) it = map_.erase(it);
            else ++it;
        }
        map_[b] = std::move(r);
    }
    bool remove(const void* host) {
        std::lock_guard<std::mutex> g(mu_);
        return map_.erase((uintptr_t)host) > 0;
    }
    // Device address of [host, host+n) if one registered range holds all of it.
    std::shared_ptr<Resident> find(const void* host, size_t n, const void** dev) const {
        std::lock_guard<std::mutex> g(mu_);
        const uintptr_t p = (uintptr_t)host;
        auto it = map_.upper_bound(p);
        if (it == map_.begin()) return nullptr;
        --it;
        if (p + n > it->first + it->second->bytes) return nullptr;
        *dev = (const char*)it->second->dev + (p - it->first);
        return it->second;
    }
    size_t total() const {
        std::lock_guard<std::mutex> g(mu_);
        size_t t = 0;
        for (auto& kv : map_) t += kv.second->bytes;
        return t;
    }

private:
    mutable std::mutex mu_;
    std::map<uintptr_t, std::shared_ptr<Resident>> map_;
};

inline Registry& registry() {
    static Registry r;
    return r;
}

// Per-thread device staging area.  carve() hands out 256-byte aligned slices
// of one allocation; begin() starts a new call.
class Arena {
public:
    ~Arena() {
        if (blas_) (void)rocblas_destroy_handle(blas_);
        if (base_) (void)hipFree(base_);
        if (stream_) (void)hipStreamDestroy(stream_);
    }
    void begin(size_t bytes_needed) {
        if (!stream_) hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
        if (bytes_needed > cap_) {
            if (base_) hip_check(hipFree(base_), "hipFree");
            base_ = nullptr;
            cap_ = 0;
            hip_check(hipMalloc(&base_, bytes_needed), "hipMalloc");
            cap_ = bytes_needed;
        }
        off_ = 0;
        held_.clear();
    }
    static size_t pad(size_t b) { return (b + 255) / 256 * 256; }
    void* carve(size_t bytes) {
        void* p = (char*)base_ + off_;
        off_ += pad(bytes);
        return p;
    }
    template <typename T> T* upload(const T* host, size_t n) {
        T* d = (T*)carve(n * sizeof(T));
        if (n) hip_check(hipMemcpyAsync(d, host, n * sizeof(T), hipMemcpyHostToDevice, stream_), "hipMemcpy H2D");
        return d;
    }
    // A weight operand: its resident copy when registered (held until the
    // next begin()), else staged like any input.  Size the arena with
    // P(bytes) for it either way.
    template <typename T> const T* weights(const T* host, size_t n) {
        const void* dev = nullptr;
        auto r = registry().find(host, n * sizeof(T), &dev);
        if (r) {
            held_.push_back(std::move(r));
            carve(n * sizeof(T));
            return (const T*)dev;
        }
        return upload(host, n);
    }
    template <typename T> void download(T* host, const T* dev, size_t n) {
        if (n) hip_check(hipMemcpyAsync(host, dev, n * sizeof(T), hipMemcpyDeviceToHost, stream_), "hipMemcpy D2H");
    }
    void sync() { hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize"); }
    mth_stream_t stream() const { return (mth_stream_t)stream_; }
    rocblas_handle blas() {
        if (!blas_) {
            if (rocblas_create_handle(&blas_) != rocblas_status_success) throw Error("rocblas_create_handle failed");
        }
        if (rocblas_set_stream(blas_, stream_) != rocblas_status_success) throw Error("rocblas_set_stream failed");
        return blas_;
    }

private:
    void* base_ = nullptr;
    size_t cap_ = 0, off_ = 0;
    hipStream_t stream_ = nullptr;
    rocblas_handle blas_ = nullptr;
    std::vector<std::shared_ptr<Resident>> held_;
};

inline Arena& arena() {
    thread_local Arena a;
    return a;
}

inline size_t P(size_t b) { return Arena::pad(b); }

inline void check_dims(int M, int N, int K, const char* what) {
    if (M <= 0 || N <= 0 || K <= 0)
        throw Error(std::string(what) + ": M, N, K must be positive");
}


}  // namespace detail
}  // namespace oil
