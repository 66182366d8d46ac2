// oil/types.h — the subset of the reference's core types that the quantized
// operator signatures use (include/oil/types.h:17-149 in MYTHOS.cpp): Format,
// DType and its byte sizes, Shape, Error and OIL_CHECK.  Enum values and
// dtype sizes are kept identical so code written against the reference
// compiles and means the same thing.
#pragma once

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <stdexcept>
#include <string>

namespace oil {

enum class Format : uint8_t { BINARY = 0, TERNARY = 1, OIL4 = 2, OIL8 = 3, FP16 = 4, FP32 = 5 };

// U4 / I2 / I1 are still counted as one byte per element, as in the reference.
enum class DType : uint8_t { I64, U8, U4, I2, I1, F16, F32 };

inline size_t dtype_size(DType dt) {
    switch (dt) {
        case DType::I64: return 8;
        case DType::U8: case DType::U4: case DType::I2: case DType::I1: return 1;
        case DType::F16: return 2;
        case DType::F32: return 4;
    }
    return 0;
}

struct Shape {
    int64_t dims[8];
    int rank;
    Shape() : rank(0) {}
    explicit Shape(int64_t d0) : rank(1) { dims[0] = d0; }
    Shape(int64_t d0, int64_t d1) : rank(2) { dims[0] = d0; dims[1] = d1; }
    Shape(int64_t d0, int64_t d1, int64_t d2) : rank(3) { dims[0] = d0; dims[1] = d1; dims[2] = d2; }
    Shape(std::initializer_list<int64_t> l) : rank((int)l.size()) {
        if (rank > 8) throw std::runtime_error("Shape: rank exceeds maximum of 8");
        int i = 0;
        for (auto x : l) dims[i++] = x;
    }
    int64_t numel() const {
        int64_t n = 1;
        for (int i = 0; i < rank; i++) n *= dims[i];
        return n;
    }
};

class Error : public std::runtime_error {
public:
    explicit Error(const std::string& msg) : std::runtime_error(msg) {}
};

#define OIL_CHECK(cond, msg) \
    do {                     \
        if (!(cond)) throw oil::Error(msg); \
    } while (0)

}  // namespace oil
