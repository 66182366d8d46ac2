// oil/int8_quant.h — drop-in for MYTHOS.cpp's include/oil/int8_quant.h
// (lines 7-28), computed on the GPU by mth_quantize_per_token.
// Host pointers, synchronous; bit-exact with src/int8_quant.cpp:8-41.
#pragma once

#include <cstdint>
#include <vector>

#include "oil/tensor.h"

namespace oil {

struct Int8QuantParams {
    float scale;      // multiplier: int8 = round(fp32 * scale)
    float inv_scale;  // 1/scale for dequant (max_abs / 127)
};

Int8QuantParams quantize_per_tensor(const float* src, int8_t* dst, int64_t n);
std::vector<Int8QuantParams> quantize_per_token(const float* src, int8_t* dst, int64_t rows, int64_t cols);
void dequantize_per_tensor(const int8_t* src, float* dst, int64_t n, float inv_scale);
Int8QuantParams quantize_tensor(const Tensor& src, Tensor& dst);

}  // namespace oil
