// Common types of the C++ host API (mirrors include/cudeep/common.cuh:10-53
// of the reference: DType, Layout, ceil_div).  Wavefronts are 64 lanes on
// CDNA4; nothing here assumes 32-wide warps.
#pragma once

#include <cstddef>
#include <cstdint>
#include <hip/hip_runtime_api.h>

namespace cudeep {

enum class DType { Float16, Float32, Float64 };
enum class Layout { NCHW, NHWC };

constexpr int WAVE_SIZE = 64;

inline size_t dtype_size(DType d) {
    switch (d) {
        case DType::Float16: return 2;
        case DType::Float32: return 4;
        case DType::Float64: return 8;
    }
    return 4;
}

inline constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace cudeep
