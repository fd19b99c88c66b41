// Elementwise launchers used by the host Tensor and nn.Linear (the subset of
// include/cudeep/kernels/elementwise.cuh:8-29 on this path).
#pragma once

#include "../common.hpp"

namespace cudeep {
namespace kernels {

template <typename T>
void launch_add_kernel(const T* a, const T* b, T* out, int64_t n, hipStream_t stream = nullptr);
template <typename T>
void launch_sub_kernel(const T* a, const T* b, T* out, int64_t n, hipStream_t stream = nullptr);
template <typename T>
void launch_mul_kernel(const T* a, const T* b, T* out, int64_t n, hipStream_t stream = nullptr);
template <typename T>
void launch_fill_kernel(T* data, T value, int64_t n, hipStream_t stream = nullptr);
template <typename T>
void launch_broadcast_add_row_kernel(const T* matrix, const T* row, T* output, int64_t rows,
                                     int64_t cols, hipStream_t stream = nullptr);

}  // namespace kernels
}  // namespace cudeep
