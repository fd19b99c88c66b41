// Column-sum launcher (include/cudeep/kernels/unary.cuh:32-35): the bias
// gradient of nn.Linear.
#pragma once

#include "../common.hpp"

namespace cudeep {
namespace kernels {

template <typename T>
void launch_sum_reduce_rows_kernel(const T* input, T* output, int64_t rows, int64_t cols,
                                   hipStream_t stream = nullptr);

}  // namespace kernels
}  // namespace cudeep
