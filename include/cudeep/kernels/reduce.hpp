// Full-sum launcher (include/cudeep/kernels/reduce.cuh:9): Tensor.sum() in
// autograd graphs.  Deterministic.
#pragma once

#include "../common.hpp"

namespace cudeep {
namespace kernels {

template <typename T>
void launch_sum_kernel(const T* input, T* output, int64_t n, hipStream_t stream = nullptr);

}  // namespace kernels
}  // namespace cudeep
