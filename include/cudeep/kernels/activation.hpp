// Activation launchers (include/cudeep/kernels/activation.cuh:8-31).  Every
// ActivationType of the reference (ReLU, GELU in its tanh form, SiLU,
// Sigmoid, Tanh, LeakyReLU) runs on the GPU, in float and double.
#pragma once

#include "../common.hpp"

namespace cudeep {
namespace kernels {

enum class ActivationType { ReLU, Sigmoid, Tanh, GELU, SiLU, LeakyReLU };

template <typename T>
void launch_activation_forward_kernel(const T* input, T* output, int64_t n,
                                      ActivationType act_type, float alpha = 0.01f,
                                      hipStream_t stream = nullptr);

template <typename T>
void launch_activation_backward_kernel(const T* grad_output, const T* input, T* grad_input,
                                       int64_t n, ActivationType act_type, float alpha = 0.01f,
                                       hipStream_t stream = nullptr);

}  // namespace kernels
}  // namespace cudeep
