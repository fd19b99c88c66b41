// Conv2d launchers of the C++ host API, same signatures as the reference's
// include/cudeep/kernels/conv.cuh:8-36 (NCHW input, OIHW weight, bias may be
// null), over the C-ABI.  Scratch is allocated stream-ordered, as the
// reference does.  float and double, as the reference instantiates them
// (src/kernels/conv_kernel.cu:793-798); double runs direct fp64 sums.
#pragma once

#include "../common.hpp"

namespace cudeep {
namespace kernels {

// Algorithm of launch_conv2d_forward_kernel<float> and
// launch_conv2d_backward_data_kernel<float>.  Auto follows the reference's
// forward routing (src/kernels/conv_kernel.cu:242-275): Winograd F(4x4,
// 3x3) for 3x3 stride-1 layers with at least 16 output pixels per image,
// the implicit GEMM for other layers whose column buffer would exceed
// 4 MiB, im2col + GEMM otherwise; backward data applies the Winograd rule
// to the transposed convolution it runs (3x3, stride 1, padding <= 2, at
// least 16 input pixels per image) in the TF32 modes, and keeps the GEMM
// route in FP32 (whose error bound is twice the reference's GEMM + col2im
// route).  Im2col never takes Winograd (large non-3x3 layers still take
// the implicit GEMM, which needs no column buffer); Implicit forces the
// implicit GEMM forward (backward data as Im2col).  Winograd on another
// geometry throws.
enum class ConvAlgorithm { Auto, Im2col, Winograd, Implicit };
void set_conv_algorithm(ConvAlgorithm a);
ConvAlgorithm get_conv_algorithm();

template <typename T>
void launch_conv2d_forward_kernel(const T* input, const T* weight, const T* bias, T* output,
                                  int batch, int in_channels, int out_channels, int in_h,
                                  int in_w, int kernel_h, int kernel_w, int stride_h,
                                  int stride_w, int pad_h, int pad_w,
                                  hipStream_t stream = nullptr);

template <typename T>
void launch_conv2d_backward_data_kernel(const T* grad_output, const T* weight, T* grad_input,
                                        int batch, int in_channels, int out_channels, int in_h,
                                        int in_w, int kernel_h, int kernel_w, int stride_h,
                                        int stride_w, int pad_h, int pad_w,
                                        hipStream_t stream = nullptr);

template <typename T>
void launch_conv2d_backward_weight_kernel(const T* grad_output, const T* input, T* grad_weight,
                                          int batch, int in_channels, int out_channels,
                                          int in_h, int in_w, int kernel_h, int kernel_w,
                                          int stride_h, int stride_w, int pad_h, int pad_w,
                                          hipStream_t stream = nullptr);

// grad_bias[c] = sum of grad_output[:, c, :, :] (on the GPU).
void launch_conv2d_backward_bias_kernel(const float* grad_output, float* grad_bias, int batch,
                                        int out_channels, int spatial,
                                        hipStream_t stream = nullptr);
void launch_conv2d_backward_bias_kernel(const double* grad_output, double* grad_bias, int batch,
                                        int out_channels, int spatial,
                                        hipStream_t stream = nullptr);

}  // namespace kernels
}  // namespace cudeep
