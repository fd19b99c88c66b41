// GEMM launchers of the C++ host API, same names and argument meaning as
// the reference's include/cudeep/kernels/matmul.cuh:8-44 (row-major, C
// overwritten, caller-owned device pointers), implemented over the C-ABI.
//
//  * launch_matmul_kernel<float>: the library's default float precision,
//    TF32 mode unless set_matmul_precision(FP32) -- the reference's default
//    float GEMM is its TF32 tensor-core path on SM >= 8
//    (src/kernels/matmul_kernel.cu:1785-1841).  <double> is the fp64 GEMM.
//  * launch_matmul_kernel_fp32<float>: always FP32 MFMA (the reference's
//    "SGEMM", matmul_kernel.cu:1851-1863).
//  * launch_matmul_kernel_fp16: fp16 A, B -> fp32 C (the reference's
//    hgemm_tc_kernel, matmul_kernel.cu:745-930, :1926-1943).
//  * launch_matmul_fused_act: GEMM + activation epilogue.
//  * launch_matmul_ex: transposes, leading dimensions, bias, epilogue.
// Errors throw std::runtime_error.
#pragma once

#include <hip/hip_fp16.h>

#include "../common.hpp"

namespace cudeep {
namespace kernels {

// FP32: true-FP32 MFMA.  TF32Mode: bf16x3 split MFMA (per-product relative
// error <= 2^-15).  TF32Mode4: bf16x4 (<= 2^-16; exact products for
// TF32-rounded operands).
enum class MatmulPrecision { FP32, TF32Mode, TF32Mode4 };

// Process-wide precision of launch_matmul_kernel<float> and everything
// built on it (Tensor::matmul, conv, Linear).  Default: TF32Mode.
void set_matmul_precision(MatmulPrecision p);
MatmulPrecision get_matmul_precision();

template <typename T>
void launch_matmul_kernel(const T* A, const T* B, T* C, int M, int N, int K,
                          hipStream_t stream = nullptr);

template <typename T>
void launch_matmul_kernel_fp32(const T* A, const T* B, T* C, int M, int N, int K,
                               hipStream_t stream = nullptr);

void launch_matmul_kernel_fp16(const __half* A, const __half* B, float* C, int M, int N, int K,
                               hipStream_t stream = nullptr);

// tile_size is accepted for interface compatibility and ignored (as in the
// reference, matmul_kernel.cu:1871-1875).
template <typename T>
void launch_matmul_tiled_kernel(const T* A, const T* B, T* C, int M, int N, int K,
                                int tile_size, hipStream_t stream = nullptr);

enum class GemmEpilogue { None, ReLU, GELU, SiLU, Sigmoid };

void launch_matmul_fused_act(const float* A, const float* B, float* C, int M, int N, int K,
                             GemmEpilogue epilogue, hipStream_t stream = nullptr);

// C = epi(op(A) op(B) + bias): bias_per_col (Linear) or per row; bias may
// be null.  Uses the process-wide precision unless `precision` >= 0.
void launch_matmul_ex(const float* A, const float* B, float* C, int64_t M, int64_t N,
                      int64_t K, bool transA, bool transB, int64_t lda, int64_t ldb,
                      int64_t ldc, const float* bias, bool bias_per_col,
                      GemmEpilogue epilogue, hipStream_t stream = nullptr, int precision = -1);

// Weight and bias gradient of a Linear layer in one launch:
// grad_w[out, in] = dz^T x  and  grad_b[out] = column sums of dz, for
// dz [batch, out] and x [batch, in] row-major (grad_b may be null: then
// just the product).  Replaces MatMulOp.backward's dW GEMM plus
// sum_reduce_rows (python/cuDeep/tensor.py:430-443, :617-631).
void launch_linear_weight_grad(const float* dz, const float* x, float* grad_w, float* grad_b,
                               int64_t batch, int64_t out_features, int64_t in_features,
                               hipStream_t stream = nullptr, int precision = -1);

// Input gradient of a Linear layer with the activation derivative of the
// layer that produced its input applied in the same launch:
// grad_x[batch, in] = act'(aux) (.) (dz W), for dz [batch, out], weight
// [out, in] and aux [batch, in] row-major -- the producer's saved
// pre-activation (GELU / SiLU / Sigmoid) or, for ReLU, its output.  With
// epilogue None (aux ignored, may be null) it is the plain dz W.  Replaces
// MatMulOp.backward's dA GEMM followed by activation_backward on the result
// (python/cuDeep/tensor.py:430-443, src/bindings/module.cpp:837-872).
void launch_linear_input_grad(const float* dz, const float* weight, const float* aux,
                              float* grad_x, int64_t batch, int64_t out_features,
                              int64_t in_features, GemmEpilogue act,
                              hipStream_t stream = nullptr, int precision = -1);

void launch_matmul_dgemm_ex(const double* A, const double* B, double* C, int64_t M,
                            int64_t N, int64_t K, bool transA, bool transB, int64_t lda,
                            int64_t ldb, int64_t ldc, hipStream_t stream = nullptr);

}  // namespace kernels
}  // namespace cudeep
