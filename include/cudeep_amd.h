/*
 * cudeep_amd.h -- C-ABI of the MI355X (gfx950) dense-contraction library.
 *
 * This is the drop-in boundary for cuDeep's dense-contraction hot path:
 * the FP32 SGEMM, the "TF32" GEMM (here an explicit bf16x3 split-precision
 * MFMA GEMM), the fused-epilogue GEMM, the fp64 GEMM, im2col and the
 * im2col-Conv2d forward, plus the small helpers nn.Linear needs (bias
 * broadcast, column sums, ReLU/GELU forward and backward).
 *
 * Each entry point names the reference interface it replaces
 * (/root/reference = KevinWeiss1995/cuDeep, file:line).
 *
 * Conventions
 *  - All pointers are device pointers (hipMalloc'd or equivalent) unless
 *    stated; sizes are 64-bit element counts.  Matrices are row-major and
 *    dense unless a leading dimension is given.
 *  - Every entry point returns CDX_OK (0) or a CDX_ERR_* code and never
 *    throws; cdx_last_error() gives a message for the calling thread.
 *  - Work is enqueued on `stream` (NULL = the null stream) and is
 *    asynchronous: execution faults surface at the caller's next sync.
 *  - The library keeps no global device state: concurrent calls on different
 *    streams are safe.  Routines that need scratch take a `workspace`
 *    pointer; passing NULL makes the library allocate and free it
 *    stream-ordered, as the reference does -- from a library-owned memory
 *    pool per device that keeps freed blocks for reuse
 *    (hipMallocFromPoolAsync / hipFreeAsync).
 */
#ifndef CUDEEP_AMD_H
#define CUDEEP_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define CDX_OK                 0
#define CDX_ERR_INVALID_ARG    1   /* null pointer, bad dims, bad enum      */
#define CDX_ERR_UNSUPPORTED    2   /* valid request the library cannot do   */
#define CDX_ERR_HIP            3   /* a HIP runtime call failed             */
#define CDX_ERR_WORKSPACE      4   /* workspace given but too small         */

/* ---- enums ------------------------------------------------------------- */
#define CDX_OP_N 0                 /* use the operand as stored             */
#define CDX_OP_T 1                 /* use its transpose                     */

/* Epilogues / activations; values follow cudeep::kernels::GemmEpilogue
 * (include/cudeep/kernels/matmul.cuh:32-38).  GELU is the tanh form,
 * SiLU = x * sigmoid(x), Sigmoid = 1 / (1 + exp(-x))
 * (src/kernels/matmul_kernel.cu:1538-1550). */
#define CDX_EPI_NONE    0
#define CDX_EPI_RELU    1
#define CDX_EPI_GELU    2
#define CDX_EPI_SILU    3
#define CDX_EPI_SIGMOID 4
/* elementwise activations only (cdx_activation_*), not GEMM epilogues */
#define CDX_ACT_TANH       5
#define CDX_ACT_LEAKY_RELU 6
/* Activation-backward epilogues (cdx_gemm_fused only): C = P * act'(aux) with
 * P = op(A) * op(B) and aux the forward pre-activation (for ReLU its output
 * works too), elementwise with the reference's activation_backward formulas
 * (src/kernels/activation_kernel.cu:256-319): ReLU aux > 0 ? P : 0. */
#define CDX_EPI_BWD_RELU    8
#define CDX_EPI_BWD_GELU    9
#define CDX_EPI_BWD_SILU    10
#define CDX_EPI_BWD_SIGMOID 11

#define CDX_BIAS_NONE 0
#define CDX_BIAS_ROW  1            /* C[m][n] += bias[m]  (conv: per channel) */
#define CDX_BIAS_COL  2            /* C[m][n] += bias[n]  (Linear)            */

#define CDX_PREC_FP32      0       /* true-FP32 MFMA (v_mfma_f32_16x16x4_f32) */
#define CDX_PREC_TF32MODE  1       /* bf16x3 split MFMA, |rel err| <= 2^-15 per product */
#define CDX_PREC_TF32MODE4 2       /* bf16x4 split MFMA, |rel err| <= 2^-16 per product;
                                      exact products for operands of <= 16 significant
                                      bits (TF32-rounded inputs) */

#define CDX_DTYPE_F32  0
#define CDX_DTYPE_F64  1
#define CDX_DTYPE_F16  2           /* IEEE binary16 (GEMM operands only) */
#define CDX_DTYPE_BF16 3           /* bfloat16 (GEMM operands only)      */

#define CDX_BINARY_ADD 0
#define CDX_BINARY_SUB 1
#define CDX_BINARY_MUL 2

/* ---- library --------------------------------------------------------- */
const char* cdx_last_error(void);
const char* cdx_version(void);

/* ---- GEMM ------------------------------------------------------------ */

/* C[M,N] = A[M,K] * B[K,N], FP32 MFMA, C overwritten.
 * Replaces cudeep::kernels::launch_matmul_kernel_fp32<float>
 * (include/cudeep/kernels/matmul.cuh:14-18, src/kernels/matmul_kernel.cu:1851-1863). */
int cdx_sgemm_f32(const float* A, const float* B, float* C,
                  int64_t M, int64_t N, int64_t K, hipStream_t stream);

/* Same product in TF32 mode (bf16x3 split-precision MFMA).
 * Replaces cudeep::kernels::launch_matmul_kernel<float>, whose SM>=8 path is
 * the TF32 tensor-core GEMM (matmul.cuh:8-12, matmul_kernel.cu:1785-1841). */
int cdx_gemm_tf32mode(const float* A, const float* B, float* C,
                      int64_t M, int64_t N, int64_t K, hipStream_t stream);

/* General form: C = epi(op(A) * op(B) + bias), with leading dimensions,
 * transposes, a bias vector (per row or per column) and a ReLU/GELU
 * epilogue.  op(A) is M x K, op(B) is K x N.  Backs the reference's
 * launch_matmul_fused_act (matmul.cuh:40-44) and lets nn.Linear run
 * x*W^T + b with ReLU in one launch instead of the strided copy,
 * broadcast_add and activation kernels (python/cuDeep/nn.py:110-115,
 * src/tensor.cu:26-68, src/kernels/elementwise_kernel.cu:186-204). */
int cdx_gemm_ex(int precision, int opA, int opB,
                int64_t M, int64_t N, int64_t K,
                const float* A, int64_t lda,
                const float* B, int64_t ldb,
                float* C, int64_t ldc,
                const float* bias, int bias_mode, int epilogue,
                hipStream_t stream);

/* Bytes of scratch cdx_gemm_ex_ws needs for this problem: the split-K
 * partials of long-K problems with few output tiles (e.g. weight gradients),
 * 0 when the launch does not split.  The same (precision, transposes, sizes)
 * always give the same answer. */
size_t cdx_gemm_workspace_size(int precision, int opA, int opB,
                               int64_t M, int64_t N, int64_t K);

/* cdx_gemm_ex with caller scratch: with a workspace of at least
 * cdx_gemm_workspace_size bytes the call allocates nothing (safe inside HIP
 * graph capture); NULL falls back to stream-ordered allocation.  The
 * reference's GEMM launchers allocate nothing because they never split K
 * (matmul_kernel.cu:1785-1841); this is the same contract for the split
 * launches.  Too small a workspace is CDX_ERR_WORKSPACE. */
int cdx_gemm_ex_ws(int precision, int opA, int opB,
                   int64_t M, int64_t N, int64_t K,
                   const float* A, int64_t lda,
                   const float* B, int64_t ldb,
                   float* C, int64_t ldc,
                   const float* bias, int bias_mode, int epilogue,
                   void* workspace, size_t workspace_bytes,
                   hipStream_t stream);

/* cdx_gemm_ex_ws with the two fusions a Linear layer's backward wants, both
 * computed by the same launch (the reference runs each as a kernel of its
 * own: activation_backward, module.cpp:837-872 / activation_kernel.cu:256-319,
 * and sum_reduce_rows, unary_kernel.cu:204-238, after the GEMMs of
 * MatMulOp.backward, python/cuDeep/tensor.py:430-443, :617-631):
 *  - epilogue CDX_EPI_BWD_*: C = act'(aux) (.) (op(A) * op(B)), aux [M, N]
 *    with leading dimension ldaux (no bias with these epilogues);
 *  - colsum (may be NULL): colsum[m] = sum over k of op(A)(m, k), the
 *    product's row sums of op(A) -- with op(A) = dZ^T (opA = T) the bias
 *    gradient of the layer whose weight gradient dZ^T X the call computes.
 *    Formed as an extra output column of the product against a column of
 *    ones (exact products, the GEMM's own accumulation), so it costs no
 *    extra pass over dZ; requires bias_mode NONE and epilogue NONE and runs
 *    the FP32 MFMA kernel in every precision mode (its products are exact).
 * Workspace: cdx_gemm_fused_workspace_size (split-K partials, which then
 * hold the extra column too); NULL allocates stream-ordered. */
size_t cdx_gemm_fused_workspace_size(int precision, int opA, int opB,
                                     int64_t M, int64_t N, int64_t K, int with_colsum);
int cdx_gemm_fused(int precision, int opA, int opB,
                   int64_t M, int64_t N, int64_t K,
                   const float* A, int64_t lda,
                   const float* B, int64_t ldb,
                   float* C, int64_t ldc,
                   const float* bias, int bias_mode, int epilogue,
                   const float* aux, int64_t ldaux, float* colsum,
                   void* workspace, size_t workspace_bytes,
                   hipStream_t stream);

/* C = act(A * B), TF32 mode, no bias.
 * Replaces cudeep::kernels::launch_matmul_fused_act
 * (matmul.cuh:40-44, matmul_kernel.cu:1884-1924); epilogue is CDX_EPI_*. */
int cdx_matmul_fused_act(const float* A, const float* B, float* C,
                         int64_t M, int64_t N, int64_t K, int epilogue,
                         hipStream_t stream);

/* C[M,N] = A * B with fp16 A [M,K] and B [K,N] (row-major), fp32
 * accumulation and fp32 C (v_mfma_f32_16x16x32_f16).
 * Replaces cudeep::kernels::launch_matmul_kernel_fp16
 * (matmul.cuh:27-30, matmul_kernel.cu:745-930, :1926-1943). */
int cdx_hgemm_f16(const void* A, const void* B, float* C,
                  int64_t M, int64_t N, int64_t K, hipStream_t stream);

/* General 16-bit-operand form: in_dtype is CDX_DTYPE_F16 or CDX_DTYPE_BF16;
 * transposes, leading dimensions, bias and epilogue as in cdx_gemm_ex; fp32
 * accumulation and C.  No counterpart in the reference beyond
 * launch_matmul_kernel_fp16 (the bf16 / transposed / fused forms). */
int cdx_gemm16_ex(int in_dtype, int opA, int opB,
                  int64_t M, int64_t N, int64_t K,
                  const void* A, int64_t lda,
                  const void* B, int64_t ldb,
                  float* C, int64_t ldc,
                  const float* bias, int bias_mode, int epilogue,
                  hipStream_t stream);

/* C[M,N] = op(A) * op(B) in fp64 (v_mfma_f64_16x16x4_f64).
 * Replaces cudeep::kernels::launch_matmul_kernel<double>
 * (matmul_kernel.cu:1843-1849, sgemm_double_kernel :691-743). */
int cdx_dgemm(int opA, int opB, int64_t M, int64_t N, int64_t K,
              const double* A, int64_t lda, const double* B, int64_t ldb,
              double* C, int64_t ldc, hipStream_t stream);

/* ---- convolution ------------------------------------------------------ */

/* col[K_col, B*OH*OW] from NCHW input, K_col = IC*KH*KW; bit-exact with
 * im2col_kernel (src/kernels/conv_kernel.cu:32-65). */
int cdx_im2col_f32(const float* input, float* col,
                   int64_t batch, int64_t in_channels, int64_t in_h, int64_t in_w,
                   int64_t kernel_h, int64_t kernel_w,
                   int64_t stride_h, int64_t stride_w,
                   int64_t pad_h, int64_t pad_w, hipStream_t stream);

/* Bytes of workspace cdx_conv2d_forward_f32 needs: the im2col buffer of one
 * round of images (the whole batch while its buffer stays within 128 MiB,
 * else rounds below that sized for whole waves of GEMM tiles), or 0 for
 * layers it sends to the implicit GEMM (see below). */
size_t cdx_conv2d_forward_workspace_size(
    int64_t batch, int64_t in_channels, int64_t in_h, int64_t in_w,
    int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
    int64_t pad_h, int64_t pad_w);

/* NCHW conv forward: im2col -> one GEMM weight[OC,K_col] * col -> NCHW
 * output with the bias added in the GEMM epilogue (no transpose pass), per
 * round of images (same sums as one pass over the batch).
 * Layers whose column buffer would exceed 4 MiB, other than 3x3 stride-1
 * layers with >= 16 output pixels per image, run the implicit GEMM of
 * cdx_conv2d_forward_implicit_f32 instead (no workspace), as the reference
 * dispatches them to its implicit kernel (conv_kernel.cu:263-275).
 * Replaces cudeep::kernels::launch_conv2d_forward_kernel<float>
 * (include/cudeep/kernels/conv.cuh:8-16, src/kernels/conv_kernel.cu:225-335).
 * bias may be NULL.  precision is CDX_PREC_*.  workspace may be NULL. */
int cdx_conv2d_forward_f32(const float* input, const float* weight,
                           const float* bias, float* output,
                           int64_t batch, int64_t in_channels, int64_t out_channels,
                           int64_t in_h, int64_t in_w,
                           int64_t kernel_h, int64_t kernel_w,
                           int64_t stride_h, int64_t stride_w,
                           int64_t pad_h, int64_t pad_w, int precision,
                           void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

/* NCHW conv forward as an implicit GEMM: each tile's input window is staged
 * in LDS once per chunk of input channels (the taps become LDS offsets), or,
 * where that window does not fit, gathered per k-tile; FP32 products, fp32
 * accumulation, bias added, no column buffer and no workspace.  Replaces
 * implicit_gemm_conv2d_kernel (src/kernels/conv_kernel.cu:172-215).
 * Geometries needing 64-bit pixel or in-image indices return
 * CDX_ERR_UNSUPPORTED.  bias may be NULL. */
int cdx_conv2d_forward_implicit_f32(const float* input, const float* weight,
                                    const float* bias, float* output,
                                    int64_t batch, int64_t in_channels,
                                    int64_t out_channels, int64_t in_h, int64_t in_w,
                                    int64_t kernel_h, int64_t kernel_w,
                                    int64_t stride_h, int64_t stride_w,
                                    int64_t pad_h, int64_t pad_w, hipStream_t stream);

/* Bytes of workspace cdx_conv2d_forward_winograd_f32 needs:
 * 36 * (OC*IC + IC*T + OC*T) floats, T = batch * ceil(OH/4) * ceil(OW/4). */
size_t cdx_conv2d_winograd_workspace_size(
    int64_t batch, int64_t in_channels, int64_t out_channels,
    int64_t in_h, int64_t in_w, int64_t pad_h, int64_t pad_w);

/* NCHW 3x3 stride-1 conv forward by Winograd F(4x4, 3x3): filter / input
 * transforms, one batched GEMM over the 36 transform points, output
 * transform + bias.  Replaces launch_conv2d_winograd_f43
 * (src/kernels/conv_kernel.cu:557-789), the reference's route for 3x3
 * stride-1 layers (:242-248).  Winograd adds transform rounding: expect
 * errors several times those of the im2col route.  precision is CDX_PREC_*
 * (the GEMM's); workspace may be NULL. */
int cdx_conv2d_forward_winograd_f32(const float* input, const float* weight,
                                    const float* bias, float* output,
                                    int64_t batch, int64_t in_channels,
                                    int64_t out_channels, int64_t in_h, int64_t in_w,
                                    int64_t pad_h, int64_t pad_w, int precision,
                                    void* workspace, size_t workspace_bytes,
                                    hipStream_t stream);

/* grad_input[B, IC, IH, IW] from grad_col[K_col, B*OH*OW]: sums, per input
 * element, every column entry it was copied to (kh then kw ascending, fp32);
 * bit-exact with col2im_kernel (src/kernels/conv_kernel.cu:344-380). */
int cdx_col2im_f32(const float* col, float* grad_input,
                   int64_t batch, int64_t in_channels, int64_t in_h, int64_t in_w,
                   int64_t kernel_h, int64_t kernel_w,
                   int64_t stride_h, int64_t stride_w,
                   int64_t pad_h, int64_t pad_w, hipStream_t stream);

/* Conv backward data.  Stride 1 (with pad_h <= kernel_h - 1, pad_w <=
 * kernel_w - 1): the forward convolution of grad_out with the filter
 * channel-swapped and spatially reversed, padded kernel - 1 - pad: an
 * implicit GEMM from per-tile input windows staged in LDS (no column buffer;
 * workspace = the flipped filter; FP32 products in every precision mode), or
 * where that window does not fit, im2col of grad_out + one long-K GEMM
 * written straight to NCHW.  Both sum k in two levels, keeping the rounding
 * chain no longer than the reference's OC-term dot products + KH*KW-term
 * col2im sums.  Other strides:
 * grad_col = weight^T * grad_out[OC, B*S] (one GEMM with a transposed
 * operand, no weight transpose pass), then col2im.  Both compute the
 * reference's sums (src/kernels/conv_kernel.cu:417-478) in another order.
 * Replaces cudeep::kernels::launch_conv2d_backward_data_kernel<float>
 * (include/cudeep/kernels/conv.cuh:18-26).
 * grad_input is overwritten.  workspace may be NULL. */
size_t cdx_conv2d_backward_data_workspace_size(
    int64_t batch, int64_t in_channels, int64_t out_channels, int64_t in_h, int64_t in_w,
    int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
    int64_t pad_h, int64_t pad_w);
int cdx_conv2d_backward_data_f32(const float* grad_output, const float* weight,
                                 float* grad_input,
                                 int64_t batch, int64_t in_channels, int64_t out_channels,
                                 int64_t in_h, int64_t in_w,
                                 int64_t kernel_h, int64_t kernel_w,
                                 int64_t stride_h, int64_t stride_w,
                                 int64_t pad_h, int64_t pad_w, int precision,
                                 void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);

/* Conv backward data of a 3x3 stride-1 layer by Winograd F(4x4, 3x3): the
 * forward Winograd convolution of grad_out with the channel-swapped,
 * spatially reversed filter, padded 2 - pad (pad_h, pad_w <= 2).  Same
 * arguments and meaning as cdx_conv2d_backward_data_f32 for kernel 3x3,
 * stride 1; errors are those of the Winograd forward.  The reference has no
 * Winograd backward (its backward data is conv_kernel.cu:417-478); this is
 * the faster route to the same gradient for the layers whose forward it
 * runs by Winograd (:242-248). */
size_t cdx_conv2d_backward_data_winograd_workspace_size(
    int64_t batch, int64_t in_channels, int64_t out_channels,
    int64_t in_h, int64_t in_w, int64_t pad_h, int64_t pad_w);
int cdx_conv2d_backward_data_winograd_f32(const float* grad_output, const float* weight,
                                          float* grad_input,
                                          int64_t batch, int64_t in_channels,
                                          int64_t out_channels, int64_t in_h, int64_t in_w,
                                          int64_t pad_h, int64_t pad_w, int precision,
                                          void* workspace, size_t workspace_bytes,
                                          hipStream_t stream);

/* Conv backward weight: grad_weight[OC, K_col] = grad_out[OC, B*S] * col^T,
 * as an implicit FP32-MFMA GEMM that reads both operands from the NCHW
 * grad_out and input: no col buffer, no reshape (3x3 stride-1 layers stage
 * whole input rows and form each tap as a shifted window; other geometries
 * gather per element).
 * All precisions take it (exact fp32 products meet the TF32 bounds too);
 * problems beyond its 32-bit index range fall back to im2col + a GEMM that
 * reads col transposed.  The long K = B*S is split across workgroups and
 * reduced in a fixed order.  The workspace size query returns exactly what
 * the route this problem takes uses.
 * Replaces cudeep::kernels::launch_conv2d_backward_weight_kernel<float>
 * (include/cudeep/kernels/conv.cuh:28-36, src/kernels/conv_kernel.cu:486-545).
 * grad_weight is overwritten.  workspace may be NULL. */
size_t cdx_conv2d_backward_weight_workspace_size(
    int64_t batch, int64_t in_channels, int64_t out_channels, int64_t in_h, int64_t in_w,
    int64_t kernel_h, int64_t kernel_w, int64_t stride_h, int64_t stride_w,
    int64_t pad_h, int64_t pad_w);
int cdx_conv2d_backward_weight_f32(const float* grad_output, const float* input,
                                   float* grad_weight,
                                   int64_t batch, int64_t in_channels, int64_t out_channels,
                                   int64_t in_h, int64_t in_w,
                                   int64_t kernel_h, int64_t kernel_w,
                                   int64_t stride_h, int64_t stride_w,
                                   int64_t pad_h, int64_t pad_w, int precision,
                                   void* workspace, size_t workspace_bytes,
                                   hipStream_t stream);

/* Bytes of device scratch the allocation-free entry point below owns on each
 * GPU it runs on (held until the process ends). */
#define CDX_NOALLOC_SCRATCH_BYTES (40u << 20)

/* cdx_conv2d_backward_weight_f32 without a workspace argument and without
 * any allocation: no hipMalloc / hipMallocAsync / hipFree, no allocating
 * library routine.  Its split partials live in a library-owned device array
 * of CDX_NOALLOC_SCRATCH_BYTES per GPU.  No counterpart in the reference: it
 * is for callers that cannot allocate (code under HIP graph capture, tight
 * training or serving loops, harnesses that forbid allocation).  Same
 * arguments, routes and results as cdx_conv2d_backward_weight_f32; a layer
 * whose scratch (cdx_conv2d_backward_weight_workspace_size) exceeds the
 * limit is refused with CDX_ERR_UNSUPPORTED before anything is launched
 * (C5's 64x64x3x3 layer at batch 32 needs 9 MiB, larger 3x3 stride-1
 * layers on the 64-channel row-window kernel 36 MiB).  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (different streams
 * or threads without ordering between them) race and must be serialised by
 * the caller. */
int cdx_conv2d_backward_weight_f32_noalloc(const float* grad_output, const float* input,
                                           float* grad_weight,
                                           int64_t batch, int64_t in_channels,
                                           int64_t out_channels, int64_t in_h, int64_t in_w,
                                           int64_t kernel_h, int64_t kernel_w,
                                           int64_t stride_h, int64_t stride_w,
                                           int64_t pad_h, int64_t pad_w, int precision,
                                           hipStream_t stream);

/* grad_bias[c] = sum over b, s of grad_output[b, c, s] (NCHW, S = OH*OW),
 * deterministic.  Replaces the host-side NumPy reduction of the reference's
 * Conv2dOp.backward (python/cuDeep/tensor.py:718-721). */
int cdx_conv2d_backward_bias_f32(const float* grad_output, float* grad_bias,
                                 int64_t batch, int64_t out_channels, int64_t spatial,
                                 hipStream_t stream);

/* float64 conv (no workspace).  Forward: each output the reference's fp64
 * explicit-route chain -- sum over k = (ic*KH + kh)*KW + kw ascending of
 * weight * input (zero padded), one FMA per term, then + bias[oc] (bias may
 * be NULL).  Backward data / weight: the adjoint sums, one fp64 chain per
 * output element.  Replace the double instantiations of
 * cudeep::kernels::launch_conv2d_forward_kernel / _backward_data_kernel /
 * _backward_weight_kernel (src/kernels/conv_kernel.cu:793-798; the explicit
 * route :225-335, :417-545 with the double GEMM matmul_kernel.cu:691-743). */
int cdx_conv2d_forward_f64(const double* input, const double* weight, const double* bias,
                           double* output, int64_t batch, int64_t in_channels,
                           int64_t out_channels, int64_t in_h, int64_t in_w,
                           int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                           int64_t stride_w, int64_t pad_h, int64_t pad_w, hipStream_t stream);
int cdx_conv2d_backward_data_f64(const double* grad_output, const double* weight,
                                 double* grad_input, int64_t batch, int64_t in_channels,
                                 int64_t out_channels, int64_t in_h, int64_t in_w,
                                 int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                                 int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                 hipStream_t stream);
int cdx_conv2d_backward_weight_f64(const double* grad_output, const double* input,
                                   double* grad_weight, int64_t batch, int64_t in_channels,
                                   int64_t out_channels, int64_t in_h, int64_t in_w,
                                   int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                                   int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                   hipStream_t stream);
/* grad_bias[c] = sum over b, s of grad_output[b, c, s] in fp64 (the
 * reference's float64 Conv2dOp.backward, python/cuDeep/tensor.py:718-721). */
int cdx_conv2d_backward_bias_f64(const double* grad_output, double* grad_bias,
                                 int64_t batch, int64_t out_channels, int64_t spatial,
                                 hipStream_t stream);

/* ---- Linear helpers ---------------------------------------------------- */

/* out[j] = sum_i in[i][j] over a row-major [rows, cols] matrix.
 * Replaces cudeep::kernels::launch_sum_reduce_rows_kernel<float>
 * (include/cudeep/kernels/unary.cuh:32-35, src/kernels/unary_kernel.cu:204-245).
 * Deterministic two-pass reduction; workspace may be NULL.  The size query
 * covers both the f32 and the f64 entry point. */
size_t cdx_sum_reduce_rows_workspace_size(int64_t rows, int64_t cols);
int cdx_sum_reduce_rows_f32(const float* input, float* output,
                            int64_t rows, int64_t cols,
                            void* workspace, size_t workspace_bytes,
                            hipStream_t stream);

/* out[i][j] = m[i][j] + row[j].  Replaces
 * cudeep::kernels::launch_broadcast_add_row_kernel<float>
 * (include/cudeep/kernels/elementwise.cuh:26-29, elementwise_kernel.cu:186-204). */
int cdx_broadcast_add_row_f32(const float* matrix, const float* row, float* out,
                              int64_t rows, int64_t cols, hipStream_t stream);
/* fp64 variants of the Linear helpers (float64 Linear, the reference's
 * double instantiations of the same launchers). */
int cdx_broadcast_add_row_f64(const double* matrix, const double* row, double* out,
                              int64_t rows, int64_t cols, hipStream_t stream);
int cdx_sum_reduce_rows_f64(const double* input, double* output,
                            int64_t rows, int64_t cols,
                            void* workspace, size_t workspace_bytes,
                            hipStream_t stream);

/* Activation forward and backward, act = CDX_EPI_RELU, _GELU, _SILU,
 * _SIGMOID, CDX_ACT_TANH or CDX_ACT_LEAKY_RELU (alpha: its negative slope,
 * ignored by the others); the backward takes the pre-activation input.
 * Replace launch_activation_forward_kernel / launch_activation_backward_kernel
 * (include/cudeep/kernels/activation.cuh:17-31,
 * src/kernels/activation_kernel.cu:19-66, :206-330). */
int cdx_activation_forward_f32(const float* input, float* output, int64_t n,
                               int act, float alpha, hipStream_t stream);
int cdx_activation_backward_f32(const float* grad_output, const float* input,
                                float* grad_input, int64_t n, int act, float alpha,
                                hipStream_t stream);
int cdx_activation_forward_f64(const double* input, double* output, int64_t n,
                               int act, float alpha, hipStream_t stream);
int cdx_activation_backward_f64(const double* grad_output, const double* input,
                                double* grad_input, int64_t n, int act, float alpha,
                                hipStream_t stream);

/* ---- tensor runtime ----------------------------------------------------- */

/* dst (contiguous) <- src viewed with `shape` / `src_strides` (elements,
 * ndim <= 8; shape and strides are host arrays).  dtype is CDX_DTYPE_*.
 * Replaces launch_strided_copy / strided_copy_kernel (src/tensor.cu:26-68)
 * without its device allocation, H2D copies and stream synchronize. */
int cdx_strided_copy(const void* src, void* dst, int ndim, const int64_t* shape,
                     const int64_t* src_strides, int dtype, hipStream_t stream);

/* dst[i] = value for i < n.  Replaces launch_fill_kernel<T>
 * (include/cudeep/kernels/elementwise.cuh:23-24). */
int cdx_fill(void* dst, int64_t n, double value, int dtype, hipStream_t stream);

/* out = a (+|-|*) b elementwise, op = CDX_BINARY_*.  Replaces
 * launch_add_kernel / launch_sub_kernel / launch_mul_kernel
 * (include/cudeep/kernels/elementwise.cuh:8-15). */
int cdx_binary(int op, int dtype, const void* a, const void* b, void* out, int64_t n,
               hipStream_t stream);

/* dst[i] ~ N(0, 1): a pure function of (seed, offset, i) (SplitMix64 +
 * Box-Muller).  Replaces Tensor::randn's cuRAND generator
 * (src/tensor.cu:158-206); `offset` lets callers draw disjoint streams. */
int cdx_randn(void* dst, int64_t n, int dtype, uint64_t seed, uint64_t offset,
              hipStream_t stream);

/* out[0] = sum of x[0..n), deterministic two-stage reduction.  Replaces
 * launch_sum_kernel<T> (include/cudeep/kernels/reduce.cuh:9,
 * src/kernels/reduce_kernel.cu:21-195).  workspace may be NULL. */
size_t cdx_sum_workspace_size(int dtype);
int cdx_sum(const void* x, void* out, int64_t n, int dtype, void* workspace,
            size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CUDEEP_AMD_H */
