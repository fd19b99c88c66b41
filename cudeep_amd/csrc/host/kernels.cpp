// cudeep::kernels launchers (the reference's C++ operator API,
// include/cudeep/kernels/*.cuh) implemented over the C-ABI of
// libcudeep_amd.so.  Each template is explicitly instantiated for float and
// double, as the reference does.  GEMM epilogues are ReLU / GELU / SiLU /
// Sigmoid (the reference's GemmEpilogue set); the elementwise activation
// launchers take every ActivationType.
#include <atomic>
#include <string>

#include "../../../include/cudeep/error.hpp"
#include "../../../include/cudeep/kernels/activation.hpp"
#include "../../../include/cudeep/kernels/conv.hpp"
#include "../../../include/cudeep/kernels/elementwise.hpp"
#include "../../../include/cudeep/kernels/matmul.hpp"
#include "../../../include/cudeep/kernels/reduce.hpp"
#include "../../../include/cudeep/kernels/unary.hpp"
#include "../../../include/cudeep/memory.hpp"

namespace cudeep {
namespace kernels {

namespace {

std::atomic<int> g_precision{CDX_PREC_TF32MODE};
std::atomic<int> g_conv_algo{(int)ConvAlgorithm::Auto};

template <typename T>
constexpr int dtype_code() {
    return sizeof(T) == 4 ? CDX_DTYPE_F32 : CDX_DTYPE_F64;
}

int epi_code(GemmEpilogue e) {
    switch (e) {
        case GemmEpilogue::None: return CDX_EPI_NONE;
        case GemmEpilogue::ReLU: return CDX_EPI_RELU;
        case GemmEpilogue::GELU: return CDX_EPI_GELU;
        case GemmEpilogue::SiLU: return CDX_EPI_SILU;
        case GemmEpilogue::Sigmoid: return CDX_EPI_SIGMOID;
    }
    throw std::runtime_error("unknown GEMM epilogue");
}

int act_code(ActivationType a) {
    if (a == ActivationType::ReLU) return CDX_EPI_RELU;
    if (a == ActivationType::GELU) return CDX_EPI_GELU;
    if (a == ActivationType::SiLU) return CDX_EPI_SILU;
    if (a == ActivationType::Sigmoid) return CDX_EPI_SIGMOID;
    if (a == ActivationType::Tanh) return CDX_ACT_TANH;
    if (a == ActivationType::LeakyReLU) return CDX_ACT_LEAKY_RELU;
    throw std::runtime_error("unknown activation");
}

// Scratch for one launch.  On the null stream it comes from the runtime's
// exact-size scratch cache (MemoryPool::allocate_scratch) -- after the first
// call of a size a map lookup, where the stream-ordered pool costs tens of
// microseconds of host time for a large block -- and is handed back when the
// launch is enqueued: that cache serves only later null-stream launches,
// which the null stream orders after this one, never tensor storage.  On any
// other stream the C-ABI allocates stream-ordered itself.
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
    Workspace(size_t n, hipStream_t s) {
        if (n > 0 && s == nullptr) {
            ptr = MemoryPool::instance().allocate_scratch(n);
            bytes = n;
        }
    }
    ~Workspace() {
        if (!ptr) return;
        try {
            MemoryPool::instance().deallocate_scratch(ptr);
        } catch (...) {
            // (only an unknown pointer throws; never from a destructor)
        }
    }
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
};

}  // namespace

void set_conv_algorithm(ConvAlgorithm a) { g_conv_algo = (int)a; }

ConvAlgorithm get_conv_algorithm() { return (ConvAlgorithm)g_conv_algo.load(); }

void set_matmul_precision(MatmulPrecision p) {
    g_precision = p == MatmulPrecision::FP32       ? CDX_PREC_FP32
                  : p == MatmulPrecision::TF32Mode4 ? CDX_PREC_TF32MODE4
                                                    : CDX_PREC_TF32MODE;
}

MatmulPrecision get_matmul_precision() {
    const int p = g_precision.load();
    return p == CDX_PREC_FP32        ? MatmulPrecision::FP32
           : p == CDX_PREC_TF32MODE4 ? MatmulPrecision::TF32Mode4
                                     : MatmulPrecision::TF32Mode;
}

void launch_matmul_ex(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                      bool transA, bool transB, int64_t lda, int64_t ldb, int64_t ldc,
                      const float* bias, bool bias_per_col, GemmEpilogue epilogue,
                      hipStream_t stream, int precision) {
    const int prec = precision >= 0 ? precision : g_precision.load();
    const int bm = bias ? (bias_per_col ? CDX_BIAS_COL : CDX_BIAS_ROW) : CDX_BIAS_NONE;
    const int oa = transA ? CDX_OP_T : CDX_OP_N, ob = transB ? CDX_OP_T : CDX_OP_N;
    Workspace ws(cdx_gemm_workspace_size(prec, oa, ob, M, N, K), stream);
    CUDEEP_CHECK_CDX(cdx_gemm_ex_ws(prec, oa, ob, M, N, K, A, lda, B, ldb, C, ldc, bias, bm,
                                    epi_code(epilogue), ws.ptr, ws.bytes, stream));
}

void launch_linear_weight_grad(const float* dz, const float* x, float* grad_w, float* grad_b,
                               int64_t batch, int64_t out_features, int64_t in_features,
                               hipStream_t stream, int precision) {
    const int prec = precision >= 0 ? precision : g_precision.load();
    const int64_t ldz = out_features > 1 ? out_features : 1, ldx = in_features > 1 ? in_features : 1;
    Workspace ws(cdx_gemm_fused_workspace_size(prec, CDX_OP_T, CDX_OP_N, out_features,
                                               in_features, batch, grad_b != nullptr),
                 stream);
    CUDEEP_CHECK_CDX(cdx_gemm_fused(prec, CDX_OP_T, CDX_OP_N, out_features, in_features, batch,
                                    dz, ldz, x, ldx, grad_w, in_features, nullptr, CDX_BIAS_NONE,
                                    CDX_EPI_NONE, nullptr, 0, grad_b, ws.ptr, ws.bytes, stream));
}

void launch_linear_input_grad(const float* dz, const float* weight, const float* aux,
                              float* grad_x, int64_t batch, int64_t out_features,
                              int64_t in_features, GemmEpilogue act, hipStream_t stream,
                              int precision) {
    const int prec = precision >= 0 ? precision : g_precision.load();
    const int64_t ldz = out_features > 1 ? out_features : 1, ldw = in_features > 1 ? in_features : 1;
    int epi = CDX_EPI_NONE;
    switch (act) {
        case GemmEpilogue::None: break;
        case GemmEpilogue::ReLU: epi = CDX_EPI_BWD_RELU; break;
        case GemmEpilogue::GELU: epi = CDX_EPI_BWD_GELU; break;
        case GemmEpilogue::SiLU: epi = CDX_EPI_BWD_SILU; break;
        case GemmEpilogue::Sigmoid: epi = CDX_EPI_BWD_SIGMOID; break;
    }
    Workspace ws(cdx_gemm_fused_workspace_size(prec, CDX_OP_N, CDX_OP_N, batch, in_features,
                                               out_features, 0),
                 stream);
    CUDEEP_CHECK_CDX(cdx_gemm_fused(prec, CDX_OP_N, CDX_OP_N, batch, in_features, out_features,
                                    dz, ldz, weight, ldw, grad_x, in_features, nullptr,
                                    CDX_BIAS_NONE, epi, epi == CDX_EPI_NONE ? nullptr : aux,
                                    in_features, nullptr, ws.ptr, ws.bytes, stream));
}

void launch_matmul_dgemm_ex(const double* A, const double* B, double* C, int64_t M, int64_t N,
                            int64_t K, bool transA, bool transB, int64_t lda, int64_t ldb,
                            int64_t ldc, hipStream_t stream) {
    CUDEEP_CHECK_CDX(cdx_dgemm(transA ? CDX_OP_T : CDX_OP_N, transB ? CDX_OP_T : CDX_OP_N, M, N, K,
                               A, lda, B, ldb, C, ldc, stream));
}

template <>
void launch_matmul_kernel<float>(const float* A, const float* B, float* C, int M, int N, int K,
                                 hipStream_t stream) {
    launch_matmul_ex(A, B, C, M, N, K, false, false, K > 1 ? K : 1, N > 1 ? N : 1, N, nullptr,
                     true, GemmEpilogue::None, stream);
}

template <>
void launch_matmul_kernel<double>(const double* A, const double* B, double* C, int M, int N,
                                  int K, hipStream_t stream) {
    launch_matmul_dgemm_ex(A, B, C, M, N, K, false, false, K > 1 ? K : 1, N > 1 ? N : 1, N,
                           stream);
}

template <>
void launch_matmul_kernel_fp32<float>(const float* A, const float* B, float* C, int M, int N,
                                      int K, hipStream_t stream) {
    CUDEEP_CHECK_CDX(cdx_sgemm_f32(A, B, C, M, N, K, stream));
}

void launch_matmul_kernel_fp16(const __half* A, const __half* B, float* C, int M, int N, int K,
                               hipStream_t stream) {
    CUDEEP_CHECK_CDX(cdx_hgemm_f16(A, B, C, M, N, K, stream));
}

template <>
void launch_matmul_kernel_fp32<double>(const double* A, const double* B, double* C, int M, int N,
                                       int K, hipStream_t stream) {
    launch_matmul_kernel<double>(A, B, C, M, N, K, stream);
}

template <typename T>
void launch_matmul_tiled_kernel(const T* A, const T* B, T* C, int M, int N, int K, int,
                                hipStream_t stream) {
    launch_matmul_kernel<T>(A, B, C, M, N, K, stream);
}
template void launch_matmul_tiled_kernel<float>(const float*, const float*, float*, int, int, int,
                                                int, hipStream_t);
template void launch_matmul_tiled_kernel<double>(const double*, const double*, double*, int, int,
                                                 int, int, hipStream_t);

void launch_matmul_fused_act(const float* A, const float* B, float* C, int M, int N, int K,
                             GemmEpilogue epilogue, hipStream_t stream) {
    launch_matmul_ex(A, B, C, M, N, K, false, false, K > 1 ? K : 1, N > 1 ? N : 1, N, nullptr,
                     true, epilogue, stream);
}

// ---- conv ------------------------------------------------------------------

template <>
void launch_conv2d_forward_kernel<float>(const float* input, const float* weight, const float* bias,
                                         float* output, int batch, int IC, int OC, int IH, int IW,
                                         int KH, int KW, int SH, int SW, int PH, int PW,
                                         hipStream_t stream) {
    const int64_t OH = ((int64_t)IH + 2 * PH - KH) / SH + 1;
    const int64_t OW = ((int64_t)IW + 2 * PW - KW) / SW + 1;
    const bool wino_ok = KH == 3 && KW == 3 && SH == 1 && SW == 1;
    const ConvAlgorithm algo = get_conv_algorithm();
    if (algo == ConvAlgorithm::Winograd && !wino_ok)
        throw std::runtime_error("conv2d: Winograd needs a 3x3 kernel with stride 1");
    const bool wino = algo == ConvAlgorithm::Winograd ||
                      (algo == ConvAlgorithm::Auto && wino_ok && OH * OW >= 16);
    if (algo == ConvAlgorithm::Implicit) {
        CUDEEP_CHECK_CDX(cdx_conv2d_forward_implicit_f32(input, weight, bias, output, batch, IC,
                                                         OC, IH, IW, KH, KW, SH, SW, PH, PW,
                                                         stream));
    } else if (wino) {
        Workspace ws(cdx_conv2d_winograd_workspace_size(batch, IC, OC, IH, IW, PH, PW), stream);
        CUDEEP_CHECK_CDX(cdx_conv2d_forward_winograd_f32(input, weight, bias, output, batch, IC,
                                                         OC, IH, IW, PH, PW, g_precision.load(),
                                                         ws.ptr, ws.bytes, stream));
    } else {
        Workspace ws(cdx_conv2d_forward_workspace_size(batch, IC, IH, IW, KH, KW, SH, SW, PH, PW),
                     stream);
        CUDEEP_CHECK_CDX(cdx_conv2d_forward_f32(input, weight, bias, output, batch, IC, OC, IH, IW,
                                                KH, KW, SH, SW, PH, PW, g_precision.load(),
                                                ws.ptr, ws.bytes, stream));
    }
}

template <>
void launch_conv2d_forward_kernel<double>(const double* input, const double* weight,
                                          const double* bias, double* output, int batch, int IC,
                                          int OC, int IH, int IW, int KH, int KW, int SH, int SW,
                                          int PH, int PW, hipStream_t stream) {
    CUDEEP_CHECK_CDX(cdx_conv2d_forward_f64(input, weight, bias, output, batch, IC, OC, IH, IW,
                                            KH, KW, SH, SW, PH, PW, stream));
}

template <>
void launch_conv2d_backward_data_kernel<float>(const float* grad_output, const float* weight,
                                               float* grad_input, int batch, int IC, int OC,
                                               int IH, int IW, int KH, int KW, int SH, int SW,
                                               int PH, int PW, hipStream_t stream) {
    // The forward's rule, applied to the transposed convolution that
    // produces grad_input (3x3, stride 1, padding 2 - P >= 0, IH*IW pixels),
    // in the TF32 modes only: the reference's backward data is GEMM +
    // col2im, and in FP32 the Winograd transforms' rounding (~10x that
    // route's error) would not stay within twice its error, so Auto keeps
    // cdx_conv2d_backward_data_f32's flipped-filter implicit route there.
    const int prec = g_precision.load();
    const bool wino_ok = KH == 3 && KW == 3 && SH == 1 && SW == 1 && PH <= 2 && PW <= 2;
    const ConvAlgorithm algo = get_conv_algorithm();
    if (algo == ConvAlgorithm::Winograd && !wino_ok)
        throw std::runtime_error(
            "conv2d backward: Winograd needs a 3x3 kernel with stride 1 and padding <= 2");
    const bool wino = algo == ConvAlgorithm::Winograd ||
                      (algo == ConvAlgorithm::Auto && wino_ok && (int64_t)IH * IW >= 16 &&
                       prec != CDX_PREC_FP32);
    if (wino) {
        Workspace ws(cdx_conv2d_backward_data_winograd_workspace_size(batch, IC, OC, IH, IW, PH,
                                                                      PW),
                     stream);
        CUDEEP_CHECK_CDX(cdx_conv2d_backward_data_winograd_f32(grad_output, weight, grad_input,
                                                               batch, IC, OC, IH, IW, PH, PW,
                                                               prec, ws.ptr, ws.bytes, stream));
    } else {
        Workspace ws(cdx_conv2d_backward_data_workspace_size(batch, IC, OC, IH, IW, KH, KW, SH, SW,
                                                             PH, PW),
                     stream);
        CUDEEP_CHECK_CDX(cdx_conv2d_backward_data_f32(grad_output, weight, grad_input, batch, IC,
                                                      OC, IH, IW, KH, KW, SH, SW, PH, PW, prec,
                                                      ws.ptr, ws.bytes, stream));
    }
}

template <>
void launch_conv2d_backward_data_kernel<double>(const double* grad_output, const double* weight,
                                                double* grad_input, int batch, int IC, int OC,
                                                int IH, int IW, int KH, int KW, int SH, int SW,
                                                int PH, int PW, hipStream_t stream) {
    CUDEEP_CHECK_CDX(cdx_conv2d_backward_data_f64(grad_output, weight, grad_input, batch, IC, OC,
                                                  IH, IW, KH, KW, SH, SW, PH, PW, stream));
}

template <>
void launch_conv2d_backward_weight_kernel<float>(const float* grad_output, const float* input,
                                                 float* grad_weight, int batch, int IC, int OC,
                                                 int IH, int IW, int KH, int KW, int SH, int SW,
                                                 int PH, int PW, hipStream_t stream) {
    Workspace ws(cdx_conv2d_backward_weight_workspace_size(batch, IC, OC, IH, IW, KH, KW, SH, SW,
                                                           PH, PW),
                 stream);
    CUDEEP_CHECK_CDX(cdx_conv2d_backward_weight_f32(grad_output, input, grad_weight, batch, IC,
                                                    OC, IH, IW, KH, KW, SH, SW, PH, PW,
                                                    g_precision.load(), ws.ptr, ws.bytes, stream));
}

template <>
void launch_conv2d_backward_weight_kernel<double>(const double* grad_output, const double* input,
                                                  double* grad_weight, int batch, int IC, int OC,
                                                  int IH, int IW, int KH, int KW, int SH, int SW,
                                                  int PH, int PW, hipStream_t stream) {
    CUDEEP_CHECK_CDX(cdx_conv2d_backward_weight_f64(grad_output, input, grad_weight, batch, IC,
                                                    OC, IH, IW, KH, KW, SH, SW, PH, PW, stream));
}

void launch_conv2d_backward_bias_kernel(const float* grad_output, float* grad_bias, int batch,
                                        int out_channels, int spatial, hipStream_t stream) {
    CUDEEP_CHECK_CDX(cdx_conv2d_backward_bias_f32(grad_output, grad_bias, batch, out_channels,
                                                  spatial, stream));
}

void launch_conv2d_backward_bias_kernel(const double* grad_output, double* grad_bias, int batch,
                                        int out_channels, int spatial, hipStream_t stream) {
    CUDEEP_CHECK_CDX(cdx_conv2d_backward_bias_f64(grad_output, grad_bias, batch, out_channels,
                                                  spatial, stream));
}

// ---- elementwise / reductions / activations ---------------------------------

template <typename T>
void launch_add_kernel(const T* a, const T* b, T* out, int64_t n, hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_binary(CDX_BINARY_ADD, dtype_code<T>(), a, b, out, n, s));
}
template <typename T>
void launch_sub_kernel(const T* a, const T* b, T* out, int64_t n, hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_binary(CDX_BINARY_SUB, dtype_code<T>(), a, b, out, n, s));
}
template <typename T>
void launch_mul_kernel(const T* a, const T* b, T* out, int64_t n, hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_binary(CDX_BINARY_MUL, dtype_code<T>(), a, b, out, n, s));
}
template <typename T>
void launch_fill_kernel(T* data, T value, int64_t n, hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_fill(data, n, (double)value, dtype_code<T>(), s));
}

template <>
void launch_broadcast_add_row_kernel<float>(const float* m, const float* row, float* out,
                                            int64_t rows, int64_t cols, hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_broadcast_add_row_f32(m, row, out, rows, cols, s));
}

template <>
void launch_broadcast_add_row_kernel<double>(const double* m, const double* row, double* out,
                                             int64_t rows, int64_t cols, hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_broadcast_add_row_f64(m, row, out, rows, cols, s));
}

template <>
void launch_sum_reduce_rows_kernel<float>(const float* in, float* out, int64_t rows, int64_t cols,
                                          hipStream_t s) {
    Workspace ws(cdx_sum_reduce_rows_workspace_size(rows, cols), s);
    CUDEEP_CHECK_CDX(cdx_sum_reduce_rows_f32(in, out, rows, cols, ws.ptr, ws.bytes, s));
}

template <>
void launch_sum_reduce_rows_kernel<double>(const double* in, double* out, int64_t rows,
                                           int64_t cols, hipStream_t s) {
    Workspace ws(cdx_sum_reduce_rows_workspace_size(rows, cols), s);
    CUDEEP_CHECK_CDX(cdx_sum_reduce_rows_f64(in, out, rows, cols, ws.ptr, ws.bytes, s));
}

template <typename T>
void launch_sum_kernel(const T* input, T* output, int64_t n, hipStream_t s) {
    Workspace ws(cdx_sum_workspace_size(dtype_code<T>()), s);
    CUDEEP_CHECK_CDX(cdx_sum(input, output, n, dtype_code<T>(), ws.ptr, ws.bytes, s));
}

template <>
void launch_activation_forward_kernel<float>(const float* in, float* out, int64_t n,
                                             ActivationType act, float alpha, hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_activation_forward_f32(in, out, n, act_code(act), alpha, s));
}

template <>
void launch_activation_forward_kernel<double>(const double* in, double* out, int64_t n,
                                              ActivationType act, float alpha, hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_activation_forward_f64(in, out, n, act_code(act), alpha, s));
}

template <>
void launch_activation_backward_kernel<float>(const float* go, const float* in, float* gi,
                                              int64_t n, ActivationType act, float alpha,
                                              hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_activation_backward_f32(go, in, gi, n, act_code(act), alpha, s));
}

template <>
void launch_activation_backward_kernel<double>(const double* go, const double* in, double* gi,
                                               int64_t n, ActivationType act, float alpha,
                                               hipStream_t s) {
    CUDEEP_CHECK_CDX(cdx_activation_backward_f64(go, in, gi, n, act_code(act), alpha, s));
}

#define CDX_INST(T)                                                                         \
    template void launch_add_kernel<T>(const T*, const T*, T*, int64_t, hipStream_t);       \
    template void launch_sub_kernel<T>(const T*, const T*, T*, int64_t, hipStream_t);       \
    template void launch_mul_kernel<T>(const T*, const T*, T*, int64_t, hipStream_t);       \
    template void launch_fill_kernel<T>(T*, T, int64_t, hipStream_t);                       \
    template void launch_sum_kernel<T>(const T*, T*, int64_t, hipStream_t);
CDX_INST(float)
CDX_INST(double)
#undef CDX_INST

}  // namespace kernels
}  // namespace cudeep
