// Internal declarations shared by the gfx950 kernels and the C-ABI layer.
// Nothing here crosses the library boundary; the public contract is
// include/cudeep_amd.h.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>

#include "../../include/cudeep_amd.h"

namespace cdx {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef double doublex4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short shortx8 __attribute__((ext_vector_type(8)));

// Records a message for cdx_last_error() on this thread and returns `code`.
int set_error(int code, const std::string& msg);
int hip_error(hipError_t e, const char* what);

// Stream-ordered scratch for calls without a caller workspace: blocks from a
// library-owned memory pool per device whose release threshold keeps freed
// memory for reuse.  (The device's default pool hands freed memory back to
// the driver at every synchronization, so a large workspace -- 231 MB for a
// C5 backward-data column buffer -- was mapped again on every call, ~150 us
// of host time per free.)
int stream_alloc(void** p, size_t bytes, hipStream_t stream, const char* what);
int stream_free(void* p, hipStream_t stream, const char* what);

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Division by a run-time constant d (1 <= d < 2^31) of n < 2^31 by a
// multiply-high: q = (mulhi(n, m) + n) >> l (Granlund & Montgomery 1994).
struct DivMagic {
    uint32_t m;
    int l;
};

inline DivMagic div_magic(int64_t d) {
    int l = 0;
    while (((int64_t)1 << l) < d) ++l;
    const uint64_t m = ((((uint64_t)1 << 32) * (((uint64_t)1 << l) - (uint64_t)d)) / (uint64_t)d) + 1;
    return {(uint32_t)m, l};
}

__device__ __forceinline__ uint32_t div_u31(uint32_t n, DivMagic g) {
    return (__umulhi(n, g.m) + n) >> g.l;
}

// One GEMM problem in the library's internal form.  Element (i, j) of op(A)
// is A[i*lda + j] (opA = N) or A[j*lda + i] (opA = T); likewise for B.
// C is written through the output map:
//   addr(m, n) = m * ldc + (n / n_split) * ldc_split + (n % n_split)
// n_split = 0 means the plain row-major map addr = m * ldc + n.  The split
// map writes the conv GEMM's [OC, B*S] result straight into NCHW.
// A and B point at fp32 elements, or at 16-bit ones for launch_gemm_16.
struct GemmArgs {
    int opA, opB;
    int64_t M, N, K;
    const void* A; int64_t lda;
    const void* B; int64_t ldb;
    float* C; int64_t ldc;
    int64_t n_split, ldc_split;
    const float* bias; int bias_mode;   // CDX_BIAS_*
    int epilogue;                       // CDX_EPI_*
    // Batched form: `batch` independent problems, problem z at A + z*stride_a,
    // B + z*stride_b, C + z*stride_c (elements); bias shared.
    int64_t batch = 1, stride_a = 0, stride_b = 0, stride_c = 0;
    // FP32 NN products only: sum k in two levels (32-k partial sums added to
    // the running total) instead of one running sum -- a rounding-error
    // chain of ~32 + K/32 additions instead of ~K.
    bool blocked_sum = false;
    // Caller scratch for split-K partials (the launchers allocate stream-
    // ordered when it is null); gemm_*_workspace() gives the bytes needed.
    void* ws = nullptr;
    size_t ws_bytes = 0;
    // Activation-backward epilogues (CDX_EPI_BWD_*): C = P * act'(aux), aux
    // [M, N] with leading dimension ldaux (plain output map, no bias).
    const float* aux = nullptr;
    int64_t ldaux = 0;
    // colsum[m] = sum_k op(A)(m, k), computed as an extra output column N of
    // the product with a virtual column of ones appended to op(B) (FP32
    // kernel only; plain output map, no bias, no epilogue).
    float* colsum = nullptr;
    // Set by with_ones_column(): op(B) has ones_col columns and the product
    // N = ones_col + 1 (the last one the virtual ones column); -1 = none.
    int64_t ones_col = -1;
};

// The GEMM with the ones column appended (for GemmArgs::colsum).
inline GemmArgs with_ones_column(GemmArgs g) {
    g.ones_col = g.N;
    g.N += 1;
    return g;
}

// Launchers (no argument validation: the C-ABI validates first).  The
// *_workspace functions return the split-K partial bytes the same launch
// would use (0 when it does not split); they follow the launchers' own
// configuration choice.
int launch_gemm_f32(const GemmArgs& g, hipStream_t stream);
size_t gemm_f32_workspace(const GemmArgs& g);
size_t gemm_bf16x3_workspace(const GemmArgs& g, int terms);
// terms = 3 (bf16x3: hi*hi + hi*lo + lo*hi) or 4 (adds lo*lo).
int launch_gemm_bf16x3(const GemmArgs& g, int terms, hipStream_t stream);
// 16-bit operands (in_dtype CDX_DTYPE_F16 or CDX_DTYPE_BF16), fp32 accumulation and C.
int launch_gemm_16(const GemmArgs& g, int in_dtype, hipStream_t stream);
// GEMMs with K <= 16 (narrow_kind 1) or N <= 16 (2), plain output map, no
// batch / ones column, no workspace; or M <= 16 with op(B) = B and K >= 1024
// (3, ones column allowed: split-K partials of skinny_m_workspace bytes).
// 0: use the tiled kernels.
int narrow_kind(const GemmArgs& g);
size_t skinny_m_workspace(const GemmArgs& g);
// The FP32 GEMM's 128 x 112 tiles apply (widths a multiple of 112 but not
// of 64, enough rows): faster than the split-precision kernels there.
bool f32_takes_w112(const GemmArgs& g);
int launch_gemm_narrow(const GemmArgs& g, hipStream_t stream);
int launch_dgemm(int opA, int opB, int64_t M, int64_t N, int64_t K,
                 const double* A, int64_t lda, const double* B, int64_t ldb,
                 double* C, int64_t ldc, hipStream_t stream);

// Split-K reduction: C = epi(sum_s P[s] + bias) through the output map, the
// partials summed in slice order (deterministic).  P is [splits][M][N]; with
// a ones column its sums go to g.colsum.
int launch_splitk_reduce(const float* P, int splits, const GemmArgs& g, hipStream_t stream);

// Split-K policy shared by the GEMM kernels: split only when the tile grid
// cannot fill the GPU (fewer than 128 tiles) and K is long; aim at ~768
// workgroups with at least min_k k per slice.  FP32 (BK 16) uses min_k 256
// (measured on the MLP / conv weight gradients: 10x256x8192 best at 32
// slices; 256x784x8192 at ~16 on 64x64 slices and at the 29 this gives on
// the 128x64 slices it takes now -- 15 / 20 slices: 52.5-55.9 against 48
// us; 64x576x100352 at ~64-128); the bf16x3 kernels
// (BK 32-64, a longer pipeline fill per slice) 1024 (256x784x8192: 8 slices
// 47.6 us NN / 35.2 NT against 55.9 / 42.3 at 15).  Returns the slice count
// and sets *k_chunk (a multiple of bk).
inline bool splitk_applies(int64_t tiles, int64_t K) { return tiles < 128 && K >= 2048; }

inline int choose_splitk(int64_t tiles, int64_t K, int bk, int64_t* k_chunk, int64_t min_k = 256) {
    *k_chunk = K;
    if (!splitk_applies(tiles, K)) return 1;
    int64_t s = (768 + tiles / 2) / tiles;
    if (s > K / min_k) s = K / min_k;
    if (s < 2) return 1;
    int64_t kc = ceil_div(ceil_div(K, s), bk) * bk;
    *k_chunk = kc;
    return (int)ceil_div(K, kc);
}

// Split-K partial bytes of a GEMM whose tile grid is `tiles` (0: no split).
inline size_t splitk_bytes(const GemmArgs& g, int64_t tiles, int bk, int64_t min_k = 256) {
    if (g.batch > 1) return 0;
    int64_t k_chunk;
    const int splits = choose_splitk(tiles, g.K, bk, &k_chunk, min_k);
    return splits > 1 ? (size_t)splits * (size_t)g.M * (size_t)g.N * sizeof(float) : 0;
}

// Runs a GEMM whose tile grid is `tiles` through split-K when the policy
// asks for it: takes the partials from g.ws (or allocates them stream-
// ordered), calls launch(kparams-adjusted GemmArgs, splits, k_chunk) and
// reduces.
template <class LaunchFn>
int with_splitk(const GemmArgs& g, int64_t tiles, int bk, hipStream_t stream, LaunchFn launch,
                int64_t min_k = 256) {
    int64_t k_chunk;
    const int splits = g.batch > 1 ? (k_chunk = g.K, 1)
                                   : choose_splitk(tiles, g.K, bk, &k_chunk, min_k);
    if (splits == 1) return launch(g, 1, g.K);
    float* part = static_cast<float*>(g.ws);
    const size_t bytes = (size_t)splits * (size_t)g.M * (size_t)g.N * sizeof(float);
    int st = CDX_OK;
    if (part) {
        if (g.ws_bytes < bytes) return set_error(CDX_ERR_WORKSPACE, "gemm: workspace too small");
    } else {
        st = stream_alloc(reinterpret_cast<void**>(&part), bytes, stream, "gemm split-K scratch");
        if (st) return st;
    }
    GemmArgs q = g;
    q.C = part; q.ldc = g.N; q.n_split = 0; q.ldc_split = 0;
    q.bias = nullptr; q.bias_mode = CDX_BIAS_NONE; q.epilogue = CDX_EPI_NONE;
    q.aux = nullptr; q.colsum = nullptr;   // the reduction applies both
    st = launch(q, splits, k_chunk);
    if (!st) st = launch_splitk_reduce(part, splits, g, stream);
    if (!g.ws) {
        int st2 = stream_free(part, stream, "gemm split-K scratch");
        if (!st) st = st2;
    }
    return st;
}

int launch_im2col_f32(const float* in, float* col, int64_t batch, int64_t IC,
                      int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                      int64_t SH, int64_t SW, int64_t PH, int64_t PW,
                      hipStream_t stream);

// Winograd F(4x4, 3x3) forward for 3x3 stride-1 convolution; ws holds
// winograd_workspace_floats(...) floats (U, V and M).  With flip_filter the
// filter is read as the stride-1 transposed convolution's: weight is
// [IC][OC][3][3] (the forward layer's OIHW with O = this call's IC) and is
// used channel-swapped and spatially reversed (backward data).
size_t winograd_workspace_floats(int64_t batch, int64_t IC, int64_t OC, int64_t OH, int64_t OW);
int launch_conv2d_winograd_f32(const float* input, const float* weight, const float* bias,
                               float* output, int64_t batch, int64_t IC, int64_t OC,
                               int64_t IH, int64_t IW, int64_t PH, int64_t PW, int precision,
                               float* ws, hipStream_t stream, bool flip_filter = false);

// wf[ic][oc][k'] = w[oc][ic][KHW-1-k'] (stride-1 transposed-conv filter).
int launch_flip_filter_f32(const float* w, float* wf, int64_t OC, int64_t IC, int64_t KHW,
                           hipStream_t stream);

// Conv backward weight as an implicit GEMM (FP32 MFMA; operands gathered
// from NCHW dY and x, no column buffer).  `ws` holds
// conv_wgrad_implicit_floats(...) floats (the split partials).
bool conv_wgrad_implicit_ok(int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                            int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                            int64_t PW);
size_t conv_wgrad_implicit_floats(int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                                  int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                                  int64_t PW);
int launch_conv_wgrad_f32(const float* dy, const float* x, float* dw, float* ws, int64_t batch,
                          int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                          int64_t SH, int64_t SW, int64_t PH, int64_t PW, hipStream_t stream);

// Conv forward as an implicit GEMM (FP32 MFMA, operands gathered from the
// NCHW input while staging k-tiles; no column buffer), with bias; output
// NCHW.  conv_fwd_implicit_ok() gives the geometries it takes (32-bit
// in-image and pixel indices).
bool conv_fwd_implicit_ok(int64_t batch, int64_t IC, int64_t IH, int64_t IW, int64_t KH,
                          int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW);
int launch_conv_fwd_implicit_f32(const float* x, const float* w, const float* bias, float* y,
                                 int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                                 int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                                 int64_t PW, hipStream_t stream);
// The same product in its row-window form (the input window of a 128-pixel
// tile staged in LDS per 16-channel chunk; any kernel size and stride whose
// window fits).  two_level: each run of 32 consecutive k summed from zero,
// then added to the total (the FP32 backward-data route).
bool conv_rowwin_ok(int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH,
                    int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW);
int launch_conv_rowwin_f32(const float* x, const float* w, const float* bias, float* y,
                           int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                           int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                           int64_t PW, bool two_level, hipStream_t stream);

int launch_col2im_f32(const float* col, float* grad_in, int64_t batch, int64_t IC,
                      int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                      int64_t SH, int64_t SW, int64_t PH, int64_t PW, hipStream_t stream);
int launch_nchw_to_cm_f32(const float* src, float* dst, int64_t batch, int64_t C, int64_t S,
                          hipStream_t stream);
int launch_conv_bias_grad_f32(const float* dy, float* db, int64_t batch, int64_t C, int64_t S,
                              hipStream_t stream);

// float64 conv (conv_f64.hip): direct fp64 sums, one chain per output.
int launch_conv2d_forward_f64(const double* x, const double* w, const double* bias, double* out,
                              int64_t B, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                              int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                              int64_t PW, hipStream_t stream);
int launch_conv2d_backward_data_f64(const double* dy, const double* w, double* dx, int64_t B,
                                    int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH,
                                    int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW,
                                    hipStream_t stream);
int launch_conv2d_backward_weight_f64(const double* dy, const double* x, double* dw, int64_t B,
                                      int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH,
                                      int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW,
                                      hipStream_t stream);
int launch_conv_bias_grad_f64(const double* dy, double* db, int64_t B, int64_t C, int64_t S,
                              hipStream_t stream);

int launch_strided_copy(const void* src, void* dst, int ndim, const int64_t* shape,
                        const int64_t* strides, int dtype, hipStream_t stream);
int launch_fill(void* dst, int64_t n, double v, int dtype, hipStream_t stream);
int launch_binary(int op, int dtype, const void* a, const void* b, void* y, int64_t n,
                  hipStream_t stream);
int launch_randn(void* dst, int64_t n, int dtype, uint64_t seed, uint64_t offset,
                 hipStream_t stream);
int64_t sum_partials();
int launch_sum(const void* x, void* out, int64_t n, int dtype, void* partials,
               hipStream_t stream);

int launch_colsum_f32(const float* in, float* out, int64_t rows, int64_t cols,
                      float* partials, int64_t partial_rows, hipStream_t stream);
int64_t colsum_partial_rows(int64_t rows, int64_t cols);

int launch_colsum_f64(const double* in, double* out, int64_t rows, int64_t cols,
                      double* partials, int64_t partial_rows, hipStream_t stream);
int launch_broadcast_add_row_f32(const float* m, const float* row, float* out,
                                 int64_t rows, int64_t cols, hipStream_t stream);
int launch_broadcast_add_row_f64(const double* m, const double* row, double* out,
                                 int64_t rows, int64_t cols, hipStream_t stream);
int launch_activation_f32(const float* in, float* out, int64_t n, int act, float alpha,
                          hipStream_t stream);
int launch_activation_f64(const double* in, double* out, int64_t n, int act, float alpha,
                          hipStream_t stream);
int launch_activation_backward_f32(const float* grad_out, const float* in, float* grad_in,
                                   int64_t n, int act, float alpha, hipStream_t stream);
int launch_activation_backward_f64(const double* grad_out, const double* in, double* grad_in,
                                   int64_t n, int act, float alpha, hipStream_t stream);

// GELU, tanh form 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3)
// (Hendrycks & Gimpel 2016; the reference's constants 0.7978845608 and
// 0.044715, activation_kernel.cu:40-46).  Evaluated through the identity
// 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)), which has no cancellation in
// either tail: gelu(x) = x / (1 + exp(-2u)).
__device__ __forceinline__ float gelu_f32(float x) {
    const float c = 0.7978845608f, k = 0.044715f;
    float u = c * (x + k * x * x * x);
    return x / (1.0f + expf(-2.0f * u));
}

// d gelu / dx = s + 2 x s (1 - s) du/dx with s = 1 / (1 + exp(-2u)),
// since 0.5 (1 - tanh^2 u) = 2 s (1 - s); 1 - s = 1 / (1 + exp(2u)) is
// computed directly so neither factor cancels or overflows to inf * 0.
__device__ __forceinline__ float gelu_grad_f32(float x) {
    const float c = 0.7978845608f, k = 0.044715f;
    float u = c * (x + k * x * x * x);
    float s = 1.0f / (1.0f + expf(-2.0f * u));
    float one_minus_s = 1.0f / (1.0f + expf(2.0f * u));
    float du = c * (1.0f + 3.0f * k * x * x);
    return s + 2.0f * x * s * one_minus_s * du;
}

// fp64 GELU / GELU' with the same formulas in double precision.
__device__ __forceinline__ double gelu_f64(double x) {
    const double c = 0.7978845608, k = 0.044715;
    double u = c * (x + k * x * x * x);
    return x / (1.0 + exp(-2.0 * u));
}

__device__ __forceinline__ double gelu_grad_f64(double x) {
    const double c = 0.7978845608, k = 0.044715;
    double u = c * (x + k * x * x * x);
    double s = 1.0 / (1.0 + exp(-2.0 * u));
    double one_minus_s = 1.0 / (1.0 + exp(2.0 * u));
    double du = c * (1.0 + 3.0 * k * x * x);
    return s + 2.0 * x * s * one_minus_s * du;
}

__device__ __forceinline__ float exp_t(float x) { return expf(x); }
__device__ __forceinline__ double exp_t(double x) { return exp(x); }

// Sigmoid 1 / (1 + exp(-x)) and SiLU x * sigmoid(x) (the reference's
// epilogue definitions, matmul_kernel.cu:1538-1550).  For x -> -inf,
// exp(-x) overflows to inf and both go to (-)0 without a NaN.
template <typename T>
__device__ __forceinline__ T sigmoid_t(T x) { return T(1) / (T(1) + exp_t(-x)); }
template <typename T>
__device__ __forceinline__ T silu_t(T x) { return x / (T(1) + exp_t(-x)); }
// sigmoid' = s (1 - s);  silu' = s + x s (1 - s), with 1 - s = 1 / (1 + e^x)
// computed directly (no cancellation for large x).
template <typename T>
__device__ __forceinline__ T sigmoid_grad_t(T x) {
    return T(1) / (T(1) + exp_t(-x)) * (T(1) / (T(1) + exp_t(x)));
}
template <typename T>
__device__ __forceinline__ T silu_grad_t(T x) {
    const T s = T(1) / (T(1) + exp_t(-x)), one_minus_s = T(1) / (T(1) + exp_t(x));
    return s + x * s * one_minus_s;
}

__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == CDX_EPI_RELU) return v > 0.0f ? v : 0.0f;
    if (act == CDX_EPI_GELU) return gelu_f32(v);
    if (act == CDX_EPI_SILU) return silu_t(v);
    if (act == CDX_EPI_SIGMOID) return sigmoid_t(v);
    return v;
}

template <int ACT>
__device__ __forceinline__ float act_fixed(float v) {
    if constexpr (ACT == CDX_EPI_RELU) return v > 0.0f ? v : 0.0f;
    if constexpr (ACT == CDX_EPI_GELU) return gelu_f32(v);
    if constexpr (ACT == CDX_EPI_SILU) return silu_t(v);
    if constexpr (ACT == CDX_EPI_SIGMOID) return sigmoid_t(v);
    return v;
}

// Activation-backward epilogues: grad * act'(x) with the same float formulas
// (and operand order) as the elementwise activation-backward kernels, so the
// fused and the separate forms agree bit for bit; ReLU is the mask x > 0.
template <int ACT>
__device__ __forceinline__ float bwd_fixed(float g, float x) {
    if constexpr (ACT == CDX_EPI_BWD_RELU) return x > 0.0f ? g : 0.0f;
    if constexpr (ACT == CDX_EPI_BWD_GELU) return g * gelu_grad_f32(x);
    if constexpr (ACT == CDX_EPI_BWD_SILU) return g * silu_grad_t(x);
    if constexpr (ACT == CDX_EPI_BWD_SIGMOID) return g * sigmoid_grad_t(x);
    return g;
}

__device__ __forceinline__ bool is_bwd_epilogue(int e) {
    return e >= CDX_EPI_BWD_RELU && e <= CDX_EPI_BWD_SIGMOID;
}

// Where a GEMM's output element (m, n) goes, with the bias and activation
// of the epilogue (see GemmArgs for the output map).  With colsum set the
// kernel computes N = n_main + 1 columns and column n_main goes to
// colsum[m] (plain, no bias or activation).
struct EpiArgs {
    float* C; int64_t ldc, M, N, n_split, ldc_split;
    const float* bias; int bias_mode, epilogue;
    const float* aux = nullptr; int64_t ldaux = 0;
    float* colsum = nullptr; int64_t n_main = 0;
};

// One output element through the epilogue, the activation chosen at run
// time: the operations and their order of write_acc_act below.
__device__ __forceinline__ void store_one(const EpiArgs& e, int64_t m, int64_t n, float v) {
    if (e.colsum && n == e.n_main) {
        e.colsum[m] = v;
        return;
    }
    float r;
    if (is_bwd_epilogue(e.epilogue)) {
        const float x = e.aux[m * e.ldaux + n];
        switch (e.epilogue) {
            case CDX_EPI_BWD_RELU: r = bwd_fixed<CDX_EPI_BWD_RELU>(v, x); break;
            case CDX_EPI_BWD_GELU: r = bwd_fixed<CDX_EPI_BWD_GELU>(v, x); break;
            case CDX_EPI_BWD_SILU: r = bwd_fixed<CDX_EPI_BWD_SILU>(v, x); break;
            default: r = bwd_fixed<CDX_EPI_BWD_SIGMOID>(v, x); break;
        }
    } else {
        const float bcol = e.bias_mode == CDX_BIAS_COL ? e.bias[n] : 0.0f;
        const float brow = e.bias_mode == CDX_BIAS_ROW ? e.bias[m] : 0.0f;
        r = apply_act(v + bcol + brow, e.epilogue);
    }
    const int64_t col = e.n_split > 0 ? (n / e.n_split) * e.ldc_split + n % e.n_split : n;
    e.C[m * e.ldc + col] = r;
}

// Row (or column) of element `idx` (0..15) of 16 x 16 accumulator block
// `blk` in a wave tile whose blocks are interleaved V at a time: block blk
// covers rows 16 V (blk / V) + V idx + blk % V.  V = 1 is the plain layout
// (rows 16 blk + idx); V = 2 / 4 is the layout an m/n-contiguous operand
// gets when each lane reads V consecutive rows with one LDS read and feeds
// them to V different MFMAs.
template <int V>
__device__ __forceinline__ int blk_pos(int blk, int idx) {
    return 16 * V * (blk / V) + V * idx + blk % V;
}

// Writes one wave's FM x FN grid of 16 x 16 MFMA accumulator tiles (D
// layout of v_mfma_f32_16x16x*: register r of lane l is row 4 (l / 16) + r,
// column l % 16 of its block), whose top-left element is (m0, n0); VM / VN
// are the row / column block interleaves (blk_pos).  The activation is a
// template parameter so the per-element code is straight-line; CHECK adds
// the M / N bounds tests that ragged tiles need.
template <int FM, int FN, bool CHECK, bool SPLITN, int ACT, int VM = 1, int VN = 1>
__device__ __forceinline__ void write_acc_act(const floatx4 (&acc)[FM][FN], const EpiArgs& e,
                                              int64_t m0, int64_t n0, int lane) {
    const int l16 = lane & 15, lq = lane >> 4;
    const bool bias_col = e.bias_mode == CDX_BIAS_COL, bias_row = e.bias_mode == CDX_BIAS_ROW;
    int64_t col_off[FN];
    float bcol[FN];
#pragma unroll
    for (int jn = 0; jn < FN; ++jn) {
        const int64_t n = n0 + blk_pos<VN>(jn, l16);
        col_off[jn] = n;
        if (SPLITN) {
            // NCHW map; 32-bit quotient when it fits (a 64-bit divide is a
            // long instruction sequence)
            if (e.N <= (int64_t)UINT32_MAX) {
                const uint32_t nn = (uint32_t)n, ns = (uint32_t)e.n_split;
                const uint32_t q = nn / ns;
                col_off[jn] = (int64_t)q * e.ldc_split + (int64_t)(nn - q * ns);
            } else {
                col_off[jn] = (n / e.n_split) * e.ldc_split + (n % e.n_split);
            }
        }
        bcol[jn] = (bias_col && (!CHECK || n < e.N)) ? e.bias[n] : 0.0f;
    }
    constexpr bool BWD = ACT >= CDX_EPI_BWD_RELU;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t m = m0 + blk_pos<VM>(i, 4 * lq + r);
            if (CHECK && m >= e.M) continue;
            const float brow = bias_row ? e.bias[m] : 0.0f;
            float* crow = e.C + m * e.ldc;
#pragma unroll
            for (int jn = 0; jn < FN; ++jn) {
                const int64_t n = n0 + blk_pos<VN>(jn, l16);
                if (CHECK && n >= e.N) continue;
                if (CHECK && e.colsum && n == e.n_main) {   // the ones column
                    e.colsum[m] = acc[i][jn][r];
                    continue;
                }
                if constexpr (BWD)
                    crow[col_off[jn]] = bwd_fixed<ACT>(acc[i][jn][r], e.aux[m * e.ldaux + n]);
                else
                    crow[col_off[jn]] = act_fixed<ACT>(acc[i][jn][r] + bcol[jn] + brow);
            }
        }
    }
}

template <int FM, int FN, bool CHECK, bool SPLITN, int VM = 1, int VN = 1>
__device__ __forceinline__ void write_acc(const floatx4 (&acc)[FM][FN], const EpiArgs& e,
                                          int64_t m0, int64_t n0, int lane) {
    if constexpr (!SPLITN) {   // backward epilogues: plain output map only
        switch (e.epilogue) {
            case CDX_EPI_BWD_RELU: write_acc_act<FM, FN, CHECK, false, CDX_EPI_BWD_RELU, VM, VN>(acc, e, m0, n0, lane); return;
            case CDX_EPI_BWD_GELU: write_acc_act<FM, FN, CHECK, false, CDX_EPI_BWD_GELU, VM, VN>(acc, e, m0, n0, lane); return;
            case CDX_EPI_BWD_SILU: write_acc_act<FM, FN, CHECK, false, CDX_EPI_BWD_SILU, VM, VN>(acc, e, m0, n0, lane); return;
            case CDX_EPI_BWD_SIGMOID: write_acc_act<FM, FN, CHECK, false, CDX_EPI_BWD_SIGMOID, VM, VN>(acc, e, m0, n0, lane); return;
            default: break;
        }
    }
    switch (e.epilogue) {
        case CDX_EPI_RELU: write_acc_act<FM, FN, CHECK, SPLITN, CDX_EPI_RELU, VM, VN>(acc, e, m0, n0, lane); break;
        case CDX_EPI_GELU: write_acc_act<FM, FN, CHECK, SPLITN, CDX_EPI_GELU, VM, VN>(acc, e, m0, n0, lane); break;
        case CDX_EPI_SILU: write_acc_act<FM, FN, CHECK, SPLITN, CDX_EPI_SILU, VM, VN>(acc, e, m0, n0, lane); break;
        case CDX_EPI_SIGMOID: write_acc_act<FM, FN, CHECK, SPLITN, CDX_EPI_SIGMOID, VM, VN>(acc, e, m0, n0, lane); break;
        default: write_acc_act<FM, FN, CHECK, SPLITN, CDX_EPI_NONE, VM, VN>(acc, e, m0, n0, lane); break;
    }
}

}  // namespace cdx
