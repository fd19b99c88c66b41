// extern "C" entry points of libcudeep_amd.so (declared in
// include/cudeep_amd.h).  This layer validates every argument on the host,
// turns problems into status codes with a per-thread message, and then
// calls the gfx950 launchers.  No exception crosses the boundary; nothing
// here falls back to the CPU.
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "cdx_internal.hpp"

namespace cdx {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_error(hipError_t e, const char* what) {
    if (e == hipSuccess) return CDX_OK;
    return set_error(CDX_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

namespace {

constexpr int kPoolDevices = 64;
std::mutex g_pool_mu;
hipMemPool_t g_pools[kPoolDevices] = {};

int scratch_pool(hipMemPool_t* out, const char* what) {
    int dev = -1;
    int st = hip_error(hipGetDevice(&dev), what);
    if (st) return st;
    if (dev < 0 || dev >= kPoolDevices)
        return set_error(CDX_ERR_UNSUPPORTED, std::string(what) + ": device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_pool_mu);
    if (!g_pools[dev]) {
        hipMemPoolProps props = {};
        props.allocType = hipMemAllocationTypePinned;
        props.handleTypes = hipMemHandleTypeNone;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = dev;
        hipMemPool_t pool = nullptr;
        st = hip_error(hipMemPoolCreate(&pool, &props), what);
        if (st) return st;
        uint64_t keep = UINT64_MAX;   // never hand freed blocks back on sync
        st = hip_error(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep), what);
        if (st) {
            (void)hipMemPoolDestroy(pool);
            return st;
        }
        g_pools[dev] = pool;
    }
    *out = g_pools[dev];
    return CDX_OK;
}

}  // namespace

int stream_alloc(void** p, size_t bytes, hipStream_t stream, const char* what) {
    hipMemPool_t pool = nullptr;
    int st = scratch_pool(&pool, what);
    if (st) return st;
    return hip_error(hipMallocFromPoolAsync(p, bytes, pool, stream), what);
}

int stream_free(void* p, hipStream_t stream, const char* what) {
    return hip_error(hipFreeAsync(p, stream), what);
}

}  // namespace cdx

using cdx::set_error;

namespace {

constexpr int64_t kMaxDim = (int64_t)1 << 40;

bool bad_dim(int64_t d) { return d < 0 || d > kMaxDim; }

// Validates a GEMM request; returns CDX_OK or an error code (with message).
int check_gemm(const char* fn, int opA, int opB, int64_t M, int64_t N, int64_t K,
               const void* A, int64_t lda, const void* B, int64_t ldb,
               const void* C, int64_t ldc) {
    if (opA != CDX_OP_N && opA != CDX_OP_T) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad opA");
    if (opB != CDX_OP_N && opB != CDX_OP_T) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad opB");
    if (bad_dim(M) || bad_dim(N) || bad_dim(K))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": dimensions must be in [0, 2^40]");
    if (M == 0 || N == 0) return CDX_OK;
    if (!C) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": C is NULL");
    if (K > 0 && (!A || !B)) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": A or B is NULL");
    const int64_t a_cols = opA == CDX_OP_N ? K : M;
    const int64_t b_cols = opB == CDX_OP_N ? N : K;
    if (lda < (a_cols > 1 ? a_cols : 1)) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": lda too small");
    if (ldb < (b_cols > 1 ? b_cols : 1)) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": ldb too small");
    if (ldc < N) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": ldc too small");
    return CDX_OK;
}

bool valid_precision(int p) {
    return p == CDX_PREC_FP32 || p == CDX_PREC_TF32MODE || p == CDX_PREC_TF32MODE4;
}

bool valid_epilogue(int e) { return e >= CDX_EPI_NONE && e <= CDX_EPI_SIGMOID; }

int run_gemm(int precision, cdx::GemmArgs g, hipStream_t stream) {
    if (g.M == 0 || g.N == 0) return CDX_OK;
    if (precision == CDX_PREC_FP32) return cdx::launch_gemm_f32(g, stream);
    if (precision == CDX_PREC_TF32MODE) return cdx::launch_gemm_bf16x3(g, 3, stream);
    if (precision == CDX_PREC_TF32MODE4) return cdx::launch_gemm_bf16x3(g, 4, stream);
    return set_error(CDX_ERR_INVALID_ARG, "gemm: unknown precision");
}

int64_t conv_out(int64_t in, int64_t k, int64_t s, int64_t p) { return (in + 2 * p - k) / s + 1; }

int check_conv(const char* fn, int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
               int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    if (bad_dim(batch) || bad_dim(IC) || bad_dim(OC) || bad_dim(IH) || bad_dim(IW) ||
        KH <= 0 || KW <= 0 || SH <= 0 || SW <= 0 || PH < 0 || PW < 0 ||
        KH > kMaxDim || KW > kMaxDim || SH > kMaxDim || SW > kMaxDim || PH > kMaxDim || PW > kMaxDim)
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": invalid geometry");
    if (IH + 2 * PH < KH || IW + 2 * PW < KW)
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": kernel larger than padded input");
    // every flat index must fit in int64 with room to spare
    const int64_t OH = conv_out(IH, KH, SH, PH), OW = conv_out(IW, KW, SW, PW);
    long double col = (long double)IC * KH * KW * batch * OH * OW;
    if (col > (long double)((int64_t)1 << 46))
        return set_error(CDX_ERR_UNSUPPORTED, std::string(fn) + ": problem too large");
    return CDX_OK;
}

// Bytes of the im2col column buffer [IC*KH*KW, B*OH*OW].
size_t col_bytes(int64_t batch, int64_t IC, int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                 int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    const int64_t OH = conv_out(IH, KH, SH, PH), OW = conv_out(IW, KW, SW, PW);
    return (size_t)(IC * KH * KW) * (size_t)(batch * OH * OW) * sizeof(float);
}

// Images per im2col + GEMM round of the column route: the whole batch while
// its column buffer stays within 128 MiB, else rounds below that (the last
// one takes the remainder).  A round's buffer, input and output then stay in
// the 256 MB Infinity Cache between the im2col write and the GEMM read (C5,
// 32 x 64 x 56^2 3x3, 231 MB of columns: 145 -> 139 us FP32 and 118 -> 106
// us in TF32 mode with two rounds of 16 images).  Among round sizes from the
// cap down to half of it, the one whose rounds need the fewest waves of GEMM
// tiles over the 256 CUs is taken, the largest on a tie; tiles are counted
// as the 64-column tiles of one 64-channel row (the output-channel-skinny
// GEMM's; the size query does not see the channel count).  C5's rounds of
// 16 run 784 tiles each, four waves where 3.06 are work, so 18 + 14 images
// (882 + 686 tiles: 4 + 3 waves against 4 + 4).  The sums are the same:
// every output column is one image's.
constexpr size_t kColRoundBytes = (size_t)128 << 20;

int64_t col_round_images(int64_t batch, size_t per_image_bytes, int64_t pixels) {
    const size_t total = per_image_bytes * (size_t)batch;
    if (per_image_bytes == 0 || total <= kColRoundBytes) return batch;
    const int64_t cap = std::max<int64_t>(1, (int64_t)(kColRoundBytes / per_image_bytes));
    auto waves = [&](int64_t nb) {
        return cdx::ceil_div(cdx::ceil_div(nb * pixels, (int64_t)64), (int64_t)256);
    };
    int64_t best = cap, best_cost = -1;
    for (int64_t r = cap; r >= std::max<int64_t>(1, cap / 2); --r) {
        const int64_t cost = (batch / r) * waves(r) + (batch % r ? waves(batch % r) : 0);
        if (best_cost < 0 || cost < best_cost) { best = r; best_cost = cost; }
    }
    return best;
}

// Workspace of the column route: one round's column buffer.
size_t col_round_bytes(int64_t batch, int64_t IC, int64_t IH, int64_t IW, int64_t KH,
                       int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    if (batch <= 0) return 0;
    const size_t per = col_bytes(1, IC, IH, IW, KH, KW, SH, SW, PH, PW);
    const int64_t S = conv_out(IH, KH, SH, PH) * conv_out(IW, KW, SW, PW);
    return per * (size_t)col_round_images(batch, per, S);
}

// The reference's forward dispatch (conv_kernel.cu:242-275) below its
// Winograd route: a layer whose column buffer would exceed 4 MiB runs the
// implicit GEMM (no buffer) unless it is a 3x3 stride-1 layer with >= 16
// output pixels per image (the Winograd shape, which keeps the im2col route
// here when it is not sent to Winograd).  The reference's naive-kernel
// shapes (K_col < 9 or fewer than 4 output pixels per image, checked before
// the implicit route at conv_kernel.cu:250) take the im2col route, which
// computes the same sums.
bool forward_takes_implicit(int64_t batch, int64_t IC, int64_t IH, int64_t IW, int64_t KH,
                            int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    const int64_t OH = conv_out(IH, KH, SH, PH), OW = conv_out(IW, KW, SW, PW);
    if (KH == 3 && KW == 3 && SH == 1 && SW == 1 && OH * OW >= 16) return false;
    if (IC * KH * KW < 9 || OH * OW < 4) return false;
    return col_bytes(batch, IC, IH, IW, KH, KW, SH, SW, PH, PW) > ((size_t)4 << 20) &&
           cdx::conv_fwd_implicit_ok(batch, IC, IH, IW, KH, KW, SH, SW, PH, PW);
}

}  // namespace

extern "C" {

const char* cdx_last_error(void) { return cdx::g_last_error.c_str(); }

const char* cdx_version(void) { return "cudeep_amd 0.1.0 (gfx950)"; }

int cdx_sgemm_f32(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                  hipStream_t stream) {
    int st = check_gemm("cdx_sgemm_f32", CDX_OP_N, CDX_OP_N, M, N, K, A, K > 1 ? K : 1, B,
                        N > 1 ? N : 1, C, N);
    if (st) return st;
    cdx::GemmArgs g{CDX_OP_N, CDX_OP_N, M, N, K, A, K, B, N, C, N, 0, 0,
                    nullptr, CDX_BIAS_NONE, CDX_EPI_NONE};
    return run_gemm(CDX_PREC_FP32, g, stream);
}

int cdx_gemm_tf32mode(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                      hipStream_t stream) {
    int st = check_gemm("cdx_gemm_tf32mode", CDX_OP_N, CDX_OP_N, M, N, K, A, K > 1 ? K : 1, B,
                        N > 1 ? N : 1, C, N);
    if (st) return st;
    cdx::GemmArgs g{CDX_OP_N, CDX_OP_N, M, N, K, A, K, B, N, C, N, 0, 0,
                    nullptr, CDX_BIAS_NONE, CDX_EPI_NONE};
    return run_gemm(CDX_PREC_TF32MODE, g, stream);
}

size_t cdx_gemm_workspace_size(int precision, int opA, int opB, int64_t M, int64_t N, int64_t K) {
    if (!valid_precision(precision) || (opA != CDX_OP_N && opA != CDX_OP_T) ||
        (opB != CDX_OP_N && opB != CDX_OP_T) || bad_dim(M) || bad_dim(N) || bad_dim(K)) {
        set_error(CDX_ERR_INVALID_ARG, "cdx_gemm_workspace_size: bad arguments");
        return 0;
    }
    if (M == 0 || N == 0) return 0;
    cdx::GemmArgs g{opA, opB, M, N, K, nullptr, 1, nullptr, 1, nullptr, N, 0, 0,
                    nullptr, CDX_BIAS_NONE, CDX_EPI_NONE};
    if (precision == CDX_PREC_FP32) return cdx::gemm_f32_workspace(g);
    return cdx::gemm_bf16x3_workspace(g, precision == CDX_PREC_TF32MODE4 ? 4 : 3);
}

int cdx_gemm_ex_ws(int precision, int opA, int opB, int64_t M, int64_t N, int64_t K,
                   const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                   int64_t ldc, const float* bias, int bias_mode, int epilogue, void* workspace,
                   size_t workspace_bytes, hipStream_t stream) {
    int st = check_gemm("cdx_gemm_ex", opA, opB, M, N, K, A, lda, B, ldb, C, ldc);
    if (st) return st;
    if (!valid_precision(precision))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_gemm_ex: bad precision");
    if (bias_mode != CDX_BIAS_NONE && bias_mode != CDX_BIAS_ROW && bias_mode != CDX_BIAS_COL)
        return set_error(CDX_ERR_INVALID_ARG, "cdx_gemm_ex: bad bias_mode");
    if (bias_mode != CDX_BIAS_NONE && !bias && M > 0 && N > 0)
        return set_error(CDX_ERR_INVALID_ARG, "cdx_gemm_ex: bias is NULL");
    if (!valid_epilogue(epilogue))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_gemm_ex: bad epilogue");
    cdx::GemmArgs g{opA, opB, M, N, K, A, lda, B, ldb, C, ldc, 0, 0, bias, bias_mode, epilogue};
    g.ws = workspace;
    g.ws_bytes = workspace ? workspace_bytes : 0;
    return run_gemm(precision, g, stream);
}

size_t cdx_gemm_fused_workspace_size(int precision, int opA, int opB, int64_t M, int64_t N,
                                     int64_t K, int with_colsum) {
    if (!with_colsum) return cdx_gemm_workspace_size(precision, opA, opB, M, N, K);
    if (!valid_precision(precision) || (opA != CDX_OP_N && opA != CDX_OP_T) ||
        (opB != CDX_OP_N && opB != CDX_OP_T) || bad_dim(M) || bad_dim(N) || bad_dim(K)) {
        set_error(CDX_ERR_INVALID_ARG, "cdx_gemm_fused_workspace_size: bad arguments");
        return 0;
    }
    if (M == 0) return 0;
    cdx::GemmArgs g{opA, opB, M, N, K, nullptr, 1, nullptr, 1, nullptr, N, 0, 0,
                    nullptr, CDX_BIAS_NONE, CDX_EPI_NONE};
    return cdx::gemm_f32_workspace(cdx::with_ones_column(g));   // FP32 kernel in every mode
}

int cdx_gemm_fused(int precision, int opA, int opB, int64_t M, int64_t N, int64_t K,
                   const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                   int64_t ldc, const float* bias, int bias_mode, int epilogue, const float* aux,
                   int64_t ldaux, float* colsum, void* workspace, size_t workspace_bytes,
                   hipStream_t stream) {
    const char* fn = "cdx_gemm_fused";
    int st = check_gemm(fn, opA, opB, M, N, K, A, lda, B, ldb, C, ldc);
    if (st) return st;
    if (!valid_precision(precision))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad precision");
    if (bias_mode != CDX_BIAS_NONE && bias_mode != CDX_BIAS_ROW && bias_mode != CDX_BIAS_COL)
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad bias_mode");
    if (bias_mode != CDX_BIAS_NONE && !bias && M > 0 && N > 0)
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bias is NULL");
    const bool bwd = epilogue >= CDX_EPI_BWD_RELU && epilogue <= CDX_EPI_BWD_SIGMOID;
    if (!valid_epilogue(epilogue) && !bwd)
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad epilogue");
    if (bwd) {
        if (bias_mode != CDX_BIAS_NONE)
            return set_error(CDX_ERR_INVALID_ARG,
                             std::string(fn) + ": no bias with an activation-backward epilogue");
        if (M > 0 && N > 0 && !aux)
            return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": aux is NULL");
        if (ldaux < N)
            return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": ldaux too small");
    } else if (aux) {
        return set_error(CDX_ERR_INVALID_ARG,
                         std::string(fn) + ": aux needs a CDX_EPI_BWD_* epilogue");
    }
    if (colsum && (bias_mode != CDX_BIAS_NONE || epilogue != CDX_EPI_NONE))
        return set_error(CDX_ERR_INVALID_ARG,
                         std::string(fn) + ": colsum needs bias_mode NONE and epilogue NONE");
    cdx::GemmArgs g{opA, opB, M, N, K, A, lda, B, ldb, C, ldc, 0, 0, bias, bias_mode, epilogue};
    g.ws = workspace;
    g.ws_bytes = workspace ? workspace_bytes : 0;
    g.aux = aux;
    g.ldaux = ldaux;
    if (colsum) {
        if (M == 0) return CDX_OK;
        g.colsum = colsum;
        return cdx::launch_gemm_f32(cdx::with_ones_column(g), stream);
    }
    return run_gemm(precision, g, stream);
}

int cdx_gemm_ex(int precision, int opA, int opB, int64_t M, int64_t N, int64_t K,
                const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc,
                const float* bias, int bias_mode, int epilogue, hipStream_t stream) {
    return cdx_gemm_ex_ws(precision, opA, opB, M, N, K, A, lda, B, ldb, C, ldc, bias, bias_mode,
                          epilogue, nullptr, 0, stream);
}

int cdx_gemm16_ex(int in_dtype, int opA, int opB, int64_t M, int64_t N, int64_t K,
                  const void* A, int64_t lda, const void* B, int64_t ldb, float* C, int64_t ldc,
                  const float* bias, int bias_mode, int epilogue, hipStream_t stream) {
    int st = check_gemm("cdx_gemm16_ex", opA, opB, M, N, K, A, lda, B, ldb, C, ldc);
    if (st) return st;
    if (in_dtype != CDX_DTYPE_F16 && in_dtype != CDX_DTYPE_BF16)
        return set_error(CDX_ERR_INVALID_ARG, "cdx_gemm16_ex: in_dtype must be F16 or BF16");
    if (bias_mode != CDX_BIAS_NONE && bias_mode != CDX_BIAS_ROW && bias_mode != CDX_BIAS_COL)
        return set_error(CDX_ERR_INVALID_ARG, "cdx_gemm16_ex: bad bias_mode");
    if (bias_mode != CDX_BIAS_NONE && !bias && M > 0 && N > 0)
        return set_error(CDX_ERR_INVALID_ARG, "cdx_gemm16_ex: bias is NULL");
    if (!valid_epilogue(epilogue))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_gemm16_ex: bad epilogue");
    if (M == 0 || N == 0) return CDX_OK;
    cdx::GemmArgs g{opA, opB, M, N, K, A, lda, B, ldb, C, ldc, 0, 0, bias, bias_mode, epilogue};
    return cdx::launch_gemm_16(g, in_dtype, stream);
}

int cdx_hgemm_f16(const void* A, const void* B, float* C, int64_t M, int64_t N, int64_t K,
                  hipStream_t stream) {
    return cdx_gemm16_ex(CDX_DTYPE_F16, CDX_OP_N, CDX_OP_N, M, N, K, A, K > 1 ? K : 1, B,
                         N > 1 ? N : 1, C, N, nullptr, CDX_BIAS_NONE, CDX_EPI_NONE, stream);
}

int cdx_matmul_fused_act(const float* A, const float* B, float* C, int64_t M, int64_t N,
                         int64_t K, int epilogue, hipStream_t stream) {
    return cdx_gemm_ex(CDX_PREC_TF32MODE, CDX_OP_N, CDX_OP_N, M, N, K, A, K > 1 ? K : 1, B,
                       N > 1 ? N : 1, C, N, nullptr, CDX_BIAS_NONE, epilogue, stream);
}

int cdx_dgemm(int opA, int opB, int64_t M, int64_t N, int64_t K, const double* A, int64_t lda,
              const double* B, int64_t ldb, double* C, int64_t ldc, hipStream_t stream) {
    int st = check_gemm("cdx_dgemm", opA, opB, M, N, K, A, lda, B, ldb, C, ldc);
    if (st) return st;
    if (M == 0 || N == 0) return CDX_OK;
    return cdx::launch_dgemm(opA, opB, M, N, K, A, lda, B, ldb, C, ldc, stream);
}

int cdx_im2col_f32(const float* input, float* col, int64_t batch, int64_t in_channels,
                   int64_t in_h, int64_t in_w, int64_t kernel_h, int64_t kernel_w,
                   int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                   hipStream_t stream) {
    int st = check_conv("cdx_im2col_f32", batch, in_channels, 1, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    if (batch * in_channels == 0) return CDX_OK;
    if (!input || !col) return set_error(CDX_ERR_INVALID_ARG, "cdx_im2col_f32: NULL pointer");
    return cdx::launch_im2col_f32(input, col, batch, in_channels, in_h, in_w, kernel_h, kernel_w,
                                  stride_h, stride_w, pad_h, pad_w, stream);
}

size_t cdx_conv2d_forward_workspace_size(int64_t batch, int64_t in_channels, int64_t in_h,
                                         int64_t in_w, int64_t kernel_h, int64_t kernel_w,
                                         int64_t stride_h, int64_t stride_w, int64_t pad_h,
                                         int64_t pad_w) {
    if (check_conv("cdx_conv2d_forward_workspace_size", batch, in_channels, 1, in_h, in_w,
                   kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w))
        return 0;
    if (forward_takes_implicit(batch, in_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                               stride_w, pad_h, pad_w))
        return 0;
    return col_round_bytes(batch, in_channels, in_h, in_w, kernel_h, kernel_w, stride_h, stride_w,
                     pad_h, pad_w);
}

int cdx_conv2d_forward_implicit_f32(const float* input, const float* weight, const float* bias,
                                    float* output, int64_t batch, int64_t in_channels,
                                    int64_t out_channels, int64_t in_h, int64_t in_w,
                                    int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                                    int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                    hipStream_t stream) {
    const char* fn = "cdx_conv2d_forward_implicit_f32";
    int st = check_conv(fn, batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    const int64_t OH = conv_out(in_h, kernel_h, stride_h, pad_h);
    const int64_t OW = conv_out(in_w, kernel_w, stride_w, pad_w);
    if (batch == 0 || out_channels == 0 || OH * OW == 0) return CDX_OK;
    if (!output || !weight || !input)
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    if (!cdx::conv_fwd_implicit_ok(batch, in_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                                   stride_w, pad_h, pad_w))
        return set_error(CDX_ERR_UNSUPPORTED, std::string(fn) + ": geometry beyond 32-bit indices");
    return cdx::launch_conv_fwd_implicit_f32(input, weight, bias, output, batch, in_channels,
                                             out_channels, in_h, in_w, kernel_h, kernel_w,
                                             stride_h, stride_w, pad_h, pad_w, stream);
}

}  // extern "C"

namespace {

// im2col + one GEMM into NCHW per round of images (col_round_images);
// blocked_sum asks the FP32 GEMM for its two-level k sum (see GemmArgs).
int conv_forward_im2col(const float* input, const float* weight, const float* bias,
                        float* output, int64_t batch, int64_t in_channels,
                        int64_t out_channels, int64_t in_h, int64_t in_w, int64_t kernel_h,
                        int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                        int64_t pad_w, int precision, void* workspace,
                        size_t workspace_bytes, hipStream_t stream, bool blocked_sum) {
    int st = check_conv("cdx_conv2d_forward_f32", batch, in_channels, out_channels, in_h, in_w,
                        kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    if (!valid_precision(precision))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_conv2d_forward_f32: bad precision");
    const int64_t OH = conv_out(in_h, kernel_h, stride_h, pad_h);
    const int64_t OW = conv_out(in_w, kernel_w, stride_w, pad_w);
    const int64_t S = OH * OW, Kc = in_channels * kernel_h * kernel_w;
    if (batch == 0 || out_channels == 0 || S == 0) return CDX_OK;
    if (!output || !weight || (Kc > 0 && !input))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_conv2d_forward_f32: NULL pointer");
    const size_t per_image = (size_t)Kc * (size_t)S * sizeof(float);
    const int64_t round = col_round_images(batch, per_image, S);
    const size_t need = per_image * (size_t)round;
    float* col = static_cast<float*>(workspace);
    bool owned = false;
    if (workspace) {
        if (workspace_bytes < need)
            return set_error(CDX_ERR_WORKSPACE, "cdx_conv2d_forward_f32: workspace too small");
    } else if (need > 0) {
        st = cdx::stream_alloc(reinterpret_cast<void**>(&col), need, stream,
                               "cdx_conv2d_forward_f32: scratch");
        if (st) return st;
        owned = true;
    }
    for (int64_t b0 = 0; b0 < batch && !st; b0 += round) {
        const int64_t nb = batch - b0 < round ? batch - b0 : round, ns = nb * S;
        if (Kc > 0) {
            st = cdx::launch_im2col_f32(input + b0 * in_channels * in_h * in_w, col, nb,
                                        in_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                                        stride_w, pad_h, pad_w, stream);
        }
        if (!st) {
            // weight[OC, Kc] * col[Kc, nb*S] -> NCHW: addr = oc*S + (n/S)*OC*S + n%S
            cdx::GemmArgs g{CDX_OP_N, CDX_OP_N, out_channels, ns, Kc, weight, Kc > 0 ? Kc : 1,
                            col, ns, output + b0 * out_channels * S, S, S, out_channels * S,
                            bias, bias ? CDX_BIAS_ROW : CDX_BIAS_NONE, CDX_EPI_NONE};
            g.blocked_sum = blocked_sum;
            st = run_gemm(precision, g, stream);
        }
    }
    if (owned) {
        int st2 = cdx::stream_free(col, stream, "cdx_conv2d_forward_f32: scratch");
        if (!st) st = st2;
    }
    return st;
}

}  // namespace

extern "C" {

int cdx_conv2d_forward_f32(const float* input, const float* weight, const float* bias,
                           float* output, int64_t batch, int64_t in_channels,
                           int64_t out_channels, int64_t in_h, int64_t in_w, int64_t kernel_h,
                           int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                           int64_t pad_w, int precision, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
    if (!check_conv("cdx_conv2d_forward_f32", batch, in_channels, out_channels, in_h, in_w,
                    kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w) &&
        forward_takes_implicit(batch, in_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                               stride_w, pad_h, pad_w)) {
        if (!valid_precision(precision))
            return set_error(CDX_ERR_INVALID_ARG, "cdx_conv2d_forward_f32: bad precision");
        return cdx_conv2d_forward_implicit_f32(input, weight, bias, output, batch, in_channels,
                                               out_channels, in_h, in_w, kernel_h, kernel_w,
                                               stride_h, stride_w, pad_h, pad_w, stream);
    }
    return conv_forward_im2col(input, weight, bias, output, batch, in_channels, out_channels,
                               in_h, in_w, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w,
                               precision, workspace, workspace_bytes, stream, false);
}

size_t cdx_conv2d_winograd_workspace_size(int64_t batch, int64_t in_channels,
                                          int64_t out_channels, int64_t in_h, int64_t in_w,
                                          int64_t pad_h, int64_t pad_w) {
    if (check_conv("cdx_conv2d_winograd_workspace_size", batch, in_channels, out_channels, in_h,
                   in_w, 3, 3, 1, 1, pad_h, pad_w))
        return 0;
    return cdx::winograd_workspace_floats(batch, in_channels, out_channels, in_h + 2 * pad_h - 2,
                                          in_w + 2 * pad_w - 2) * sizeof(float);
}

int cdx_conv2d_forward_winograd_f32(const float* input, const float* weight, const float* bias,
                                    float* output, int64_t batch, int64_t in_channels,
                                    int64_t out_channels, int64_t in_h, int64_t in_w,
                                    int64_t pad_h, int64_t pad_w, int precision, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
    const char* fn = "cdx_conv2d_forward_winograd_f32";
    int st = check_conv(fn, batch, in_channels, out_channels, in_h, in_w, 3, 3, 1, 1, pad_h, pad_w);
    if (st) return st;
    if (!valid_precision(precision)) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad precision");
    const int64_t OH = in_h + 2 * pad_h - 2, OW = in_w + 2 * pad_w - 2;
    if (batch == 0 || out_channels == 0 || OH * OW == 0) return CDX_OK;
    if (!output || !weight || (in_channels > 0 && !input))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    if (in_channels == 0) {   // empty sum: the output is the bias
        return cdx_conv2d_forward_f32(input, weight, bias, output, batch, 0, out_channels, in_h,
                                      in_w, 3, 3, 1, 1, pad_h, pad_w, precision, nullptr, 0, stream);
    }
    const size_t need =
        cdx::winograd_workspace_floats(batch, in_channels, out_channels, OH, OW) * sizeof(float);
    float* ws = static_cast<float*>(workspace);
    bool owned = false;
    if (workspace) {
        if (workspace_bytes < need)
            return set_error(CDX_ERR_WORKSPACE, std::string(fn) + ": workspace too small");
    } else {
        st = cdx::stream_alloc(reinterpret_cast<void**>(&ws), need, stream,
                               "cdx_conv2d_forward_winograd_f32: scratch");
        if (st) return st;
        owned = true;
    }
    st = cdx::launch_conv2d_winograd_f32(input, weight, bias, output, batch, in_channels,
                                         out_channels, in_h, in_w, pad_h, pad_w, precision, ws,
                                         stream);
    if (owned) {
        int st2 = cdx::stream_free(ws, stream, "cdx_conv2d_forward_winograd_f32: scratch");
        if (!st) st = st2;
    }
    return st;
}

int cdx_col2im_f32(const float* col, float* grad_input, int64_t batch, int64_t in_channels,
                   int64_t in_h, int64_t in_w, int64_t kernel_h, int64_t kernel_w,
                   int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                   hipStream_t stream) {
    int st = check_conv("cdx_col2im_f32", batch, in_channels, 1, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    if (batch * in_channels * in_h * in_w == 0) return CDX_OK;
    if (!col || !grad_input) return set_error(CDX_ERR_INVALID_ARG, "cdx_col2im_f32: NULL pointer");
    return cdx::launch_col2im_f32(col, grad_input, batch, in_channels, in_h, in_w, kernel_h,
                                  kernel_w, stride_h, stride_w, pad_h, pad_w, stream);
}

}  // extern "C"

// ---- scratch of the allocation-free entry point ----------------------------
// cdx_conv2d_backward_weight_f32_noalloc keeps its split partials here: one
// copy of the array on every GPU the library runs on, held until the process
// ends.  On the host the array's name is only a stand-in for the device
// symbol, never an address: host code uses the device address that
// hipGetSymbolAddress returns, looked up once per device.
static __device__ __align__(256) unsigned char scratch[CDX_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};   // device address of `scratch`, per device

// The current device's copy of `scratch` (resolved on the first call on that
// device, with the device current).
int noalloc_scratch(void** out, const char* fn) {
    int dev = -1;
    int st = cdx::hip_error(hipGetDevice(&dev), fn);
    if (st) return st;
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(CDX_ERR_UNSUPPORTED, std::string(fn) + ": device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        st = cdx::hip_error(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), fn);
        if (st) return st;
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return CDX_OK;
}

}  // namespace

extern "C" {

namespace {

struct ConvSizes {
    int64_t OH, OW, S, BS, Kc;
};

ConvSizes conv_sizes(int64_t batch, int64_t IC, int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                     int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    ConvSizes z;
    z.OH = conv_out(IH, KH, SH, PH);
    z.OW = conv_out(IW, KW, SW, PW);
    z.S = z.OH * z.OW;
    z.BS = batch * z.S;
    z.Kc = IC * KH * KW;
    return z;
}

// Stride-1 backward data is the forward convolution of grad_output with the
// filter channel-swapped and spatially reversed, padded KH-1-PH / KW-1-PW:
//   dX[b,ic,ih,iw] = sum_{oc,kh,kw} dY[b,oc,ih+PH-kh,iw+PW-kw] W[oc,ic,kh,kw]
// and with kh' = KH-1-kh the dY row is ih + kh' - (KH-1-PH).  Needs that
// padding to be >= 0 (and OC > 0: an empty sum takes the GEMM route, which
// writes zeros).
bool bwd_data_as_forward(int64_t OC, int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                         int64_t PW) {
    return OC > 0 && SH == 1 && SW == 1 && PH <= KH - 1 && PW <= KW - 1;
}

// Stride-1 backward data as the row-window implicit conv of grad_out with the
// flipped filter (no column buffer), where that kernel's window fits.
bool bwd_data_rowwin(int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH,
                     int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    if (!bwd_data_as_forward(OC, KH, KW, SH, SW, PH, PW)) return false;
    const int64_t OH = conv_out(IH, KH, SH, PH), OW = conv_out(IW, KW, SW, PW);
    return cdx::conv_rowwin_ok(batch, OC, IC, OH, OW, KH, KW, 1, 1, KH - 1 - PH, KW - 1 - PW);
}

// Workspace of the implicit backward-weight kernel (0 when it does not apply).
size_t wgrad_implicit_floats(int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                             int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                             int64_t PW) {
    if (!cdx::conv_wgrad_implicit_ok(batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW)) return 0;
    return cdx::conv_wgrad_implicit_floats(batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW);
}

// Stream-ordered scratch: the caller's workspace, or a hipMallocAsync block
// freed on the same stream when the call ends.
struct Scratch {
    void* ptr = nullptr;
    bool owned = false;
    hipStream_t stream = nullptr;
    int acquire(void* ws, size_t ws_bytes, size_t need, hipStream_t s, const char* fn) {
        stream = s;
        if (ws) {
            if (ws_bytes < need) return set_error(CDX_ERR_WORKSPACE, std::string(fn) + ": workspace too small");
            ptr = ws;
            return CDX_OK;
        }
        if (need == 0) return CDX_OK;
        int st = cdx::stream_alloc(&ptr, need, s, fn);
        owned = st == CDX_OK;
        return st;
    }
    int release(int st) {
        if (owned) {
            int st2 = cdx::stream_free(ptr, stream, "scratch free");
            owned = false;
            if (!st) st = st2;
        }
        return st;
    }
};

// Scratch of the backward-weight GEMM route (problems beyond the implicit
// kernel's index range): col [Kc, BS], (batch > 1) grad_out as [OC, BS], then
// the split-K partials of the [OC, Kc] x BS product (the largest any
// precision's launch takes), 256-byte aligned.
struct WgradGemmBytes {
    size_t gemm_off, gemm, total;
};

WgradGemmBytes wgrad_gemm_route_bytes(int64_t batch, int64_t out_channels, const ConvSizes& z) {
    const size_t n = (size_t)z.Kc * z.BS + (batch > 1 ? (size_t)out_channels * z.BS : 0);
    cdx::GemmArgs g{CDX_OP_N, CDX_OP_T, out_channels, z.Kc, z.BS, nullptr, 1, nullptr, 1,
                    nullptr, z.Kc, 0, 0, nullptr, CDX_BIAS_NONE, CDX_EPI_NONE};
    size_t gemm = 0;
    if (out_channels * z.Kc > 0) {
        gemm = cdx::gemm_f32_workspace(g);
        for (int terms = 3; terms <= 4; ++terms) {
            const size_t t = cdx::gemm_bf16x3_workspace(g, terms);
            if (t > gemm) gemm = t;
        }
    }
    const size_t off = (n * sizeof(float) + 255) / 256 * 256;
    return {off, gemm, gemm > 0 ? off + gemm : n * sizeof(float)};
}

}  // namespace

size_t cdx_conv2d_backward_data_workspace_size(int64_t batch, int64_t in_channels,
                                               int64_t out_channels, int64_t in_h, int64_t in_w,
                                               int64_t kernel_h, int64_t kernel_w,
                                               int64_t stride_h, int64_t stride_w,
                                               int64_t pad_h, int64_t pad_w) {
    if (check_conv("cdx_conv2d_backward_data_workspace_size", batch, in_channels, out_channels,
                   in_h, in_w, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w))
        return 0;
    ConvSizes z = conv_sizes(batch, in_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                             stride_w, pad_h, pad_w);
    if (bwd_data_rowwin(batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w))   // flipped filter only
        return (size_t)in_channels * out_channels * (size_t)(kernel_h * kernel_w) * sizeof(float);
    if (bwd_data_as_forward(out_channels, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w)) {
        // flipped filter [IC, OC, KH, KW] + one round's im2col of grad_out
        // [OC*KH*KW, nb*IH*IW] (the forward column route on the transposed conv)
        const size_t khw = (size_t)(kernel_h * kernel_w);
        return (size_t)in_channels * out_channels * khw * sizeof(float) +
               col_round_bytes(batch, out_channels, z.OH, z.OW, kernel_h, kernel_w, 1, 1,
                               kernel_h - 1 - pad_h, kernel_w - 1 - pad_w);
    }
    // grad_col [Kc, BS] + (batch > 1) grad_out in [OC, BS]
    size_t n = (size_t)z.Kc * z.BS + (batch > 1 ? (size_t)out_channels * z.BS : 0);
    return n * sizeof(float);
}

int cdx_conv2d_backward_data_f32(const float* grad_output, const float* weight, float* grad_input,
                                 int64_t batch, int64_t in_channels, int64_t out_channels,
                                 int64_t in_h, int64_t in_w, int64_t kernel_h, int64_t kernel_w,
                                 int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                 int precision, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
    const char* fn = "cdx_conv2d_backward_data_f32";
    int st = check_conv(fn, batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    if (!valid_precision(precision))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad precision");
    if (batch * in_channels * in_h * in_w == 0) return CDX_OK;
    if (!grad_input || (out_channels > 0 && (!grad_output || !weight)))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    ConvSizes z = conv_sizes(batch, in_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                             stride_w, pad_h, pad_w);
    const size_t need = cdx_conv2d_backward_data_workspace_size(
        batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w, stride_h, stride_w,
        pad_h, pad_w);
    Scratch ws;
    st = ws.acquire(workspace, workspace_bytes, need, stream, fn);
    if (st) return st;
    if (bwd_data_rowwin(batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w)) {
        // stride 1: grad_input = conv(grad_out, flipped filter, padding KH-1-PH, KW-1-PW)
        // through the row-window implicit kernel (FP32 products in every
        // precision mode, k summed in two levels: the reference sums OC
        // products per grad_col entry, then KH*KW entries in col2im, and one
        // K = OC*KH*KW running sum would be a ~KH*KW times longer rounding
        // chain)
        float* wf = static_cast<float*>(ws.ptr);
        st = cdx::launch_flip_filter_f32(weight, wf, out_channels, in_channels,
                                         kernel_h * kernel_w, stream);
        if (!st)
            st = cdx::launch_conv_rowwin_f32(grad_output, wf, nullptr, grad_input, batch,
                                             out_channels, in_channels, z.OH, z.OW, kernel_h,
                                             kernel_w, 1, 1, kernel_h - 1 - pad_h,
                                             kernel_w - 1 - pad_w, true, stream);
        return ws.release(st);
    }
    if (bwd_data_as_forward(out_channels, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w)) {
        // stride 1: grad_input = conv(grad_out, flipped filter, padding KH-1-PH, KW-1-PW),
        // one im2col + one long-K GEMM straight into NCHW (no grad_col, no col2im)
        float* wf = static_cast<float*>(ws.ptr);
        const int64_t khw = kernel_h * kernel_w;
        float* col = wf + in_channels * out_channels * khw;
        st = cdx::launch_flip_filter_f32(weight, wf, out_channels, in_channels, khw, stream);
        // The reference sums OC products per grad_col entry, then KH*KW entries
        // in col2im; one K = OC*KH*KW running sum would be a ~KH*KW times
        // longer rounding chain, so FP32 takes the GEMM's two-level sum.
        if (!st)
            st = conv_forward_im2col(grad_output, wf, nullptr, grad_input, batch, out_channels,
                                     in_channels, z.OH, z.OW, kernel_h, kernel_w, 1, 1,
                                     kernel_h - 1 - pad_h, kernel_w - 1 - pad_w, precision, col,
                                     need - (size_t)in_channels * out_channels * khw * sizeof(float),
                                     stream, true);
        return ws.release(st);
    }
    float* grad_col = static_cast<float*>(ws.ptr);
    const float* dy_cm = grad_output;                   // batch 1: NCHW is [OC, S] already
    if (batch > 1) {
        float* t = grad_col + (size_t)z.Kc * z.BS;
        st = cdx::launch_nchw_to_cm_f32(grad_output, t, batch, out_channels, z.S, stream);
        dy_cm = t;
    }
    if (!st) {
        // grad_col[Kc, BS] = weight^T [Kc, OC] * dy_cm [OC, BS]
        cdx::GemmArgs g{CDX_OP_T, CDX_OP_N, z.Kc, z.BS, out_channels, weight, z.Kc,
                        dy_cm, z.BS, grad_col, z.BS, 0, 0, nullptr, CDX_BIAS_NONE, CDX_EPI_NONE};
        st = run_gemm(precision, g, stream);
    }
    if (!st)
        st = cdx::launch_col2im_f32(grad_col, grad_input, batch, in_channels, in_h, in_w,
                                    kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w, stream);
    return ws.release(st);
}

size_t cdx_conv2d_backward_data_winograd_workspace_size(int64_t batch, int64_t in_channels,
                                                        int64_t out_channels, int64_t in_h,
                                                        int64_t in_w, int64_t pad_h,
                                                        int64_t pad_w) {
    const char* fn = "cdx_conv2d_backward_data_winograd_workspace_size";
    if (check_conv(fn, batch, in_channels, out_channels, in_h, in_w, 3, 3, 1, 1, pad_h, pad_w))
        return 0;
    if (pad_h > 2 || pad_w > 2) {
        set_error(CDX_ERR_UNSUPPORTED, std::string(fn) + ": padding above 2");
        return 0;
    }
    // the transposed problem: OC input channels -> IC output channels, IH x IW out
    return cdx::winograd_workspace_floats(batch, out_channels, in_channels, in_h, in_w) *
           sizeof(float);
}

int cdx_conv2d_backward_data_winograd_f32(const float* grad_output, const float* weight,
                                          float* grad_input, int64_t batch, int64_t in_channels,
                                          int64_t out_channels, int64_t in_h, int64_t in_w,
                                          int64_t pad_h, int64_t pad_w, int precision,
                                          void* workspace, size_t workspace_bytes,
                                          hipStream_t stream) {
    const char* fn = "cdx_conv2d_backward_data_winograd_f32";
    int st = check_conv(fn, batch, in_channels, out_channels, in_h, in_w, 3, 3, 1, 1, pad_h, pad_w);
    if (st) return st;
    if (pad_h > 2 || pad_w > 2)
        return set_error(CDX_ERR_UNSUPPORTED, std::string(fn) + ": padding above 2");
    if (!valid_precision(precision))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad precision");
    if (batch * in_channels * in_h * in_w == 0) return CDX_OK;
    if (!grad_input || (out_channels > 0 && (!grad_output || !weight)))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    if (out_channels == 0)   // empty sum: zeros, through the GEMM route
        return cdx_conv2d_backward_data_f32(grad_output, weight, grad_input, batch, in_channels,
                                            0, in_h, in_w, 3, 3, 1, 1, pad_h, pad_w, precision,
                                            nullptr, 0, stream);
    const int64_t OH = in_h + 2 * pad_h - 2, OW = in_w + 2 * pad_w - 2;
    const size_t need =
        cdx::winograd_workspace_floats(batch, out_channels, in_channels, in_h, in_w) * sizeof(float);
    Scratch ws;
    st = ws.acquire(workspace, workspace_bytes, need, stream, fn);
    if (st) return st;
    st = cdx::launch_conv2d_winograd_f32(grad_output, weight, nullptr, grad_input, batch,
                                         out_channels, in_channels, OH, OW, 2 - pad_h, 2 - pad_w,
                                         precision, static_cast<float*>(ws.ptr), stream,
                                         /*flip_filter=*/true);
    return ws.release(st);
}

size_t cdx_conv2d_backward_weight_workspace_size(int64_t batch, int64_t in_channels,
                                                 int64_t out_channels, int64_t in_h, int64_t in_w,
                                                 int64_t kernel_h, int64_t kernel_w,
                                                 int64_t stride_h, int64_t stride_w,
                                                 int64_t pad_h, int64_t pad_w) {
    if (check_conv("cdx_conv2d_backward_weight_workspace_size", batch, in_channels, out_channels,
                   in_h, in_w, kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w))
        return 0;
    ConvSizes z = conv_sizes(batch, in_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                             stride_w, pad_h, pad_w);
    // exactly what the route the launch takes uses
    if (z.BS > 0 && cdx::conv_wgrad_implicit_ok(batch, in_channels, out_channels, in_h, in_w,
                                                kernel_h, kernel_w, stride_h, stride_w, pad_h,
                                                pad_w))
        return wgrad_implicit_floats(batch, in_channels, out_channels, in_h, in_w, kernel_h,
                                     kernel_w, stride_h, stride_w, pad_h, pad_w) * sizeof(float);
    return wgrad_gemm_route_bytes(batch, out_channels, z).total;
}

int cdx_conv2d_backward_weight_f32(const float* grad_output, const float* input,
                                   float* grad_weight, int64_t batch, int64_t in_channels,
                                   int64_t out_channels, int64_t in_h, int64_t in_w,
                                   int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                                   int64_t stride_w, int64_t pad_h, int64_t pad_w, int precision,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const char* fn = "cdx_conv2d_backward_weight_f32";
    int st = check_conv(fn, batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    if (!valid_precision(precision))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad precision");
    ConvSizes z = conv_sizes(batch, in_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                             stride_w, pad_h, pad_w);
    if (out_channels * z.Kc == 0) return CDX_OK;
    if (!grad_weight || (z.BS > 0 && (!grad_output || !input)))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    const size_t need = cdx_conv2d_backward_weight_workspace_size(
        batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w, stride_h, stride_w,
        pad_h, pad_w);
    if (z.BS > 0 && cdx::conv_wgrad_implicit_ok(batch, in_channels, out_channels, in_h, in_w,
                                                kernel_h, kernel_w, stride_h, stride_w, pad_h,
                                                pad_w)) {
        // implicit GEMM from the NCHW tensors (no col buffer).  Its FP32 MFMA
        // products are also what the TF32 modes get: exact products, faster
        // here than im2col + the split-bf16 GEMM, within both error bounds.
        Scratch ws;
        st = ws.acquire(workspace, workspace_bytes,
                        wgrad_implicit_floats(batch, in_channels, out_channels, in_h, in_w,
                                              kernel_h, kernel_w, stride_h, stride_w, pad_h,
                                              pad_w) * sizeof(float),
                        stream, fn);
        if (st) return st;
        st = cdx::launch_conv_wgrad_f32(grad_output, input, grad_weight,
                                        static_cast<float*>(ws.ptr), batch, in_channels,
                                        out_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                                        stride_w, pad_h, pad_w, stream);
        return ws.release(st);
    }
    const WgradGemmBytes wb = wgrad_gemm_route_bytes(batch, out_channels, z);
    Scratch ws;
    st = ws.acquire(workspace, workspace_bytes, need, stream, fn);
    if (st) return st;
    float* col = static_cast<float*>(ws.ptr);
    const float* dy_cm = grad_output;
    if (z.BS > 0)
        st = cdx::launch_im2col_f32(input, col, batch, in_channels, in_h, in_w, kernel_h,
                                    kernel_w, stride_h, stride_w, pad_h, pad_w, stream);
    if (!st && batch > 1) {
        float* t = col + (size_t)z.Kc * z.BS;
        st = cdx::launch_nchw_to_cm_f32(grad_output, t, batch, out_channels, z.S, stream);
        dy_cm = t;
    }
    if (!st) {
        // grad_weight[OC, Kc] = dy_cm [OC, BS] * col^T [BS, Kc]
        cdx::GemmArgs g{CDX_OP_N, CDX_OP_T, out_channels, z.Kc, z.BS, dy_cm, z.BS > 0 ? z.BS : 1,
                        col, z.BS > 0 ? z.BS : 1, grad_weight, z.Kc, 0, 0, nullptr,
                        CDX_BIAS_NONE, CDX_EPI_NONE};
        if (wb.gemm > 0) {   // split-K partials from the same workspace
            g.ws = static_cast<char*>(ws.ptr) + wb.gemm_off;
            g.ws_bytes = wb.gemm;
        }
        st = run_gemm(precision, g, stream);
    }
    return ws.release(st);
}

int cdx_conv2d_backward_weight_f32_noalloc(const float* grad_output, const float* input,
                                           float* grad_weight, int64_t batch,
                                           int64_t in_channels, int64_t out_channels,
                                           int64_t in_h, int64_t in_w, int64_t kernel_h,
                                           int64_t kernel_w, int64_t stride_h, int64_t stride_w,
                                           int64_t pad_h, int64_t pad_w, int precision,
                                           hipStream_t stream) {
    const char* fn = "cdx_conv2d_backward_weight_f32_noalloc";
    int st = check_conv(fn, batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    if (!valid_precision(precision))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad precision");
    const size_t need = cdx_conv2d_backward_weight_workspace_size(
        batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w, stride_h, stride_w,
        pad_h, pad_w);
    if (need > (size_t)CDX_NOALLOC_SCRATCH_BYTES)
        return set_error(CDX_ERR_UNSUPPORTED,
                         std::string(fn) + ": this layer needs " + std::to_string(need) +
                             " bytes of scratch, more than the " +
                             std::to_string((size_t)CDX_NOALLOC_SCRATCH_BYTES) +
                             " the allocation-free entry point holds; call "
                             "cdx_conv2d_backward_weight_f32 with a workspace instead");
    void* ws = nullptr;
    st = noalloc_scratch(&ws, fn);
    if (st) return st;
    // with a workspace the general entry point allocates nothing
    return cdx_conv2d_backward_weight_f32(grad_output, input, grad_weight, batch, in_channels,
                                          out_channels, in_h, in_w, kernel_h, kernel_w,
                                          stride_h, stride_w, pad_h, pad_w, precision, ws,
                                          (size_t)CDX_NOALLOC_SCRATCH_BYTES, stream);
}

int cdx_conv2d_backward_bias_f32(const float* grad_output, float* grad_bias, int64_t batch,
                                 int64_t out_channels, int64_t spatial, hipStream_t stream) {
    if (bad_dim(batch) || bad_dim(out_channels) || bad_dim(spatial))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_conv2d_backward_bias_f32: bad dims");
    if (out_channels == 0) return CDX_OK;
    if (!grad_bias || (batch * spatial > 0 && !grad_output))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_conv2d_backward_bias_f32: NULL pointer");
    return cdx::launch_conv_bias_grad_f32(grad_output, grad_bias, batch, out_channels, spatial,
                                          stream);
}

int cdx_conv2d_forward_f64(const double* input, const double* weight, const double* bias,
                           double* output, int64_t batch, int64_t in_channels,
                           int64_t out_channels, int64_t in_h, int64_t in_w,
                           int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                           int64_t stride_w, int64_t pad_h, int64_t pad_w, hipStream_t stream) {
    const char* fn = "cdx_conv2d_forward_f64";
    int st = check_conv(fn, batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    const int64_t OH = conv_out(in_h, kernel_h, stride_h, pad_h);
    const int64_t OW = conv_out(in_w, kernel_w, stride_w, pad_w);
    if (batch * out_channels * OH * OW == 0) return CDX_OK;
    if (!output || !weight || (in_channels > 0 && !input))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    return cdx::launch_conv2d_forward_f64(input, weight, bias, output, batch, in_channels,
                                          out_channels, in_h, in_w, kernel_h, kernel_w, stride_h,
                                          stride_w, pad_h, pad_w, stream);
}

int cdx_conv2d_backward_data_f64(const double* grad_output, const double* weight,
                                 double* grad_input, int64_t batch, int64_t in_channels,
                                 int64_t out_channels, int64_t in_h, int64_t in_w,
                                 int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                                 int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                 hipStream_t stream) {
    const char* fn = "cdx_conv2d_backward_data_f64";
    int st = check_conv(fn, batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    if (batch * in_channels * in_h * in_w == 0) return CDX_OK;
    if (!grad_input || (out_channels > 0 && (!grad_output || !weight)))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    return cdx::launch_conv2d_backward_data_f64(grad_output, weight, grad_input, batch,
                                                in_channels, out_channels, in_h, in_w, kernel_h,
                                                kernel_w, stride_h, stride_w, pad_h, pad_w,
                                                stream);
}

int cdx_conv2d_backward_weight_f64(const double* grad_output, const double* input,
                                   double* grad_weight, int64_t batch, int64_t in_channels,
                                   int64_t out_channels, int64_t in_h, int64_t in_w,
                                   int64_t kernel_h, int64_t kernel_w, int64_t stride_h,
                                   int64_t stride_w, int64_t pad_h, int64_t pad_w,
                                   hipStream_t stream) {
    const char* fn = "cdx_conv2d_backward_weight_f64";
    int st = check_conv(fn, batch, in_channels, out_channels, in_h, in_w, kernel_h, kernel_w,
                        stride_h, stride_w, pad_h, pad_w);
    if (st) return st;
    if (out_channels * in_channels * kernel_h * kernel_w == 0) return CDX_OK;
    const int64_t OH = conv_out(in_h, kernel_h, stride_h, pad_h);
    const int64_t OW = conv_out(in_w, kernel_w, stride_w, pad_w);
    if (!grad_weight || (batch * OH * OW > 0 && (!grad_output || !input)))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    return cdx::launch_conv2d_backward_weight_f64(grad_output, input, grad_weight, batch,
                                                  in_channels, out_channels, in_h, in_w,
                                                  kernel_h, kernel_w, stride_h, stride_w, pad_h,
                                                  pad_w, stream);
}

int cdx_conv2d_backward_bias_f64(const double* grad_output, double* grad_bias, int64_t batch,
                                 int64_t out_channels, int64_t spatial, hipStream_t stream) {
    if (bad_dim(batch) || bad_dim(out_channels) || bad_dim(spatial))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_conv2d_backward_bias_f64: bad dims");
    if (out_channels == 0) return CDX_OK;
    if (!grad_bias || (batch * spatial > 0 && !grad_output))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_conv2d_backward_bias_f64: NULL pointer");
    return cdx::launch_conv_bias_grad_f64(grad_output, grad_bias, batch, out_channels, spatial,
                                          stream);
}

size_t cdx_sum_reduce_rows_workspace_size(int64_t rows, int64_t cols) {
    if (bad_dim(rows) || bad_dim(cols)) return 0;
    // sized for fp64 partials so one query serves both dtypes
    return (size_t)cdx::colsum_partial_rows(rows, cols) * (size_t)cols * sizeof(double);
}

extern "C++" {
template <typename T, typename Launch>
static int sum_reduce_rows_impl(const char* fn, const T* input, T* output, int64_t rows,
                                int64_t cols, void* workspace, size_t workspace_bytes,
                                hipStream_t stream, Launch launch) {
    if (bad_dim(rows) || bad_dim(cols))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad dims");
    if (cols == 0) return CDX_OK;
    if (!output || (rows > 0 && !input))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    const int64_t pr = cdx::colsum_partial_rows(rows, cols);
    Scratch ws;
    int st = ws.acquire(workspace, workspace_bytes, (size_t)pr * (size_t)cols * sizeof(T), stream, fn);
    if (st) return st;
    st = launch(input, output, rows, cols, static_cast<T*>(ws.ptr), pr, stream);
    return ws.release(st);
}
}  // extern "C++"

int cdx_sum_reduce_rows_f32(const float* input, float* output, int64_t rows, int64_t cols,
                            void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return sum_reduce_rows_impl("cdx_sum_reduce_rows_f32", input, output, rows, cols, workspace,
                                workspace_bytes, stream, cdx::launch_colsum_f32);
}

int cdx_sum_reduce_rows_f64(const double* input, double* output, int64_t rows, int64_t cols,
                            void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return sum_reduce_rows_impl("cdx_sum_reduce_rows_f64", input, output, rows, cols, workspace,
                                workspace_bytes, stream, cdx::launch_colsum_f64);
}

extern "C++" {
template <typename T, typename Launch>
static int bias_row_impl(const char* fn, const T* matrix, const T* row, T* out, int64_t rows,
                         int64_t cols, hipStream_t stream, Launch launch) {
    if (bad_dim(rows) || bad_dim(cols))
        return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad dims");
    if (rows == 0 || cols == 0) return CDX_OK;
    if (!matrix || !row || !out) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    return launch(matrix, row, out, rows, cols, stream);
}
}  // extern "C++"

int cdx_broadcast_add_row_f32(const float* matrix, const float* row, float* out, int64_t rows,
                              int64_t cols, hipStream_t stream) {
    return bias_row_impl("cdx_broadcast_add_row_f32", matrix, row, out, rows, cols, stream,
                         cdx::launch_broadcast_add_row_f32);
}

int cdx_broadcast_add_row_f64(const double* matrix, const double* row, double* out, int64_t rows,
                              int64_t cols, hipStream_t stream) {
    return bias_row_impl("cdx_broadcast_add_row_f64", matrix, row, out, rows, cols, stream,
                         cdx::launch_broadcast_add_row_f64);
}

extern "C++" {
static bool valid_activation(int act) {
    return act == CDX_EPI_RELU || act == CDX_EPI_GELU || act == CDX_EPI_SILU ||
           act == CDX_EPI_SIGMOID || act == CDX_ACT_TANH || act == CDX_ACT_LEAKY_RELU;
}

template <typename T, typename Launch>
static int act_impl(const char* fn, const T* input, T* output, int64_t n, int act, float alpha,
                    hipStream_t stream, Launch launch) {
    if (bad_dim(n)) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad n");
    if (!valid_activation(act))
        return set_error(CDX_ERR_INVALID_ARG,
                         std::string(fn) + ": act must be RELU, GELU, SILU, SIGMOID, TANH or LEAKY_RELU");
    if (n == 0) return CDX_OK;
    if (!input || !output) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    return launch(input, output, n, act, alpha, stream);
}

template <typename T, typename Launch>
static int act_bwd_impl(const char* fn, const T* go, const T* input, T* gi, int64_t n, int act,
                        float alpha, hipStream_t stream, Launch launch) {
    if (bad_dim(n)) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": bad n");
    if (!valid_activation(act))
        return set_error(CDX_ERR_INVALID_ARG,
                         std::string(fn) + ": act must be RELU, GELU, SILU, SIGMOID, TANH or LEAKY_RELU");
    if (n == 0) return CDX_OK;
    if (!go || !input || !gi) return set_error(CDX_ERR_INVALID_ARG, std::string(fn) + ": NULL pointer");
    return launch(go, input, gi, n, act, alpha, stream);
}
}  // extern "C++"

int cdx_activation_forward_f32(const float* input, float* output, int64_t n, int act, float alpha,
                               hipStream_t stream) {
    return act_impl("cdx_activation_forward_f32", input, output, n, act, alpha, stream,
                    cdx::launch_activation_f32);
}

int cdx_activation_forward_f64(const double* input, double* output, int64_t n, int act,
                               float alpha, hipStream_t stream) {
    return act_impl("cdx_activation_forward_f64", input, output, n, act, alpha, stream,
                    cdx::launch_activation_f64);
}

int cdx_activation_backward_f32(const float* grad_output, const float* input, float* grad_input,
                                int64_t n, int act, float alpha, hipStream_t stream) {
    return act_bwd_impl("cdx_activation_backward_f32", grad_output, input, grad_input, n, act,
                        alpha, stream, cdx::launch_activation_backward_f32);
}

int cdx_activation_backward_f64(const double* grad_output, const double* input,
                                double* grad_input, int64_t n, int act, float alpha,
                                hipStream_t stream) {
    return act_bwd_impl("cdx_activation_backward_f64", grad_output, input, grad_input, n, act,
                        alpha, stream, cdx::launch_activation_backward_f64);
}

static bool bad_dtype(int dtype) { return dtype != CDX_DTYPE_F32 && dtype != CDX_DTYPE_F64; }

int cdx_strided_copy(const void* src, void* dst, int ndim, const int64_t* shape,
                     const int64_t* src_strides, int dtype, hipStream_t stream) {
    if (ndim < 0 || ndim > 8) return set_error(CDX_ERR_UNSUPPORTED, "cdx_strided_copy: ndim must be <= 8");
    if (bad_dtype(dtype)) return set_error(CDX_ERR_INVALID_ARG, "cdx_strided_copy: bad dtype");
    if (ndim > 0 && (!shape || !src_strides))
        return set_error(CDX_ERR_INVALID_ARG, "cdx_strided_copy: NULL shape/strides");
    int64_t n = 1;
    for (int d = 0; d < ndim; ++d) {
        if (bad_dim(shape[d]) || src_strides[d] < 0)
            return set_error(CDX_ERR_INVALID_ARG, "cdx_strided_copy: bad shape/stride");
        n *= shape[d];
    }
    if (n == 0) return CDX_OK;
    if (!src || !dst) return set_error(CDX_ERR_INVALID_ARG, "cdx_strided_copy: NULL pointer");
    return cdx::launch_strided_copy(src, dst, ndim, shape, src_strides, dtype, stream);
}

int cdx_fill(void* dst, int64_t n, double value, int dtype, hipStream_t stream) {
    if (bad_dim(n) || bad_dtype(dtype)) return set_error(CDX_ERR_INVALID_ARG, "cdx_fill: bad args");
    if (n == 0) return CDX_OK;
    if (!dst) return set_error(CDX_ERR_INVALID_ARG, "cdx_fill: NULL pointer");
    return cdx::launch_fill(dst, n, value, dtype, stream);
}

int cdx_binary(int op, int dtype, const void* a, const void* b, void* out, int64_t n,
               hipStream_t stream) {
    if (op != CDX_BINARY_ADD && op != CDX_BINARY_SUB && op != CDX_BINARY_MUL)
        return set_error(CDX_ERR_INVALID_ARG, "cdx_binary: bad op");
    if (bad_dim(n) || bad_dtype(dtype)) return set_error(CDX_ERR_INVALID_ARG, "cdx_binary: bad args");
    if (n == 0) return CDX_OK;
    if (!a || !b || !out) return set_error(CDX_ERR_INVALID_ARG, "cdx_binary: NULL pointer");
    return cdx::launch_binary(op, dtype, a, b, out, n, stream);
}

int cdx_randn(void* dst, int64_t n, int dtype, uint64_t seed, uint64_t offset, hipStream_t stream) {
    if (bad_dim(n) || bad_dtype(dtype)) return set_error(CDX_ERR_INVALID_ARG, "cdx_randn: bad args");
    if (n == 0) return CDX_OK;
    if (!dst) return set_error(CDX_ERR_INVALID_ARG, "cdx_randn: NULL pointer");
    return cdx::launch_randn(dst, n, dtype, seed, offset, stream);
}

size_t cdx_sum_workspace_size(int dtype) {
    return (size_t)cdx::sum_partials() * (dtype == CDX_DTYPE_F64 ? sizeof(double) : sizeof(float));
}

int cdx_sum(const void* x, void* out, int64_t n, int dtype, void* workspace,
            size_t workspace_bytes, hipStream_t stream) {
    if (bad_dim(n) || bad_dtype(dtype)) return set_error(CDX_ERR_INVALID_ARG, "cdx_sum: bad args");
    if (!out || (n > 0 && !x)) return set_error(CDX_ERR_INVALID_ARG, "cdx_sum: NULL pointer");
    Scratch ws;
    int st = ws.acquire(workspace, workspace_bytes, cdx_sum_workspace_size(dtype), stream, "cdx_sum");
    if (st) return st;
    st = cdx::launch_sum(x, out, n, dtype, ws.ptr, stream);
    return ws.release(st);
}

}  // extern "C"
