/*
 * CPU oracle for the dense-contraction path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline).
 * The product (cudeep_amd/) never calls it and has no CPU fallback.
 *
 * Each routine restates the arithmetic of one reference function, cited as
 * file:line under /root/reference (KevinWeiss1995/cuDeep):
 *
 *   orc_sgemm_seqfma    src/kernels/matmul_kernel.cu:499-520 (sgemm_fast_kernel
 *                       COMPUTE: acc[m][n] += a*b, k ascending, nvcc-contracted
 *                       to one fmaf per k) and :632-647 (sgemm_general_kernel).
 *   orc_dgemm           fp64 closed form C = op(A) op(B), the error yardstick.
 *   orc_gemm_tf32emu    src/kernels/matmul_kernel.cu:179-214 (mma.m16n8k8.tf32,
 *                       four k-steps of 8 per BK_TC=32 tile), operand semantics
 *                       include/cudeep/ptx_intrinsics.cuh:316-335, 639-649.
 *   orc_im2col          src/kernels/conv_kernel.cu:32-65.
 *   orc_transpose_bias  src/kernels/conv_kernel.cu:74-93.
 *   orc_conv2d_direct64 src/kernels/conv_kernel.cu:113-159 (naive kernel:
 *                       cross-correlation, zero padding), output size :235-236.
 *   orc_conv2d_implicit src/kernels/conv_kernel.cu:172-215 (implicit_gemm_conv2d_kernel:
 *                       acc = bias, then one fmaf per in-range tap, ic -> kh -> kw).
 *   orc_col2im          src/kernels/conv_kernel.cu:344-380 (fp32, kh then kw).
 *   orc_col2im64        the same gather in double (yardstick).
 *   orc_colsum          src/kernels/unary_kernel.cu:204-238 (serial fp32 sum
 *                       down each column).
 *   orc_gelu / relu     src/kernels/activation_kernel.cu:19-52 (forward) and
 *                       :256-319 (backward), written in double.
 *   orc_winograd_f43    src/kernels/conv_kernel.cu:557-789 (Winograd F(4,3) route
 *                       for 3x3 stride-1 convolution), fp32; _64: in double.
 *
 * Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp).
 * -ffp-contract=off keeps every fma explicit (fmaf) and forbids the compiler
 * from fusing anything else, so the sequential-FMA SGEMM is bit-reproducible.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* Element (r, c) of op(X), where X is stored row-major with leading dim ld and
 * op is the identity (trans=0) or the transpose (trans=1). */
#define OPX(X, trans, ld, r, c) ((trans) ? (X)[(int64_t)(c) * (ld) + (r)] \
                                         : (X)[(int64_t)(r) * (ld) + (c)])

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/*
 * Sequential-FMA SGEMM: C[i][j] = fmaf(a_ik, b_kj, acc) for k = 0..K-1 in
 * ascending order starting from acc = +0.0f, exactly one rounding per k.
 * This is the per-output operation sequence of sgemm_fast_kernel /
 * sgemm_general_kernel (matmul_kernel.cu:499-520, :632-647).
 *
 * The loop nest is blocked (column panels of JB, row blocks of IB) for cache
 * reuse, but every output still sees its k terms in ascending order through
 * fmaf, so the result is bit-identical to the naive per-output chain.
 * Rows [row0, row1) only are produced (row sampling for large shapes); C is
 * [row1-row0][N] row-major.
 */
void orc_sgemm_seqfma_rows(const float* A, const float* B, float* C,
                           int64_t M, int64_t N, int64_t K,
                           int transA, int transB, int64_t lda, int64_t ldb,
                           int64_t row0, int64_t row1) {
    const int64_t JB = 256, IB = 16;
    (void)M;
    int64_t rows = row1 - row0;
    int64_t nib = (rows + IB - 1) / IB;
    int64_t njb = (N + JB - 1) / JB;
    float* Bt = NULL;
    /* For transB, gather a contiguous k-major copy of B once so the inner j
     * loop is unit-stride. Pure data movement; arithmetic is unchanged. */
    if (transB) {
        Bt = (float*)malloc((size_t)K * (size_t)N * sizeof(float));
        #pragma omp parallel for schedule(static)
        for (int64_t k = 0; k < K; ++k)
            for (int64_t j = 0; j < N; ++j) Bt[k * N + j] = B[j * ldb + k];
        B = Bt; ldb = N; transB = 0;
    }
    #pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t jb = 0; jb < njb; ++jb) {
        for (int64_t ib = 0; ib < nib; ++ib) {
            int64_t j0 = jb * JB, j1 = j0 + JB < N ? j0 + JB : N;
            int64_t i0 = row0 + ib * IB, i1 = i0 + IB < row1 ? i0 + IB : row1;
            float acc[16][256];
            for (int64_t i = i0; i < i1; ++i)
                for (int64_t j = j0; j < j1; ++j) acc[i - i0][j - j0] = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float* brow = B + k * ldb;
                for (int64_t i = i0; i < i1; ++i) {
                    float a = OPX(A, transA, lda, i, k);
                    float* ar = acc[i - i0];
                    for (int64_t j = j0; j < j1; ++j)
                        ar[j - j0] = fmaf(a, brow[j], ar[j - j0]);
                }
            }
            for (int64_t i = i0; i < i1; ++i)
                for (int64_t j = j0; j < j1; ++j)
                    C[(i - row0) * N + j] = acc[i - i0][j - j0];
        }
    }
    free(Bt);
}

void orc_sgemm_seqfma(const float* A, const float* B, float* C,
                      int64_t M, int64_t N, int64_t K,
                      int transA, int transB, int64_t lda, int64_t ldb) {
    orc_sgemm_seqfma_rows(A, B, C, M, N, K, transA, transB, lda, ldb, 0, M);
}

/* fp64 GEMM over fp32 or fp64 operands (double accumulation, k ascending).
 * Rows [row0, row1) only. Used as the error yardstick; any fp64 summation
 * order is far below fp32 error. */
void orc_dgemm_rows_f32in(const float* A, const float* B, double* C,
                          int64_t M, int64_t N, int64_t K,
                          int transA, int transB, int64_t lda, int64_t ldb,
                          int64_t row0, int64_t row1) {
    (void)M;
    #pragma omp parallel for schedule(dynamic, 4)
    for (int64_t i = row0; i < row1; ++i) {
        double* crow = C + (i - row0) * N;
        for (int64_t j = 0; j < N; ++j) crow[j] = 0.0;
        for (int64_t k = 0; k < K; ++k) {
            double a = (double)OPX(A, transA, lda, i, k);
            if (!transB) {
                const float* brow = B + k * ldb;
                for (int64_t j = 0; j < N; ++j) crow[j] += a * (double)brow[j];
            } else {
                for (int64_t j = 0; j < N; ++j) crow[j] += a * (double)B[j * ldb + k];
            }
        }
    }
}

void orc_dgemm_f64(const double* A, const double* B, double* C,
                   int64_t M, int64_t N, int64_t K,
                   int transA, int transB, int64_t lda, int64_t ldb) {
    #pragma omp parallel for schedule(dynamic, 4)
    for (int64_t i = 0; i < M; ++i) {
        double* crow = C + i * N;
        for (int64_t j = 0; j < N; ++j) crow[j] = 0.0;
        for (int64_t k = 0; k < K; ++k) {
            double a = OPX(A, transA, lda, i, k);
            for (int64_t j = 0; j < N; ++j) crow[j] += a * OPX(B, transB, ldb, k, j);
        }
    }
}

/* Round an fp32 value to a 10-bit mantissa (TF32 operand).
 * mode 0: round toward zero (mask 0xFFFFE000, raw bits fed to the MMA).
 * mode 1: round to nearest even (the unused helper fp32_to_tf32,
 *         ptx_intrinsics.cuh:639-649 intends round-to-nearest). */
static inline float tf32_round(float x, int mode) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7F800000u) == 0x7F800000u) return x; /* inf / nan */
    if (mode == 1) {
        uint32_t lsb = (u >> 13) & 1u;
        u += 0x0FFFu + lsb;
    }
    u &= 0xFFFFE000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}

float orc_tf32_round(float x, int mode) { return tf32_round(x, mode); }

/*
 * TF32 tensor-core GEMM emulation ("ideal MMA"): operands rounded to TF32,
 * products exact, each k-chunk of 8 (one m16n8k8 MMA) summed exactly and
 * added to the fp32 accumulator with one rounding; chunks in ascending k
 * (matmul_kernel.cu:179-214: 4 MMA k-steps of 8 per BK_TC=32 tile).
 * An 11-bit x 11-bit product is exact in double and 8 of them sum exactly.
 */
void orc_gemm_tf32emu_rows(const float* A, const float* B, float* C,
                           int64_t M, int64_t N, int64_t K, int round_mode,
                           int64_t row0, int64_t row1) {
    (void)M;
    /* Round B once (a copy); A is rounded on the fly. */
    float* Br = (float*)malloc((size_t)K * (size_t)N * sizeof(float));
    #pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < K * N; ++t) Br[t] = tf32_round(B[t], round_mode);
    #pragma omp parallel
    {
        double* chunk = (double*)malloc((size_t)N * sizeof(double));
        float* acc = (float*)malloc((size_t)N * sizeof(float));
        #pragma omp for schedule(dynamic, 1)
        for (int64_t i = row0; i < row1; ++i) {
            for (int64_t j = 0; j < N; ++j) acc[j] = 0.0f;
            for (int64_t k0 = 0; k0 < K; k0 += 8) {
                int64_t k1 = k0 + 8 < K ? k0 + 8 : K;
                for (int64_t j = 0; j < N; ++j) chunk[j] = 0.0;
                for (int64_t k = k0; k < k1; ++k) {
                    double a = (double)tf32_round(A[i * K + k], round_mode);
                    const float* brow = Br + k * N;
                    for (int64_t j = 0; j < N; ++j) chunk[j] += a * (double)brow[j];
                }
                for (int64_t j = 0; j < N; ++j) acc[j] = (float)((double)acc[j] + chunk[j]);
            }
            for (int64_t j = 0; j < N; ++j) C[(i - row0) * N + j] = acc[j];
        }
        free(chunk);
        free(acc);
    }
    free(Br);
}

void orc_gemm_tf32emu(const float* A, const float* B, float* C,
                      int64_t M, int64_t N, int64_t K, int round_mode) {
    orc_gemm_tf32emu_rows(A, B, C, M, N, K, round_mode, 0, M);
}

static inline int64_t conv_out(int64_t in, int64_t k, int64_t s, int64_t p) {
    return (in + 2 * p - k) / s + 1; /* conv_kernel.cu:235-236 */
}

/*
 * im2col, bit-exact restatement of conv_kernel.cu:32-65:
 *   col[k * B_spatial + b * spatial + s] = input[b, ic, ih, iw] or 0,
 *   k = (ic*KH + kh)*KW + kw, s = oh*OW + ow,
 *   ih = oh*SH - PH + kh, iw = ow*SW - PW + kw.
 * 64-bit indices; identical to the reference wherever its 32-bit ints do
 * not overflow.
 */
void orc_im2col(const float* input, float* col,
                int64_t batch, int64_t IC, int64_t IH, int64_t IW,
                int64_t KH, int64_t KW, int64_t SH, int64_t SW,
                int64_t PH, int64_t PW) {
    int64_t OH = conv_out(IH, KH, SH, PH), OW = conv_out(IW, KW, SW, PW);
    int64_t K_col = IC * KH * KW, spatial = OH * OW, B_spatial = batch * spatial;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t k = 0; k < K_col; ++k) {
            int64_t kw = k % KW, kh = (k / KW) % KH, ic = k / (KW * KH);
            for (int64_t s = 0; s < spatial; ++s) {
                int64_t oh = s / OW, ow = s % OW;
                int64_t ih = oh * SH - PH + kh, iw = ow * SW - PW + kw;
                float v = 0.0f;
                if (ih >= 0 && ih < IH && iw >= 0 && iw < IW)
                    v = input[((b * IC + ic) * IH + ih) * IW + iw];
                col[k * B_spatial + b * spatial + s] = v;
            }
        }
    }
}

/* [OC, B*spatial] -> NCHW [B, OC, spatial] (+ bias[oc], one fp32 add).
 * conv_kernel.cu:74-93. bias may be NULL. */
void orc_transpose_bias(const float* src, float* dst, const float* bias,
                        int64_t OC, int64_t batch, int64_t spatial) {
    int64_t B_spatial = batch * spatial;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int64_t oc = 0; oc < OC; ++oc)
        for (int64_t b = 0; b < batch; ++b)
            for (int64_t s = 0; s < spatial; ++s) {
                float v = src[oc * B_spatial + b * spatial + s];
                if (bias) v += bias[oc];
                dst[(b * OC + oc) * spatial + s] = v;
            }
}

/* fp64 direct convolution (cross-correlation, zero padding), NCHW / OIHW,
 * loop order ic -> kh -> kw as conv2d_forward_naive_kernel
 * (conv_kernel.cu:113-159). bias may be NULL. Output in double. */
void orc_conv2d_direct64(const float* input, const float* weight, const float* bias,
                         double* out, int64_t batch, int64_t IC, int64_t OC,
                         int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                         int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    int64_t OH = conv_out(IH, KH, SH, PH), OW = conv_out(IW, KW, SW, PW);
    #pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t oc = 0; oc < OC; ++oc)
            for (int64_t oh = 0; oh < OH; ++oh)
                for (int64_t ow = 0; ow < OW; ++ow) {
                    double acc = bias ? (double)bias[oc] : 0.0;
                    for (int64_t ic = 0; ic < IC; ++ic)
                        for (int64_t kh = 0; kh < KH; ++kh) {
                            int64_t ih = oh * SH - PH + kh;
                            if (ih < 0 || ih >= IH) continue;
                            for (int64_t kw = 0; kw < KW; ++kw) {
                                int64_t iw = ow * SW - PW + kw;
                                if (iw < 0 || iw >= IW) continue;
                                acc += (double)input[((b * IC + ic) * IH + ih) * IW + iw] *
                                       (double)weight[((oc * IC + ic) * KH + kh) * KW + kw];
                            }
                        }
                    out[((b * OC + oc) * OH + oh) * OW + ow] = acc;
                }
}

/* fp32 restatement of implicit_gemm_conv2d_kernel (conv_kernel.cu:172-215),
 * the reference's forward route for layers whose column buffer would exceed
 * 4 MiB outside 3x3 stride 1 (:263-275): per output, acc = bias[oc] (or 0),
 * then acc += in * w over ic, kh, kw ascending, skipping taps outside the
 * image (the `continue`s), nvcc-contracted to one fmaf per tap. */
void orc_conv2d_implicit(const float* input, const float* weight, const float* bias,
                         float* out, int64_t batch, int64_t IC, int64_t OC,
                         int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                         int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    int64_t OH = conv_out(IH, KH, SH, PH), OW = conv_out(IW, KW, SW, PW);
    #pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t oc = 0; oc < OC; ++oc)
            for (int64_t oh = 0; oh < OH; ++oh)
                for (int64_t ow = 0; ow < OW; ++ow) {
                    float acc = bias ? bias[oc] : 0.0f;
                    for (int64_t ic = 0; ic < IC; ++ic)
                        for (int64_t kh = 0; kh < KH; ++kh) {
                            int64_t ih = oh * SH - PH + kh;
                            if (ih < 0 || ih >= IH) continue;
                            for (int64_t kw = 0; kw < KW; ++kw) {
                                int64_t iw = ow * SW - PW + kw;
                                if (iw < 0 || iw >= IW) continue;
                                acc = fmaf(input[((b * IC + ic) * IH + ih) * IW + iw],
                                           weight[((oc * IC + ic) * KH + kh) * KW + kw], acc);
                            }
                        }
                    out[((b * OC + oc) * OH + oh) * OW + ow] = acc;
                }
}

/*
 * col2im, restatement of col2im_kernel (conv_kernel.cu:344-380): for each
 * input element (b, ic, ih, iw), acc = 0 then, for kh ascending and kw
 * ascending, acc += col[k * B_spatial + b * spatial + oh * OW + ow] over
 * the (oh, ow) the element was copied to.  fp32 accumulation.
 */
void orc_col2im(const float* col, float* grad_in,
                int64_t batch, int64_t IC, int64_t IH, int64_t IW,
                int64_t KH, int64_t KW, int64_t SH, int64_t SW,
                int64_t PH, int64_t PW) {
    int64_t OH = conv_out(IH, KH, SH, PH), OW = conv_out(IW, KW, SW, PW);
    int64_t spatial = OH * OW, B_spatial = batch * spatial;
    int64_t total = batch * IC * IH * IW;
    #pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int64_t iw = idx % IW, ih = (idx / IW) % IH, ic = (idx / (IW * IH)) % IC;
        int64_t b = idx / (IW * IH * IC);
        float acc = 0.0f;
        for (int64_t kh = 0; kh < KH; ++kh) {
            int64_t oh_num = ih + PH - kh;
            if (oh_num < 0 || oh_num % SH != 0) continue;
            int64_t oh = oh_num / SH;
            if (oh >= OH) continue;
            for (int64_t kw = 0; kw < KW; ++kw) {
                int64_t ow_num = iw + PW - kw;
                if (ow_num < 0 || ow_num % SW != 0) continue;
                int64_t ow = ow_num / SW;
                if (ow >= OW) continue;
                int64_t k = (ic * KH + kh) * KW + kw;
                acc += col[k * B_spatial + b * spatial + oh * OW + ow];
            }
        }
        grad_in[idx] = acc;
    }
}

void orc_col2im64(const double* col, double* grad_in,
                  int64_t batch, int64_t IC, int64_t IH, int64_t IW,
                  int64_t KH, int64_t KW, int64_t SH, int64_t SW,
                  int64_t PH, int64_t PW) {
    int64_t OH = conv_out(IH, KH, SH, PH), OW = conv_out(IW, KW, SW, PW);
    int64_t spatial = OH * OW, B_spatial = batch * spatial;
    int64_t total = batch * IC * IH * IW;
    #pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        int64_t iw = idx % IW, ih = (idx / IW) % IH, ic = (idx / (IW * IH)) % IC;
        int64_t b = idx / (IW * IH * IC);
        double acc = 0.0;
        for (int64_t kh = 0; kh < KH; ++kh) {
            int64_t oh_num = ih + PH - kh;
            if (oh_num < 0 || oh_num % SH != 0) continue;
            int64_t oh = oh_num / SH;
            if (oh >= OH) continue;
            for (int64_t kw = 0; kw < KW; ++kw) {
                int64_t ow_num = iw + PW - kw;
                if (ow_num < 0 || ow_num % SW != 0) continue;
                int64_t ow = ow_num / SW;
                if (ow >= OW) continue;
                int64_t k = (ic * KH + kh) * KW + kw;
                acc += col[k * B_spatial + b * spatial + oh * OW + ow];
            }
        }
        grad_in[idx] = acc;
    }
}

/* Column sums of a row-major [rows, cols] fp32 matrix, serial fp32
 * accumulation down each column (unary_kernel.cu:204-238). */
void orc_colsum(const float* in, float* out, int64_t rows, int64_t cols) {
    for (int64_t j = 0; j < cols; ++j) out[j] = 0.0f;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < cols; ++j) out[j] += in[r * cols + j];
}

/* GELU, tanh form (Hendrycks & Gimpel), the formula of
 * activation_kernel.cu:40-46, evaluated in double. */
double orc_gelu(double x) {
    const double c = 0.7978845608, k = 0.044715;
    return 0.5 * x * (1.0 + tanh(c * (x + k * x * x * x)));
}

/* d GELU / dx for the same form (activation_kernel.cu:293-301). */
double orc_gelu_grad(double x) {
    const double c = 0.7978845608, k = 0.044715;
    double th = tanh(c * (x + k * x * x * x));
    return 0.5 * (1.0 + th) + 0.5 * x * (1.0 - th * th) * c * (1.0 + 3.0 * k * x * x);
}

void orc_gelu_vec(const double* x, double* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_gelu(x[i]);
}

void orc_gelu_grad_vec(const double* x, double* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_gelu_grad(x[i]);
}

/*
 * Winograd F(4x4, 3x3) convolution, the reference's route for 3x3 stride-1
 * convolutions (conv_kernel.cu:242-248, :557-789), with the transform
 * matrices of Lavin & Gray (2016) for the interpolation points 0, +-1, +-2:
 *   U = G g G^T   (3x3 filter  -> 6x6),   G   = [1/4 0 0; -1/6 -1/6 -1/6;
 *                                                -1/6 1/6 -1/6; 1/24 1/12 1/6;
 *                                                1/24 -1/12 1/6; 0 0 1]
 *   V = B^T d B   (6x6 input patch at (4 th - PH, 4 tw - PW), zero padded),
 *                 B^T rows: [4 0 -5 0 1 0] [0 -4 -4 1 1 0] [0 4 -4 -1 1 0]
 *                           [0 -2 -1 2 1 0] [0 2 -1 -2 1 0] [0 4 0 -5 0 1]
 *   M_a = U_a V_a  for each of the 36 points a (a GEMM over input channels),
 *   Y = A^T m A + bias (6x6 -> 4x4 output tile),
 *                 A^T rows: [1 1 1 1 1 0] [0 1 -1 2 -2 0] [0 1 1 4 4 0]
 *                           [0 1 -1 8 -8 1]
 * Each 2-D transform applies the 1-D transform to the columns, then to the
 * rows of the result (conv_kernel.cu:611-617, :656-670, :709-728).  The
 * fp32 form sums the 36 GEMMs by sequential fmaf over ic ascending (the
 * reference's FP32 GEMM, matmul_kernel.cu:499-520); the double form is the
 * same algorithm in fp64, which equals direct convolution up to rounding.
 */
#define WINO_BODY(T, NAME, FMA, ROUND)                                                   \
static void NAME##_wcol(T g0, T g1, T g2, T* u) {                                       \
    u[0] = (T)0.25 * g0;                                                                \
    u[1] = -((T)1 / (T)6) * (g0 + g1 + g2);                                             \
    u[2] = -((T)1 / (T)6) * (g0 - g1 + g2);                                             \
    u[3] = ((T)1 / (T)24) * g0 + ((T)1 / (T)12) * g1 + ((T)1 / (T)6) * g2;              \
    u[4] = ((T)1 / (T)24) * g0 - ((T)1 / (T)12) * g1 + ((T)1 / (T)6) * g2;              \
    u[5] = g2;                                                                          \
}                                                                                       \
static void NAME##_icol(const T* d, T* t) {                                             \
    t[0] = (T)4 * d[0] - (T)5 * d[2] + d[4];                                            \
    t[1] = -(T)4 * d[1] - (T)4 * d[2] + d[3] + d[4];                                    \
    t[2] = (T)4 * d[1] - (T)4 * d[2] - d[3] + d[4];                                     \
    t[3] = -(T)2 * d[1] - d[2] + (T)2 * d[3] + d[4];                                    \
    t[4] = (T)2 * d[1] - d[2] - (T)2 * d[3] + d[4];                                     \
    t[5] = (T)4 * d[1] - (T)5 * d[3] + d[5];                                            \
}                                                                                       \
static void NAME##_ocol(const T* m, T* o) {                                             \
    o[0] = m[0] + m[1] + m[2] + m[3] + m[4];                                            \
    o[1] = m[1] - m[2] + (T)2 * m[3] - (T)2 * m[4];                                     \
    o[2] = m[1] + m[2] + (T)4 * m[3] + (T)4 * m[4];                                     \
    o[3] = m[1] - m[2] + (T)8 * m[3] - (T)8 * m[4] + m[5];                              \
}                                                                                       \
void NAME(const float* input, const float* weight, const float* bias, T* out,           \
          int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,                \
          int64_t PH, int64_t PW, int tf32_mode) {                                      \
    const int64_t OH = IH + 2 * PH - 2, OW = IW + 2 * PW - 2;                           \
    const int64_t TH = (OH + 3) / 4, TW = (OW + 3) / 4, NT = batch * TH * TW;           \
    T* U = (T*)malloc(sizeof(T) * 36 * OC * IC);                                        \
    T* V = (T*)malloc(sizeof(T) * 36 * IC * NT);                                        \
    T* Mm = (T*)malloc(sizeof(T) * 36 * OC * NT);                                       \
    _Pragma("omp parallel for schedule(static)")                                        \
    for (int64_t p = 0; p < OC * IC; ++p) {                                             \
        const float* g = weight + p * 9;                                                \
        T tmp[6][3], u[6];                                                              \
        for (int j = 0; j < 3; ++j) {                                                   \
            NAME##_wcol((T)g[j], (T)g[3 + j], (T)g[6 + j], u);                          \
            for (int i = 0; i < 6; ++i) tmp[i][j] = u[i];                               \
        }                                                                               \
        for (int i = 0; i < 6; ++i) {                                                   \
            NAME##_wcol(tmp[i][0], tmp[i][1], tmp[i][2], u);                            \
            for (int j = 0; j < 6; ++j)                                                 \
                U[(int64_t)(i * 6 + j) * OC * IC + p] = ROUND(u[j], tf32_mode);         \
        }                                                                               \
    }                                                                                   \
    _Pragma("omp parallel for schedule(static)")                                        \
    for (int64_t q = 0; q < IC * NT; ++q) {                                             \
        const int64_t ic = q / NT, tile = q % NT;                                       \
        const int64_t b = tile / (TH * TW), th = (tile / TW) % TH, tw = tile % TW;      \
        const float* src = input + (b * IC + ic) * IH * IW;                             \
        T d[6][6], tmp[6][6], col[6], t[6];                                             \
        for (int i = 0; i < 6; ++i)                                                     \
            for (int j = 0; j < 6; ++j) {                                               \
                const int64_t ih = th * 4 - PH + i, iw = tw * 4 - PW + j;               \
                d[i][j] = (ih >= 0 && ih < IH && iw >= 0 && iw < IW)                    \
                              ? (T)src[ih * IW + iw] : (T)0;                            \
            }                                                                           \
        for (int j = 0; j < 6; ++j) {                                                   \
            for (int i = 0; i < 6; ++i) col[i] = d[i][j];                               \
            NAME##_icol(col, t);                                                        \
            for (int i = 0; i < 6; ++i) tmp[i][j] = t[i];                               \
        }                                                                               \
        for (int i = 0; i < 6; ++i) {                                                   \
            NAME##_icol(tmp[i], t);                                                     \
            for (int j = 0; j < 6; ++j)                                                 \
                V[((int64_t)(i * 6 + j) * IC + ic) * NT + tile] = ROUND(t[j], tf32_mode); \
        }                                                                               \
    }                                                                                   \
    _Pragma("omp parallel for collapse(2) schedule(static)")                            \
    for (int64_t a = 0; a < 36; ++a)                                                    \
        for (int64_t oc = 0; oc < OC; ++oc) {                                           \
            T* mrow = Mm + (a * OC + oc) * NT;                                          \
            for (int64_t n = 0; n < NT; ++n) mrow[n] = (T)0;                            \
            for (int64_t ic = 0; ic < IC; ++ic) {                                       \
                const T u = U[(a * OC + oc) * IC + ic];                                 \
                const T* vrow = V + (a * IC + ic) * NT;                                 \
                for (int64_t n = 0; n < NT; ++n) mrow[n] = FMA(u, vrow[n], mrow[n]);    \
            }                                                                           \
        }                                                                               \
    _Pragma("omp parallel for schedule(static)")                                        \
    for (int64_t q = 0; q < OC * NT; ++q) {                                             \
        const int64_t oc = q / NT, tile = q % NT;                                       \
        const int64_t b = tile / (TH * TW), th = (tile / TW) % TH, tw = tile % TW;      \
        T m[6][6], tmp[4][6], col[6], o[4];                                             \
        for (int i = 0; i < 6; ++i)                                                     \
            for (int j = 0; j < 6; ++j) m[i][j] = Mm[((int64_t)(i * 6 + j) * OC + oc) * NT + tile]; \
        for (int j = 0; j < 6; ++j) {                                                   \
            for (int i = 0; i < 6; ++i) col[i] = m[i][j];                               \
            NAME##_ocol(col, o);                                                        \
            for (int i = 0; i < 4; ++i) tmp[i][j] = o[i];                               \
        }                                                                               \
        const T bv = bias ? (T)bias[oc] : (T)0;                                         \
        for (int i = 0; i < 4; ++i) {                                                   \
            NAME##_ocol(tmp[i], o);                                                     \
            const int64_t oh = th * 4 + i;                                              \
            if (oh >= OH) break;                                                        \
            for (int j = 0; j < 4; ++j) {                                               \
                const int64_t ow = tw * 4 + j;                                          \
                if (ow < OW) out[((b * OC + oc) * OH + oh) * OW + ow] = o[j] + bv;      \
            }                                                                           \
        }                                                                               \
    }                                                                                   \
    free(U); free(V); free(Mm);                                                         \
}

/* tf32_mode 0: GEMM operands as computed; 1 = RZ, 2 = RNE: rounded to TF32
 * first, as the reference's default (TF32 tensor-core) GEMM sees them. */
static inline float wino_round_f(float x, int mode) { return mode ? tf32_round(x, mode - 1) : x; }
static inline double wino_round_d(double x, int mode) { (void)mode; return x; }
WINO_BODY(float, orc_winograd_f43, fmaf, wino_round_f)
WINO_BODY(double, orc_winograd_f43_64, fma, wino_round_d)
