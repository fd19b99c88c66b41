// Small bandwidth kernels nn.Linear needs around its GEMMs:
//   * column sums (bias gradient), replacing sum_reduce_rows_kernel
//     (src/kernels/unary_kernel.cu:204-238), which runs one thread per 4
//     columns serially down all rows (64 active threads for 256 columns).
//     Here: pass 1 splits the rows into up to kColsumMaxChunks chunks of at
//     least kColsumMinRows rows (enough workgroups to fill the GPU), 4
//     row-lanes x 64 columns per workgroup, fixed-order fp32 sums into a
//     partials buffer; pass 2 reduces the partials of each column the same
//     way.  Deterministic.
//   * broadcast row add (elementwise_kernel.cu:186-204).
//   * ReLU / GELU forward and backward (activation_kernel.cu:19-52,
//     :256-319); the GELU is the tanh form written through exp
//     (cdx_internal.hpp), not an approximate-instruction sequence.
#include <type_traits>

#include "cdx_internal.hpp"

namespace cdx {
namespace {

constexpr int kColsumMinRows = 32;       // rows per pass-1 chunk, at least
constexpr int kColsumMaxChunks = 1024;   // pass-1 chunks, at most
constexpr int kColsumCols = 64;          // columns per workgroup

// Sums rows [y * chunk, (y + 1) * chunk) of each column into part[y][c]:
// 4 row-lanes stride down the chunk, then a fixed-order combine.
template <typename T>
__global__ __launch_bounds__(256)
void colsum_partial_kernel(const T* __restrict__ in, T* __restrict__ part,
                           int64_t rows, int64_t cols, int64_t chunk) {
    __shared__ T red[4][kColsumCols];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t c = (int64_t)blockIdx.x * kColsumCols + tx;
    const int64_t r0 = (int64_t)blockIdx.y * chunk;
    int64_t r1 = r0 + chunk;
    if (r1 > rows) r1 = rows;
    T acc = 0;
    if (c < cols) {
        // groups of 8 rows per lane: the 8 loads are issued together, then
        // added in row order (a plain loop would wait on each load in turn)
        int64_t r = r0 + ty;
        for (; r + 28 < r1; r += 32) {
            T v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = in[(r + 4 * u) * cols + c];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += v[u];
        }
        for (; r < r1; r += 4) acc += in[r * cols + c];
    }
    red[ty][tx] = acc;
    __syncthreads();
    if (ty == 0 && c < cols)
        part[(int64_t)blockIdx.y * cols + c] = ((red[0][tx] + red[1][tx]) + red[2][tx]) + red[3][tx];
}

int64_t colsum_chunk_rows(int64_t rows) {
    int64_t chunks = ceil_div(rows, kColsumMinRows);
    if (chunks > kColsumMaxChunks) chunks = kColsumMaxChunks;
    if (chunks < 1) chunks = 1;
    return ceil_div(rows, chunks);
}

template <typename T>
__global__ __launch_bounds__(256)
void bias_row_kernel(const T* __restrict__ m, const T* __restrict__ row,
                     T* __restrict__ out, int64_t rows, int64_t cols) {
    const int64_t n = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = m[i] + row[i % cols];
}

// alpha: the leaky ReLU's negative slope (as a float, as the reference
// passes it); the product alpha * v of two floats is exact in double, so the
// float result equals the reference's float multiply
__device__ __forceinline__ double apply_act(double v, int act, double alpha) {
    if (act == CDX_EPI_RELU) return v > 0.0 ? v : 0.0;
    if (act == CDX_EPI_GELU) return gelu_f64(v);
    if (act == CDX_EPI_SILU) return silu_t(v);
    if (act == CDX_EPI_SIGMOID) return sigmoid_t(v);
    if (act == CDX_ACT_TANH) return tanh(v);
    if (act == CDX_ACT_LEAKY_RELU) return v > 0.0 ? v : alpha * v;
    return v;
}

template <typename T>
__global__ __launch_bounds__(256)
void act_fwd_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t n, int act, float alpha) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = apply_act(x[i], act, alpha);
}

__device__ __forceinline__ float gelu_grad(float v) { return gelu_grad_f32(v); }
__device__ __forceinline__ double gelu_grad(double v) { return gelu_grad_f64(v); }

// d act / dx at the pre-activation input x (ReLU / leaky ReLU: the mask x > 0,
// handled in the kernel); tanh' = 1 - tanh(x)^2, formed in double
template <typename T>
__device__ __forceinline__ T act_grad(T x, int act) {
    if (act == CDX_EPI_GELU) return gelu_grad(x);
    if (act == CDX_EPI_SILU) return silu_grad_t(x);
    if (act == CDX_ACT_TANH) {
        const double t = tanh((double)x);
        return (T)(1.0 - t * t);
    }
    return sigmoid_grad_t(x);
}

template <typename T>
__global__ __launch_bounds__(256)
void act_bwd_kernel(const T* __restrict__ go, const T* __restrict__ x,
                    T* __restrict__ gi, int64_t n, int act, float alpha) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const T v = x[i];
        if (act == CDX_EPI_RELU) gi[i] = v > T(0) ? go[i] : T(0);
        else if (act == CDX_ACT_LEAKY_RELU) gi[i] = v > T(0) ? go[i] : (T)alpha * go[i];
        else gi[i] = go[i] * act_grad(v, act);
    }
}

// float, 16-byte aligned, n % 4 == 0: four elements per thread with 16-byte
// loads / stores (the same per-element arithmetic as the kernels above)
__global__ __launch_bounds__(256)
void act_fwd_vec4_kernel(const floatx4* __restrict__ x, floatx4* __restrict__ y, int64_t n4,
                         int act, float alpha) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * blockDim.x) {
        const floatx4 v = x[i];
        floatx4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = (float)apply_act(v[j], act, alpha);
        y[i] = r;
    }
}

__global__ __launch_bounds__(256)
void act_bwd_vec4_kernel(const floatx4* __restrict__ go, const floatx4* __restrict__ x,
                         floatx4* __restrict__ gi, int64_t n4, int act, float alpha) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * blockDim.x) {
        const floatx4 v = x[i], g = go[i];
        floatx4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (act == CDX_EPI_RELU) r[j] = v[j] > 0.0f ? g[j] : 0.0f;
            else if (act == CDX_ACT_LEAKY_RELU) r[j] = v[j] > 0.0f ? g[j] : alpha * g[j];
            else r[j] = g[j] * act_grad(v[j], act);
        }
        gi[i] = r;
    }
}

template <typename T>
__global__ __launch_bounds__(256)
void fill_kernel(T* __restrict__ y, int64_t n, T v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = v;
}

// Sum of the split-K partials in slice order, then the GEMM epilogue of
// each element (store_one: bias, activation or activation backward, output
// map, ones column) -- the same float operations as the unsplit kernels'.
// A thread owns one column of a row (rows over blockIdx.y, columns over
// blockIdx.x): coalesced loads and no index division.
__global__ __launch_bounds__(256)
void splitk_reduce_kernel(const float* __restrict__ P, int splits, EpiArgs e) {
    const int64_t MN = e.M * e.N;
    for (int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; n < e.N;
         n += (int64_t)gridDim.x * blockDim.x) {
        for (int64_t m = blockIdx.y; m < e.M; m += gridDim.y) {
            const float* __restrict__ p = P + m * e.N + n;
            float v = p[0];
            // slices in order; 8 loads in flight per group instead of one at a time
            int s = 1;
            for (; s + 7 < splits; s += 8) {
                float t[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) t[u] = p[(int64_t)(s + u) * MN];
#pragma unroll
                for (int u = 0; u < 8; ++u) v += t[u];
            }
            for (; s < splits; ++s) v += p[(int64_t)s * MN];
            store_one(e, m, n, v);
        }
    }
}

unsigned grid_for(int64_t n) {
    int64_t b = ceil_div(n, 256);
    if (b > 65536) b = 65536;
    if (b < 1) b = 1;
    return (unsigned)b;
}

}  // namespace

int launch_splitk_reduce(const float* P, int splits, const GemmArgs& g, hipStream_t stream) {
    const EpiArgs e{g.C, g.ldc, g.M, g.N, g.n_split, g.ldc_split, g.bias, g.bias_mode,
                    g.epilogue, g.aux, g.ldaux, g.colsum, g.ones_col};
    int64_t gx = ceil_div(g.N, 256), gy = g.M;
    if (gx > 65535) gx = 65535;
    if (gy > 65535) gy = 65535;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0,
                       stream, P, splits, e);
    return hip_error(hipGetLastError(), "splitk_reduce_kernel launch");
}

int64_t colsum_partial_rows(int64_t rows, int64_t cols) {
    (void)cols;
    return rows > 0 ? ceil_div(rows, colsum_chunk_rows(rows)) : 1;
}

template <typename T>
int colsum_t(const T* in, T* out, int64_t rows, int64_t cols, T* partials, int64_t partial_rows,
             hipStream_t stream) {
    if (cols <= 0) return CDX_OK;
    if (rows <= 0) {   // empty sum: zeros (a fill kernel, capture-safe)
        hipLaunchKernelGGL(fill_kernel<T>, dim3(grid_for(cols)), dim3(256), 0, stream, out, cols, T(0));
        return hip_error(hipGetLastError(), "fill_kernel launch");
    }
    const int64_t chunk = colsum_chunk_rows(rows);
    const int64_t chunks = ceil_div(rows, chunk);
    if (chunks > partial_rows) return set_error(CDX_ERR_WORKSPACE, "sum_reduce_rows: partials too small");
    const unsigned gx = (unsigned)ceil_div(cols, kColsumCols);
    hipLaunchKernelGGL(colsum_partial_kernel<T>, dim3(gx, (unsigned)chunks), dim3(256), 0, stream,
                       in, partials, rows, cols, chunk);
    int st = hip_error(hipGetLastError(), "colsum_partial_kernel launch");
    if (st) return st;
    // pass 2: the same kernel over the [chunks, cols] partials, one chunk
    hipLaunchKernelGGL(colsum_partial_kernel<T>, dim3(gx, 1u), dim3(256), 0, stream,
                       partials, out, chunks, cols, chunks);
    return hip_error(hipGetLastError(), "colsum_partial_kernel launch");
}

int launch_colsum_f32(const float* in, float* out, int64_t rows, int64_t cols,
                      float* partials, int64_t partial_rows, hipStream_t stream) {
    return colsum_t(in, out, rows, cols, partials, partial_rows, stream);
}

int launch_colsum_f64(const double* in, double* out, int64_t rows, int64_t cols,
                      double* partials, int64_t partial_rows, hipStream_t stream) {
    return colsum_t(in, out, rows, cols, partials, partial_rows, stream);
}

template <typename T>
int bias_row_t(const T* m, const T* row, T* out, int64_t rows, int64_t cols, hipStream_t stream) {
    if (rows * cols == 0) return CDX_OK;
    hipLaunchKernelGGL(bias_row_kernel<T>, dim3(grid_for(rows * cols)), dim3(256), 0, stream,
                       m, row, out, rows, cols);
    return hip_error(hipGetLastError(), "bias_row_kernel launch");
}

int launch_broadcast_add_row_f32(const float* m, const float* row, float* out,
                                 int64_t rows, int64_t cols, hipStream_t stream) {
    return bias_row_t(m, row, out, rows, cols, stream);
}

int launch_broadcast_add_row_f64(const double* m, const double* row, double* out,
                                 int64_t rows, int64_t cols, hipStream_t stream) {
    return bias_row_t(m, row, out, rows, cols, stream);
}

inline bool vec4_ok(int64_t n, const void* a, const void* b, const void* c = nullptr) {
    return n % 4 == 0 && (uintptr_t)a % 16 == 0 && (uintptr_t)b % 16 == 0 &&
           (uintptr_t)c % 16 == 0;
}

template <typename T>
int act_t(const T* in, T* out, int64_t n, int act, float alpha, hipStream_t stream) {
    if (n == 0) return CDX_OK;
    if constexpr (std::is_same_v<T, float>) {
        if (vec4_ok(n, in, out)) {
            hipLaunchKernelGGL(act_fwd_vec4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, stream,
                               reinterpret_cast<const floatx4*>(in),
                               reinterpret_cast<floatx4*>(out), n / 4, act, alpha);
            return hip_error(hipGetLastError(), "act_fwd_vec4_kernel launch");
        }
    }
    hipLaunchKernelGGL(act_fwd_kernel<T>, dim3(grid_for(n)), dim3(256), 0, stream, in, out, n, act,
                       alpha);
    return hip_error(hipGetLastError(), "act_fwd_kernel launch");
}

template <typename T>
int act_bwd_t(const T* go, const T* in, T* gi, int64_t n, int act, float alpha,
              hipStream_t stream) {
    if (n == 0) return CDX_OK;
    if constexpr (std::is_same_v<T, float>) {
        if (vec4_ok(n, go, in, gi)) {
            hipLaunchKernelGGL(act_bwd_vec4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, stream,
                               reinterpret_cast<const floatx4*>(go),
                               reinterpret_cast<const floatx4*>(in),
                               reinterpret_cast<floatx4*>(gi), n / 4, act, alpha);
            return hip_error(hipGetLastError(), "act_bwd_vec4_kernel launch");
        }
    }
    hipLaunchKernelGGL(act_bwd_kernel<T>, dim3(grid_for(n)), dim3(256), 0, stream, go, in, gi, n,
                       act, alpha);
    return hip_error(hipGetLastError(), "act_bwd_kernel launch");
}

int launch_activation_f32(const float* in, float* out, int64_t n, int act, float alpha,
                          hipStream_t stream) {
    return act_t(in, out, n, act, alpha, stream);
}

int launch_activation_f64(const double* in, double* out, int64_t n, int act, float alpha,
                          hipStream_t stream) {
    return act_t(in, out, n, act, alpha, stream);
}

int launch_activation_backward_f32(const float* go, const float* in, float* gi, int64_t n,
                                   int act, float alpha, hipStream_t stream) {
    return act_bwd_t(go, in, gi, n, act, alpha, stream);
}

int launch_activation_backward_f64(const double* go, const double* in, double* gi, int64_t n,
                                   int act, float alpha, hipStream_t stream) {
    return act_bwd_t(go, in, gi, n, act, alpha, stream);
}

}  // namespace cdx
