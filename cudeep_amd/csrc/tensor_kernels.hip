// Bandwidth kernels behind the host Tensor runtime (fp32 and fp64):
//   * strided -> contiguous copy (Tensor::contiguous), replacing
//     strided_copy_kernel (src/tensor.cu:26-68), which ships shape/strides
//     through a device allocation plus two H2D copies and a stream
//     synchronize per call.  Here the (<= 8-d) geometry travels in the
//     kernel argument block: no allocation, no copy, no synchronize.
//   * fill, elementwise add / sub / mul (Tensor factories and operators,
//     src/kernels/elementwise_kernel.cu:17-137).
//   * randn (Tensor::randn, src/tensor.cu:158-206 uses cuRAND): a
//     counter-based generator -- SplitMix64 (Steele, Lea & Flood 2014) over
//     (seed, element index) -- feeding Box-Muller, so the values are a pure
//     function of (seed, offset, index) and reproducible across launches.
//   * full sum to one scalar (Tensor.sum() in autograd graphs;
//     src/kernels/reduce_kernel.cu:21-195): per-workgroup partials in a
//     fixed order, then one workgroup adds them -- deterministic.
#include "cdx_internal.hpp"

namespace cdx {
namespace {

constexpr int kMaxDims = 8;

struct StridedGeom {
    int ndim;
    int64_t shape[kMaxDims];
    int64_t stride[kMaxDims];   // source strides, in elements
};

template <typename T>
__global__ __launch_bounds__(256)
void strided_copy_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t n, StridedGeom g) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t rem = i, off = 0;
        for (int d = g.ndim - 1; d >= 0; --d) {
            const int64_t c = rem % g.shape[d];
            rem /= g.shape[d];
            off += c * g.stride[d];
        }
        dst[i] = src[off];
    }
}

template <typename T>
__global__ __launch_bounds__(256)
void fill_kernel(T* __restrict__ y, int64_t n, T v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = v;
}

template <typename T>
__global__ __launch_bounds__(256)
void binary_kernel(const T* __restrict__ a, const T* __restrict__ b, T* __restrict__ y,
                   int64_t n, int op) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const T x = a[i], z = b[i];
        y[i] = op == CDX_BINARY_ADD ? x + z : op == CDX_BINARY_SUB ? x - z : x * z;
    }
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// uniform in (0, 1]: 53 random bits, never 0 (log is finite)
__device__ __forceinline__ double unit_open0(uint64_t bits) {
    return ((double)(bits >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

template <typename T>
__global__ __launch_bounds__(256)
void randn_kernel(T* __restrict__ y, int64_t n, uint64_t seed, uint64_t offset) {
    // pair p produces elements 2p and 2p+1 (Box-Muller cos / sin)
    const int64_t pairs = (n + 1) / 2;
    for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < pairs;
         p += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t ctr = offset + (uint64_t)p;
        const uint64_t k = splitmix64(seed ^ 0x5DEECE66Dull);
        const double u1 = unit_open0(splitmix64(k + 2 * ctr));
        const double u2 = unit_open0(splitmix64(k + 2 * ctr + 1));
        const double r = sqrt(-2.0 * log(u1));
        const double t = 6.283185307179586 * u2;
        y[2 * p] = (T)(r * cos(t));
        if (2 * p + 1 < n) y[2 * p + 1] = (T)(r * sin(t));
    }
}

constexpr int kSumBlocks = 1024;

template <typename T>
__global__ __launch_bounds__(256)
void sum_partial_kernel(const T* __restrict__ x, T* __restrict__ part, int64_t n) {
    __shared__ T red[256];
    T acc = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        acc += x[i];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

template <typename T>
__global__ __launch_bounds__(256)
void sum_final_kernel(const T* __restrict__ part, T* __restrict__ out, int nparts) {
    __shared__ T red[256];
    T acc = 0;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) acc += part[i];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = red[0];
}

unsigned grid_for(int64_t n) {
    int64_t b = ceil_div(n, 256);
    if (b > 65536) b = 65536;
    if (b < 1) b = 1;
    return (unsigned)b;
}

}  // namespace

int launch_strided_copy(const void* src, void* dst, int ndim, const int64_t* shape,
                        const int64_t* strides, int dtype, hipStream_t stream) {
    StridedGeom g{};
    g.ndim = ndim;
    int64_t n = 1;
    for (int d = 0; d < ndim; ++d) {
        g.shape[d] = shape[d];
        g.stride[d] = strides[d];
        n *= shape[d];
    }
    if (n == 0) return CDX_OK;
    if (dtype == CDX_DTYPE_F32)
        hipLaunchKernelGGL(strided_copy_kernel<float>, dim3(grid_for(n)), dim3(256), 0, stream,
                           static_cast<const float*>(src), static_cast<float*>(dst), n, g);
    else
        hipLaunchKernelGGL(strided_copy_kernel<double>, dim3(grid_for(n)), dim3(256), 0, stream,
                           static_cast<const double*>(src), static_cast<double*>(dst), n, g);
    return hip_error(hipGetLastError(), "strided_copy_kernel launch");
}

int launch_fill(void* dst, int64_t n, double v, int dtype, hipStream_t stream) {
    if (n == 0) return CDX_OK;
    if (dtype == CDX_DTYPE_F32)
        hipLaunchKernelGGL(fill_kernel<float>, dim3(grid_for(n)), dim3(256), 0, stream,
                           static_cast<float*>(dst), n, (float)v);
    else
        hipLaunchKernelGGL(fill_kernel<double>, dim3(grid_for(n)), dim3(256), 0, stream,
                           static_cast<double*>(dst), n, v);
    return hip_error(hipGetLastError(), "fill_kernel launch");
}

int launch_binary(int op, int dtype, const void* a, const void* b, void* y, int64_t n,
                  hipStream_t stream) {
    if (n == 0) return CDX_OK;
    if (dtype == CDX_DTYPE_F32)
        hipLaunchKernelGGL(binary_kernel<float>, dim3(grid_for(n)), dim3(256), 0, stream,
                           static_cast<const float*>(a), static_cast<const float*>(b),
                           static_cast<float*>(y), n, op);
    else
        hipLaunchKernelGGL(binary_kernel<double>, dim3(grid_for(n)), dim3(256), 0, stream,
                           static_cast<const double*>(a), static_cast<const double*>(b),
                           static_cast<double*>(y), n, op);
    return hip_error(hipGetLastError(), "binary_kernel launch");
}

int launch_randn(void* dst, int64_t n, int dtype, uint64_t seed, uint64_t offset,
                 hipStream_t stream) {
    if (n == 0) return CDX_OK;
    const int64_t pairs = (n + 1) / 2;
    if (dtype == CDX_DTYPE_F32)
        hipLaunchKernelGGL(randn_kernel<float>, dim3(grid_for(pairs)), dim3(256), 0, stream,
                           static_cast<float*>(dst), n, seed, offset);
    else
        hipLaunchKernelGGL(randn_kernel<double>, dim3(grid_for(pairs)), dim3(256), 0, stream,
                           static_cast<double*>(dst), n, seed, offset);
    return hip_error(hipGetLastError(), "randn_kernel launch");
}

int64_t sum_partials() { return kSumBlocks; }

int launch_sum(const void* x, void* out, int64_t n, int dtype, void* partials,
               hipStream_t stream) {
    if (n == 0) return launch_fill(out, 1, 0.0, dtype, stream);
    int64_t nb = ceil_div(n, 256);
    if (nb > kSumBlocks) nb = kSumBlocks;
    if (dtype == CDX_DTYPE_F32) {
        hipLaunchKernelGGL(sum_partial_kernel<float>, dim3((unsigned)nb), dim3(256), 0, stream,
                           static_cast<const float*>(x), static_cast<float*>(partials), n);
        hipLaunchKernelGGL(sum_final_kernel<float>, dim3(1), dim3(256), 0, stream,
                           static_cast<const float*>(partials), static_cast<float*>(out), (int)nb);
    } else {
        hipLaunchKernelGGL(sum_partial_kernel<double>, dim3((unsigned)nb), dim3(256), 0, stream,
                           static_cast<const double*>(x), static_cast<double*>(partials), n);
        hipLaunchKernelGGL(sum_final_kernel<double>, dim3(1), dim3(256), 0, stream,
                           static_cast<const double*>(partials), static_cast<double*>(out), (int)nb);
    }
    return hip_error(hipGetLastError(), "sum kernels launch");
}

}  // namespace cdx
