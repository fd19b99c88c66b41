// im2col gather for gfx950, bit-exact with the reference's im2col_kernel
// (src/kernels/conv_kernel.cu:32-65):
//   col[k * B_spatial + b * spatial + s] = input[b, ic, ih, iw]  or 0,
//   k = (ic*KH + kh)*KW + kw,  s = oh*OW + ow,
//   ih = oh*SH - PH + kh,  iw = ow*SW - PW + kw.
//
// Since k * B_spatial + b * spatial + s == (k * batch + b) * spatial + s,
// the column buffer is one flat sequence of rows (k, b), each `spatial`
// long.  Two kernels:
//  * plane kernel (input plane <= 64 KiB): one workgroup per (b, ic) input
//    plane.  The plane is read from HBM once, coalesced, into LDS; the
//    workgroup then writes the KH*KW column rows that plane feeds.  Each
//    thread owns 4 consecutive s, computes (oh, ow) once, and for every
//    (kh, kw) gathers from LDS and issues one 16-byte store, so every
//    wavefront writes 1 KiB contiguous runs.  HBM traffic is the
//    compulsory minimum: the input once plus the column buffer once.
//  * generic kernel (larger planes): one thread per 4 consecutive s of one
//    (k, b) row, gathering straight from global memory.
// Index math is 32-bit where the value is bounded by one plane or one row
// (s < spatial, k < K_col); flat offsets are 64-bit, so results agree with
// the reference wherever its int indices do not overflow and stay correct
// beyond that.
#include "cdx_internal.hpp"

namespace cdx {
namespace {

struct Im2colGeom {
    int64_t batch, IC, IH, IW, KH, KW, SH, SW, PH, PW, OH, OW, spatial, runs;
};

template <int VS>
__global__ __launch_bounds__(256)
void im2col_kernel(const float* __restrict__ in, float* __restrict__ col, Im2colGeom g) {
    const int64_t per_run = (g.spatial + VS - 1) / VS;
    const int64_t total = g.runs * per_run;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t run = t / per_run;               // run = k * batch + b
        const int s0 = (int)(t - run * per_run) * VS;
        const int b = (int)(run % g.batch);
        const int k = (int)(run / g.batch);
        const int kw = k % (int)g.KW;
        const int kh = (k / (int)g.KW) % (int)g.KH;
        const int ic = k / (int)(g.KW * g.KH);
        const float* plane = in + ((int64_t)b * g.IC + ic) * g.IH * g.IW;
        float v[VS];
#pragma unroll
        for (int e = 0; e < VS; ++e) {
            const int s = s0 + e;
            const int oh = s / (int)g.OW, ow = s % (int)g.OW;
            const int64_t ih = (int64_t)oh * g.SH - g.PH + kh;
            const int64_t iw = (int64_t)ow * g.SW - g.PW + kw;
            v[e] = (s < g.spatial && ih >= 0 && ih < g.IH && iw >= 0 && iw < g.IW)
                       ? plane[ih * g.IW + iw] : 0.0f;
        }
        float* dst = col + run * g.spatial + s0;
        if (VS == 4) {
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
            for (int e = 0; e < VS; ++e)
                if (s0 + e < g.spatial) dst[e] = v[e];
        }
    }
}

constexpr int kPlaneMaxFloats = 16384;   // 64 KiB of LDS per input plane

template <int VS>
__global__ __launch_bounds__(256)
void im2col_plane_kernel(const float* __restrict__ in, float* __restrict__ col, Im2colGeom g) {
    extern __shared__ float plane[];
    const int64_t bc = blockIdx.x;                  // b * IC + ic
    const int b = (int)(bc / g.IC), ic = (int)(bc % g.IC);
    const int IH = (int)g.IH, IW = (int)g.IW, plane_n = IH * IW;
    const float* src = in + bc * (int64_t)plane_n;
    for (int i = threadIdx.x; i < plane_n; i += blockDim.x) plane[i] = src[i];
    __syncthreads();

    const int spatial = (int)g.spatial, OW = (int)g.OW;
    const int KH = (int)g.KH, KW = (int)g.KW;
    const int runs_per_row = (spatial + VS - 1) / VS;
    // row (k, b) starts at ((ic*KH*KW + kk) * batch + b) * spatial
    float* row0 = col + ((int64_t)ic * KH * KW * g.batch + b) * g.spatial;
    const int64_t row_step = g.batch * g.spatial;   // next kk
    for (int t = threadIdx.x; t < runs_per_row; t += blockDim.x) {
        const int s0 = t * VS;
        int ih0[VS], iw0[VS];
#pragma unroll
        for (int e = 0; e < VS; ++e) {
            const int s = s0 + e < spatial ? s0 + e : spatial - 1;
            const int oh = s / OW, ow = s - (s / OW) * OW;
            ih0[e] = oh * (int)g.SH - (int)g.PH;
            iw0[e] = ow * (int)g.SW - (int)g.PW;
        }
        float* dst = row0 + s0;
        for (int kh = 0; kh < KH; ++kh) {
            for (int kw = 0; kw < KW; ++kw) {
                float v[VS];
#pragma unroll
                for (int e = 0; e < VS; ++e) {
                    const int ih = ih0[e] + kh, iw = iw0[e] + kw;
                    v[e] = (ih >= 0 && ih < IH && iw >= 0 && iw < IW) ? plane[ih * IW + iw] : 0.0f;
                }
                if (VS == 4) {
                    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int e = 0; e < VS; ++e)
                        if (s0 + e < spatial) dst[e] = v[e];
                }
                dst += row_step;
            }
        }
    }
}

}  // namespace

int launch_im2col_f32(const float* in, float* col, int64_t batch, int64_t IC,
                      int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                      int64_t SH, int64_t SW, int64_t PH, int64_t PW,
                      hipStream_t stream) {
    Im2colGeom g;
    g.batch = batch; g.IC = IC; g.IH = IH; g.IW = IW; g.KH = KH; g.KW = KW;
    g.SH = SH; g.SW = SW; g.PH = PH; g.PW = PW;
    g.OH = (IH + 2 * PH - KH) / SH + 1;
    g.OW = (IW + 2 * PW - KW) / SW + 1;
    g.spatial = g.OH * g.OW;
    g.runs = IC * KH * KW * batch;
    if (g.spatial <= 0 || g.runs <= 0) return CDX_OK;
    // 16-byte stores need every run to start 16-byte aligned.
    const bool vec = g.spatial % 4 == 0 && (uintptr_t)col % 16 == 0;
    const int VS = vec ? 4 : 1;
    if (IH * IW <= kPlaneMaxFloats && batch * IC <= INT32_MAX && g.spatial <= INT32_MAX &&
        KH * KW <= 4096) {
        const size_t lds = (size_t)(IH * IW) * sizeof(float);
        if (vec)
            hipLaunchKernelGGL(im2col_plane_kernel<4>, dim3((unsigned)(batch * IC)), dim3(256),
                               lds, stream, in, col, g);
        else
            hipLaunchKernelGGL(im2col_plane_kernel<1>, dim3((unsigned)(batch * IC)), dim3(256),
                               lds, stream, in, col, g);
        return hip_error(hipGetLastError(), "im2col_plane_kernel launch");
    }
    const int64_t threads = g.runs * ((g.spatial + VS - 1) / VS);
    int64_t blocks = ceil_div(threads, 256);
    if (blocks > (int64_t)1 << 30) blocks = (int64_t)1 << 30;
    if (vec)
        hipLaunchKernelGGL(im2col_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, stream, in, col, g);
    else
        hipLaunchKernelGGL(im2col_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, stream, in, col, g);
    return hip_error(hipGetLastError(), "im2col_kernel launch");
}

}  // namespace cdx
