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
//    thread computes (oh, ow) of its output pixels once and for every
//    (kh, kw) gathers from LDS and stores, consecutive lanes on consecutive
//    pixels.  HBM traffic is the compulsory minimum: the input once plus
//    the column buffer once.
//  * generic kernel (larger planes): one thread per 4 consecutive s of one
//    (k, b) row, gathering straight from global memory.
// Index math is 32-bit where the value is bounded by one plane or one row
// (s < spatial, k < K_col) and both bounds fit 32 bits (the generic kernel
// switches to 64-bit arithmetic otherwise); flat offsets are 64-bit, so
// results agree with the reference wherever its int indices do not overflow
// and stay correct beyond that.
#include "cdx_internal.hpp"

namespace cdx {
namespace {

struct Im2colGeom {
    int64_t batch, IC, IH, IW, KH, KW, SH, SW, PH, PW, OH, OW, spatial, runs;
};

// IDX: the integer type of the per-element index arithmetic -- int where the
// output plane (spatial) and the column count K_col fit 32 bits (the
// launcher checks), int64_t otherwise.
template <int VS, typename IDX>
__global__ __launch_bounds__(256)
void im2col_kernel(const float* __restrict__ in, float* __restrict__ col, Im2colGeom g) {
    const int64_t per_run = (g.spatial + VS - 1) / VS;
    const int64_t total = g.runs * per_run;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t run = t / per_run;               // run = k * batch + b
        const IDX s0 = (IDX)(t - run * per_run) * VS;
        const int64_t b = run % g.batch;
        const IDX k = (IDX)(run / g.batch);
        const IDX kw = k % (IDX)g.KW;
        const IDX kh = (k / (IDX)g.KW) % (IDX)g.KH;
        const IDX ic = k / (IDX)(g.KW * g.KH);
        const float* plane = in + (b * g.IC + ic) * g.IH * g.IW;
        float v[VS];
#pragma unroll
        for (int e = 0; e < VS; ++e) {
            const IDX s = s0 + e;
            const IDX oh = s / (IDX)g.OW, ow = s % (IDX)g.OW;
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

// One workgroup per (b, ic) input plane and chunk of `chunk_rows` output
// rows (blockIdx.y), with the input rows that chunk reads staged in LDS.
// Lanes walk consecutive output pixels s (a thread owns s, s + 256, ... U at
// a time), so each LDS gather of a wavefront reads consecutive words --
// conflict-free except where a row of the output wraps -- and each store
// instruction of a wavefront writes 256 contiguous bytes of a column row.
// (Four consecutive s per thread with 16-byte stores made every gather a
// 4-way bank conflict: lanes 16 apart read words 64 apart.)  Splitting the
// planes into row chunks gives several workgroups per CU at different
// phases, so one stages its rows while others store (C5: 4 chunks of 14
// rows: 44.0 -> 42.7 us on one box).
template <int U>
__global__ __launch_bounds__(256)
void im2col_plane_kernel(const float* __restrict__ in, float* __restrict__ col, Im2colGeom g,
                         int chunk_rows) {
    extern __shared__ float rows[];
    const int64_t bc = blockIdx.x;                  // b * IC + ic
    const int b = (int)(bc / g.IC), ic = (int)(bc % g.IC);
    const int IH = (int)g.IH, IW = (int)g.IW, OW = (int)g.OW;
    const int SH = (int)g.SH, PH = (int)g.PH;
    const int KH = (int)g.KH, KW = (int)g.KW;
    const int oh0 = (int)blockIdx.y * chunk_rows;
    const int oh1 = oh0 + chunk_rows < (int)g.OH ? oh0 + chunk_rows : (int)g.OH;
    // input rows [ih_lo, ih_lo + nrows) feed output rows [oh0, oh1)
    const int ih_lo = oh0 * SH - PH, nrows = (oh1 - oh0 - 1) * SH + KH;
    const float* src = in + bc * (int64_t)IH * IW;
    for (int i = threadIdx.x; i < nrows * IW; i += blockDim.x) {
        const int ih = ih_lo + i / IW;
        rows[i] = ih >= 0 && ih < IH ? src[(int64_t)ih * IW + i % IW] : 0.0f;
    }
    __syncthreads();

    const int s_beg = oh0 * OW, s_end = oh1 * OW;
    // row (k, b) starts at ((ic*KH*KW + kk) * batch + b) * spatial
    float* row0 = col + ((int64_t)ic * KH * KW * g.batch + b) * g.spatial;
    const int64_t row_step = g.batch * g.spatial;   // next kk
    for (int s0 = s_beg + threadIdx.x; s0 < s_end; s0 += 256 * U) {
        int r0[U], iw0[U];
        bool live[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + 256 * u;
            live[u] = s < s_end;
            const int oh = s / OW, ow = s - oh * OW;
            r0[u] = live[u] ? (oh - oh0) * SH : 0;     // LDS row of kh = 0 (in range for idle lanes)
            iw0[u] = ow * (int)g.SW - (int)g.PW;
        }
        float* dst = row0 + s0;
        for (int kh = 0; kh < KH; ++kh) {
            for (int kw = 0; kw < KW; ++kw) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int iw = iw0[u] + kw;
                    const float v = iw >= 0 && iw < IW ? rows[(r0[u] + kh) * IW + iw] : 0.0f;
                    if (live[u]) dst[256 * u] = v;
                }
                dst += row_step;
            }
        }
    }
}

// col2im gather, bit-exact with the reference's col2im_kernel
// (src/kernels/conv_kernel.cu:344-380): one thread per input element,
// fp32 sum over kh (outer) then kw (inner), both ascending, starting from
// 0, of every column entry that element was copied to.
//
// Fast form (every index below 2^31, stride 1): 32-bit index arithmetic
// and no division per tap -- the 64-bit form spends most of its time in
// integer division.
__global__ __launch_bounds__(256)
void col2im_s1_kernel32(const float* __restrict__ col, float* __restrict__ grad_in,
                        Im2colGeom g) {
    const uint32_t IW = (uint32_t)g.IW, IH = (uint32_t)g.IH, IC = (uint32_t)g.IC;
    const uint32_t KH = (uint32_t)g.KH, KW = (uint32_t)g.KW, OW = (uint32_t)g.OW;
    const int32_t OH = (int32_t)g.OH, OWs = (int32_t)g.OW;
    const int32_t PH = (int32_t)g.PH, PW = (int32_t)g.PW;
    const uint32_t spatial = (uint32_t)g.spatial, BS = (uint32_t)(g.batch * g.spatial);
    const uint32_t total = (uint32_t)(g.batch * g.IC * g.IH * g.IW);
    for (uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += gridDim.x * blockDim.x) {
        const uint32_t iw = idx % IW, t1 = idx / IW;
        const uint32_t ih = t1 % IH, t2 = t1 / IH;
        const uint32_t ic = t2 % IC, b = t2 / IC;
        const float* cb = col + b * spatial;
        float acc = 0.0f;
        for (uint32_t kh = 0; kh < KH; ++kh) {
            const int32_t oh = (int32_t)ih + PH - (int32_t)kh;
            if (oh < 0 || oh >= OH) continue;
            const float* crow = cb + (ic * KH + kh) * KW * BS + (uint32_t)oh * OW;
            for (uint32_t kw = 0; kw < KW; ++kw) {
                const int32_t ow = (int32_t)iw + PW - (int32_t)kw;
                if (ow < 0 || ow >= OWs) continue;
                acc += crow[kw * BS + (uint32_t)ow];
            }
        }
        grad_in[idx] = acc;
    }
}

__global__ __launch_bounds__(256)
void col2im_kernel(const float* __restrict__ col, float* __restrict__ grad_in, Im2colGeom g) {
    const int64_t total = g.batch * g.IC * g.IH * g.IW;
    const int64_t B_spatial = g.batch * g.spatial;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t iw = idx % g.IW;
        const int64_t ih = (idx / g.IW) % g.IH;
        const int64_t ic = (idx / (g.IW * g.IH)) % g.IC;
        const int64_t b = idx / (g.IW * g.IH * g.IC);
        float acc = 0.0f;
        for (int64_t kh = 0; kh < g.KH; ++kh) {
            const int64_t oh_num = ih + g.PH - kh;
            if (oh_num < 0 || oh_num % g.SH != 0) continue;
            const int64_t oh = oh_num / g.SH;
            if (oh >= g.OH) continue;
            for (int64_t kw = 0; kw < g.KW; ++kw) {
                const int64_t ow_num = iw + g.PW - kw;
                if (ow_num < 0 || ow_num % g.SW != 0) continue;
                const int64_t ow = ow_num / g.SW;
                if (ow >= g.OW) continue;
                const int64_t k = (ic * g.KH + kh) * g.KW + kw;
                acc += col[k * B_spatial + b * g.spatial + oh * g.OW + ow];
            }
        }
        grad_in[idx] = acc;
    }
}

// [B, C, S] -> [C, B*S] (NCHW grad_output to the GEMM's channel-major
// matrix), conv_kernel.cu:383-399: a copy of B*C contiguous planes of S
// floats, plane (b, c) -> dst + c*B*S + b*S.  blockIdx.y = plane, 16-byte
// copies when S % 4 == 0 and both bases are 16-byte aligned.
__global__ __launch_bounds__(256)
void nchw_to_cm_planes_kernel(const float* __restrict__ src, float* __restrict__ dst,
                              int64_t batch, int64_t C, int64_t S, int vec) {
    const int64_t plane = blockIdx.y;
    const int64_t b = plane / C, c = plane - b * C;
    const float* sp = src + plane * S;
    float* dp = dst + (c * batch + b) * S;
    if (vec) {
        const int64_t n4 = S / 4;
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
             i += (int64_t)gridDim.x * blockDim.x)
            reinterpret_cast<float4*>(dp)[i] = reinterpret_cast<const float4*>(sp)[i];
    } else {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < S;
             i += (int64_t)gridDim.x * blockDim.x)
            dp[i] = sp[i];
    }
}

__global__ __launch_bounds__(256)
void nchw_to_cm_kernel(const float* __restrict__ src, float* __restrict__ dst,
                       int64_t batch, int64_t C, int64_t S) {
    const int64_t BS = batch * S, total = C * BS;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t c = i / BS, bs = i - c * BS;
        const int64_t b = bs / S, s = bs - b * S;
        dst[i] = src[(b * C + c) * S + s];
    }
}

// db[c] = sum over b, s of dy[b, c, s]: one 1024-thread workgroup per
// channel, 16-byte loads where the planes allow, a fixed per-thread order
// then a fixed LDS tree -- deterministic.  Replaces the host-side NumPy sum
// of the reference's Conv2dOp (python/cuDeep/tensor.py:718-721).
constexpr int kBiasThreads = 1024;

__global__ __launch_bounds__(kBiasThreads)
void conv_bias_grad_kernel(const float* __restrict__ dy, float* __restrict__ db,
                           int64_t batch, int64_t C, int64_t S, int vec) {
    __shared__ float red[kBiasThreads];
    const int64_t c = blockIdx.x;
    const int t = threadIdx.x;
    float acc = 0.0f;
    if (vec) {
        // this thread's float4 slots of every plane, 4 planes' loads in flight
        // at a time, summed in (plane, slot) order
        const int64_t n4 = S / 4;
        const int64_t cs = C * S;
        for (int64_t i = t; i < n4; i += kBiasThreads) {
            const float4* p4 = reinterpret_cast<const float4*>(dy + c * S) + i;
            int64_t b = 0;
            for (; b + 3 < batch; b += 4) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = *(const float4*)((const float*)p4 + (b + u) * cs);
#pragma unroll
                for (int u = 0; u < 4; ++u) acc += ((v[u].x + v[u].y) + v[u].z) + v[u].w;
            }
            for (; b < batch; ++b) {
                const float4 v = *(const float4*)((const float*)p4 + b * cs);
                acc += ((v.x + v.y) + v.z) + v.w;
            }
        }
    } else {
        for (int64_t b = 0; b < batch; ++b) {
            const float* plane = dy + (b * C + c) * S;
            for (int64_t s = t; s < S; s += kBiasThreads) acc += plane[s];
        }
    }
    red[t] = acc;
    __syncthreads();
    for (int w = kBiasThreads / 2; w > 0; w >>= 1) {
        if (t < w) red[t] += red[t + w];
        __syncthreads();
    }
    if (t == 0) db[c] = red[0];
}

// wf[ic, oc, k'] = w[oc, ic, KHW-1-k']: the filter of the stride-1
// transposed convolution (channels swapped, both spatial axes reversed; the
// flattened kh*KW+kw index reverses as a whole).
__global__ __launch_bounds__(256)
void flip_filter_kernel(const float* __restrict__ w, float* __restrict__ wf, int64_t OC,
                        int64_t IC, int64_t KHW) {
    const int64_t total = OC * IC * KHW;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = i % KHW, p = i / KHW;      // p = oc * IC + ic
        const int64_t oc = p / IC, ic = p - oc * IC;
        wf[(ic * OC + oc) * KHW + (KHW - 1 - k)] = w[i];
    }
}

unsigned grid_for(int64_t n) {
    int64_t b = ceil_div(n, 256);
    if (b > 65536) b = 65536;
    if (b < 1) b = 1;
    return (unsigned)b;
}

Im2colGeom make_geom(int64_t batch, int64_t IC, int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                     int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    Im2colGeom g;
    g.batch = batch; g.IC = IC; g.IH = IH; g.IW = IW; g.KH = KH; g.KW = KW;
    g.SH = SH; g.SW = SW; g.PH = PH; g.PW = PW;
    g.OH = (IH + 2 * PH - KH) / SH + 1;
    g.OW = (IW + 2 * PW - KW) / SW + 1;
    g.spatial = g.OH * g.OW;
    g.runs = IC * KH * KW * batch;
    return g;
}

}  // namespace

int launch_col2im_f32(const float* col, float* grad_in, int64_t batch, int64_t IC,
                      int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                      int64_t SH, int64_t SW, int64_t PH, int64_t PW, hipStream_t stream) {
    Im2colGeom g = make_geom(batch, IC, IH, IW, KH, KW, SH, SW, PH, PW);
    const int64_t total = batch * IC * IH * IW;
    if (total == 0) return CDX_OK;
    const bool fits32 = total < ((int64_t)1 << 31) &&
                        g.IC * g.KH * g.KW * g.batch * g.spatial < ((int64_t)1 << 31);
    if (fits32 && g.SH == 1 && g.SW == 1) {
        hipLaunchKernelGGL(col2im_s1_kernel32, dim3(grid_for(total)), dim3(256), 0, stream, col,
                           grad_in, g);
        return hip_error(hipGetLastError(), "col2im_s1_kernel32 launch");
    }
    hipLaunchKernelGGL(col2im_kernel, dim3(grid_for(total)), dim3(256), 0, stream, col, grad_in, g);
    return hip_error(hipGetLastError(), "col2im_kernel launch");
}

int launch_nchw_to_cm_f32(const float* src, float* dst, int64_t batch, int64_t C, int64_t S,
                          hipStream_t stream) {
    const int64_t total = batch * C * S;
    if (total == 0) return CDX_OK;
    if (batch * C <= 65535) {
        const int vec = S % 4 == 0 && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0;
        const int64_t per = vec ? S / 4 : S;
        int64_t gx = ceil_div(per, 256);
        if (gx > 64) gx = 64;
        hipLaunchKernelGGL(nchw_to_cm_planes_kernel, dim3((unsigned)gx, (unsigned)(batch * C)),
                           dim3(256), 0, stream, src, dst, batch, C, S, vec);
        return hip_error(hipGetLastError(), "nchw_to_cm_planes_kernel launch");
    }
    hipLaunchKernelGGL(nchw_to_cm_kernel, dim3(grid_for(total)), dim3(256), 0, stream,
                       src, dst, batch, C, S);
    return hip_error(hipGetLastError(), "nchw_to_cm_kernel launch");
}

int launch_flip_filter_f32(const float* w, float* wf, int64_t OC, int64_t IC, int64_t KHW,
                           hipStream_t stream) {
    const int64_t total = OC * IC * KHW;
    if (total == 0) return CDX_OK;
    hipLaunchKernelGGL(flip_filter_kernel, dim3(grid_for(total)), dim3(256), 0, stream, w, wf,
                       OC, IC, KHW);
    return hip_error(hipGetLastError(), "flip_filter_kernel launch");
}

int launch_conv_bias_grad_f32(const float* dy, float* db, int64_t batch, int64_t C, int64_t S,
                              hipStream_t stream) {
    if (C == 0) return CDX_OK;
    if (C > INT32_MAX) return set_error(CDX_ERR_UNSUPPORTED, "conv bias grad: too many channels");
    const int vec = S % 4 == 0 && (uintptr_t)dy % 16 == 0;
    hipLaunchKernelGGL(conv_bias_grad_kernel, dim3((unsigned)C), dim3(kBiasThreads), 0, stream,
                       dy, db, batch, C, S, vec);
    return hip_error(hipGetLastError(), "conv_bias_grad_kernel launch");
}

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
    // Row chunks of ~1024 output pixels (at least one output row each).
    const int64_t chunk_rows = std::max<int64_t>(1, std::min<int64_t>(g.OH, ceil_div(1024, g.OW)));
    const int64_t chunks = ceil_div(g.OH, chunk_rows);
    const int64_t chunk_in_rows = (chunk_rows - 1) * SH + KH;
    // (the plane kernel's row and column origins oh*SH - PH, ow*SW - PW + kw
    // are int: strides and paddings beyond that take the 64-bit kernel)
    if (chunk_in_rows * IW <= kPlaneMaxFloats && batch * IC <= INT32_MAX &&
        g.spatial + 1024 <= INT32_MAX && KH * KW <= 4096 && chunks <= 65535 &&
        g.OH * SH < INT32_MAX && g.OW * SW + KW < INT32_MAX && PH < INT32_MAX &&
        PW < INT32_MAX) {
        const size_t lds = (size_t)(chunk_in_rows * IW) * sizeof(float);
        hipLaunchKernelGGL(im2col_plane_kernel<4>, dim3((unsigned)(batch * IC), (unsigned)chunks),
                           dim3(256), lds, stream, in, col, g, (int)chunk_rows);
        return hip_error(hipGetLastError(), "im2col_plane_kernel launch");
    }
    const int64_t threads = g.runs * ((g.spatial + VS - 1) / VS);
    int64_t blocks = ceil_div(threads, 256);
    if (blocks > (int64_t)1 << 30) blocks = (int64_t)1 << 30;
    const bool narrow = g.spatial + 4 <= INT32_MAX && IC * KH * KW <= INT32_MAX;
    if (narrow && vec)
        hipLaunchKernelGGL((im2col_kernel<4, int>), dim3((unsigned)blocks), dim3(256), 0, stream, in, col, g);
    else if (narrow)
        hipLaunchKernelGGL((im2col_kernel<1, int>), dim3((unsigned)blocks), dim3(256), 0, stream, in, col, g);
    else if (vec)
        hipLaunchKernelGGL((im2col_kernel<4, int64_t>), dim3((unsigned)blocks), dim3(256), 0, stream, in, col, g);
    else
        hipLaunchKernelGGL((im2col_kernel<1, int64_t>), dim3((unsigned)blocks), dim3(256), 0, stream, in, col, g);
    return hip_error(hipGetLastError(), "im2col_kernel launch");
}

}  // namespace cdx
