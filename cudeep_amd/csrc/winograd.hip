// Winograd F(4x4, 3x3) convolution for 3x3 stride-1 layers on gfx950: the
// reference's route for that case (src/kernels/conv_kernel.cu:242-248,
// :557-789).  Transform matrices are those of Lavin & Gray (2016) for the
// interpolation points 0, +-1, +-2 (G for the filter, B^T for the input,
// A^T for the output); each 2-D transform applies the 1-D one to the
// columns and then to the rows, as the reference does.
//
// Data flow (all in the caller's workspace):
//   U [36][OC][IC]     filter transform, one thread per (oc, ic)
//   V [36][IC][tiles]  input transform of every zero-padded 6x6 patch
//                      (stride 4), one thread per (ic, tile); tile index
//                      = (b * TH + th) * TW + tw, contiguous across a wave
//   M [36][OC][tiles]  one batched MFMA GEMM (36 problems OC x tiles x IC,
//                      blockIdx.z = point) through the library's GEMM
//   Y (NCHW)           output transform + bias, one thread per (oc, tile),
//                      16-byte stores of the 4-wide output rows where the
//                      tile is whole and aligned.
// Backward data of a 3x3 stride-1 layer runs the same pipeline on the
// transposed convolution (grad_output in, the filter read channel-swapped
// and spatially reversed by the filter transform, padding 2 - P).
// Compared with im2col + GEMM this moves ~2.3x fewer HBM bytes at C5
// (V and M are 36/16 of the input / output size, against the 9x im2col
// buffer) and does 4x fewer multiplies in the GEMM.
#include <type_traits>

#include "cdx_internal.hpp"

namespace cdx {
namespace {

struct WinoGeom {
    int64_t B, IC, OC, IH, IW, PH, PW, OH, OW, TH, TW, NT;
    int vec_out;   // output rows may take 16-byte stores (aligned base, OW % 4 == 0)
};

// 1-D filter transform (rows of G applied to g0..g2)
__device__ __forceinline__ void wino_g(float g0, float g1, float g2, float* u) {
    u[0] = 0.25f * g0;
    u[1] = -(1.0f / 6.0f) * (g0 + g1 + g2);
    u[2] = -(1.0f / 6.0f) * (g0 - g1 + g2);
    u[3] = (1.0f / 24.0f) * g0 + (1.0f / 12.0f) * g1 + (1.0f / 6.0f) * g2;
    u[4] = (1.0f / 24.0f) * g0 - (1.0f / 12.0f) * g1 + (1.0f / 6.0f) * g2;
    u[5] = g2;
}

// 1-D input transform (rows of B^T applied to d0..d5)
__device__ __forceinline__ void wino_bt(const float* d, float* t) {
    t[0] = 4.0f * d[0] - 5.0f * d[2] + d[4];
    t[1] = -4.0f * d[1] - 4.0f * d[2] + d[3] + d[4];
    t[2] = 4.0f * d[1] - 4.0f * d[2] - d[3] + d[4];
    t[3] = -2.0f * d[1] - d[2] + 2.0f * d[3] + d[4];
    t[4] = 2.0f * d[1] - d[2] - 2.0f * d[3] + d[4];
    t[5] = 4.0f * d[1] - 5.0f * d[3] + d[5];
}

// 1-D output transform (rows of A^T applied to m0..m5)
__device__ __forceinline__ void wino_at(const float* m, float* o) {
    o[0] = m[0] + m[1] + m[2] + m[3] + m[4];
    o[1] = m[1] - m[2] + 2.0f * m[3] - 2.0f * m[4];
    o[2] = m[1] + m[2] + 4.0f * m[3] + 4.0f * m[4];
    o[3] = m[1] - m[2] + 8.0f * m[3] - 8.0f * m[4] + m[5];
}

// FLIP: w is [IC][OC][3][3] and filter (oc, ic) is w[ic][oc] with both
// spatial axes reversed (tap t read from 8 - t): the stride-1 transposed
// convolution's filter, for backward data.
template <bool FLIP>
__device__ __forceinline__ void wino_filter_one(const float* __restrict__ w, float* __restrict__ U,
                                                int64_t OC, int64_t IC, int64_t p) {
    float g[9];
    if (FLIP) {
        const int64_t oc = p / IC, ic = p - oc * IC;
        const float* src = w + (ic * OC + oc) * 9;
#pragma unroll
        for (int t = 0; t < 9; ++t) g[t] = src[8 - t];
    } else {
#pragma unroll
        for (int t = 0; t < 9; ++t) g[t] = w[p * 9 + t];
    }
    float tmp[6][3], u[6];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        wino_g(g[j], g[3 + j], g[6 + j], u);
#pragma unroll
        for (int i = 0; i < 6; ++i) tmp[i][j] = u[i];
    }
    const int64_t plane = OC * IC;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        wino_g(tmp[i][0], tmp[i][1], tmp[i][2], u);
#pragma unroll
        for (int j = 0; j < 6; ++j) U[(i * 6 + j) * plane + p] = u[j];
    }
}

template <bool FLIP>
__global__ __launch_bounds__(256)
void wino_filter_kernel(const float* __restrict__ w, float* __restrict__ U, int64_t OC,
                        int64_t IC) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // oc * IC + ic
    if (p >= OC * IC) return;
    wino_filter_one<FLIP>(w, U, OC, IC, p);
}

__global__ __launch_bounds__(256)
void wino_input_kernel(const float* __restrict__ x, float* __restrict__ V, WinoGeom g) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // ic * NT + tile
    if (q >= g.IC * g.NT) return;
    const int64_t ic = q / g.NT, tile = q - ic * g.NT;
    const int64_t per_img = g.TH * g.TW;
    const int64_t b = tile / per_img, r = tile - b * per_img;
    const int64_t th = r / g.TW, tw = r - th * g.TW;
    const int64_t h0 = th * 4 - g.PH, w0 = tw * 4 - g.PW;
    const float* src = x + (b * g.IC + ic) * g.IH * g.IW;
    float d[6][6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int64_t ih = h0 + i;
        const bool rok = ih >= 0 && ih < g.IH;
#pragma unroll
        for (int j = 0; j < 6; ++j) {
            const int64_t iw = w0 + j;
            d[i][j] = (rok && iw >= 0 && iw < g.IW) ? src[ih * g.IW + iw] : 0.0f;
        }
    }
    float tmp[6][6], col[6], t[6];
#pragma unroll
    for (int j = 0; j < 6; ++j) {
#pragma unroll
        for (int i = 0; i < 6; ++i) col[i] = d[i][j];
        wino_bt(col, t);
#pragma unroll
        for (int i = 0; i < 6; ++i) tmp[i][j] = t[i];
    }
    const int64_t plane = g.IC * g.NT;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        wino_bt(tmp[i], t);
#pragma unroll
        for (int j = 0; j < 6; ++j) V[(i * 6 + j) * plane + q] = t[j];
    }
}

// The same transform where IW % 4 == 0, PW = 4 - SH <= 2 and the input is
// 16-byte aligned: each patch row comes from three aligned 16-byte loads of
// input columns 4 tw - 4 .. 4 tw + 7 (each wholly inside or outside the row,
// since IW % 4 == 0; consecutive lanes, whose tiles are 4 columns apart,
// read consecutive 16-byte words) instead of six 4-byte loads.  Same
// arithmetic per tile as wino_input_kernel.
template <int SH>
__device__ __forceinline__ void wino_input_v4_one(const float* __restrict__ x, float* __restrict__ V,
                                                  const WinoGeom& g, int64_t q) {
    const int64_t ic = q / g.NT, tile = q - ic * g.NT;
    const int64_t per_img = g.TH * g.TW;
    const int64_t b = tile / per_img, r = tile - b * per_img;
    const int64_t th = r / g.TW, tw = r - th * g.TW;
    const int64_t h0 = th * 4 - g.PH, a = tw * 4 - 4;   // first loaded column; w0 = a + SH
    const float* src = x + (b * g.IC + ic) * g.IH * g.IW;
    float d[6][6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int64_t ih = h0 + i;
        const bool rok = ih >= 0 && ih < g.IH;
        float row[12];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const int64_t col = a + 4 * c;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (rok && col >= 0 && col < g.IW)
                v = *reinterpret_cast<const float4*>(src + ih * g.IW + col);
            row[4 * c] = v.x; row[4 * c + 1] = v.y; row[4 * c + 2] = v.z; row[4 * c + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < 6; ++j) d[i][j] = row[SH + j];
    }
    float tmp[6][6], col6[6], t[6];
#pragma unroll
    for (int j = 0; j < 6; ++j) {
#pragma unroll
        for (int i = 0; i < 6; ++i) col6[i] = d[i][j];
        wino_bt(col6, t);
#pragma unroll
        for (int i = 0; i < 6; ++i) tmp[i][j] = t[i];
    }
    const int64_t plane = g.IC * g.NT;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        wino_bt(tmp[i], t);
#pragma unroll
        for (int j = 0; j < 6; ++j) V[(i * 6 + j) * plane + q] = t[j];
    }
}

// The filter transform rides in the same launch: workgroups [0, fblocks)
// transform the filter (independent of the input transform, and consumed
// only by the GEMM after both), the rest the input -- one launch, and the
// filter's short, latency-bound work overlaps the input transform.
template <int SH, bool FLIP>
__global__ __launch_bounds__(256)
void wino_filter_input_v4_kernel(const float* __restrict__ w, float* __restrict__ U,
                                 const float* __restrict__ x, float* __restrict__ V, WinoGeom g,
                                 int64_t fblocks) {
    if ((int64_t)blockIdx.x < fblocks) {
        const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // oc * IC + ic
        if (p < g.OC * g.IC) wino_filter_one<FLIP>(w, U, g.OC, g.IC, p);
        return;
    }
    const int64_t q = ((int64_t)blockIdx.x - fblocks) * blockDim.x + threadIdx.x;   // ic * NT + tile
    if (q < g.IC * g.NT) wino_input_v4_one<SH>(x, V, g, q);
}

__global__ __launch_bounds__(256)
void wino_output_kernel(const float* __restrict__ Mm, const float* __restrict__ bias,
                        float* __restrict__ y, WinoGeom g) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // oc * NT + tile
    if (q >= g.OC * g.NT) return;
    const int64_t oc = q / g.NT, tile = q - oc * g.NT;
    const int64_t per_img = g.TH * g.TW;
    const int64_t b = tile / per_img, r = tile - b * per_img;
    const int64_t th = r / g.TW, tw = r - th * g.TW;
    const int64_t plane = g.OC * g.NT;
    float m[6][6];
#pragma unroll
    for (int i = 0; i < 6; ++i)
#pragma unroll
        for (int j = 0; j < 6; ++j) m[i][j] = Mm[(i * 6 + j) * plane + q];
    float tmp[4][6], col[6], o[4];
#pragma unroll
    for (int j = 0; j < 6; ++j) {
#pragma unroll
        for (int i = 0; i < 6; ++i) col[i] = m[i][j];
        wino_at(col, o);
#pragma unroll
        for (int i = 0; i < 4; ++i) tmp[i][j] = o[i];
    }
    const float bv = bias ? bias[oc] : 0.0f;
    float* dst = y + (b * g.OC + oc) * g.OH * g.OW;
    const int64_t oh0 = th * 4, ow0 = tw * 4;
    const bool whole = g.vec_out && ow0 + 4 <= g.OW;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        wino_at(tmp[i], o);
        const int64_t oh = oh0 + i;
        if (oh >= g.OH) break;
        float* row = dst + oh * g.OW + ow0;
        if (whole) {
            *reinterpret_cast<float4*>(row) = make_float4(o[0] + bv, o[1] + bv, o[2] + bv, o[3] + bv);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (ow0 + j < g.OW) row[j] = o[j] + bv;
        }
    }
}

unsigned blocks_for(int64_t n) { return (unsigned)ceil_div(n, 256); }

}  // namespace

size_t winograd_workspace_floats(int64_t batch, int64_t IC, int64_t OC, int64_t OH,
                                 int64_t OW) {
    const int64_t NT = batch * ceil_div(OH, 4) * ceil_div(OW, 4);
    return (size_t)36 * (size_t)(OC * IC + IC * NT + OC * NT);
}

int launch_conv2d_winograd_f32(const float* input, const float* weight, const float* bias,
                               float* output, int64_t batch, int64_t IC, int64_t OC,
                               int64_t IH, int64_t IW, int64_t PH, int64_t PW, int precision,
                               float* ws, hipStream_t stream, bool flip_filter) {
    WinoGeom g;
    g.B = batch; g.IC = IC; g.OC = OC; g.IH = IH; g.IW = IW; g.PH = PH; g.PW = PW;
    g.OH = IH + 2 * PH - 2; g.OW = IW + 2 * PW - 2;
    g.TH = ceil_div(g.OH, 4); g.TW = ceil_div(g.OW, 4);
    g.NT = batch * g.TH * g.TW;
    g.vec_out = ((uintptr_t)output % 16 == 0) && (g.OW % 4 == 0);
    if (ceil_div(IC * g.NT, 256) > INT32_MAX || ceil_div(OC * g.NT, 256) > INT32_MAX ||
        ceil_div(OC * IC, 256) > INT32_MAX)
        return set_error(CDX_ERR_UNSUPPORTED, "winograd: problem too large");
    float* U = ws;
    float* V = U + 36 * OC * IC;
    float* Mm = V + 36 * IC * g.NT;

    int st;
    if (IW % 4 == 0 && PW >= 0 && PW <= 2 && (uintptr_t)input % 16 == 0) {
        // filter + input transforms in one launch
        const int64_t fb = blocks_for(OC * IC);
        const dim3 grid((unsigned)(fb + blocks_for(IC * g.NT)));
        auto go = [&](auto sh, auto flip) {
            hipLaunchKernelGGL((wino_filter_input_v4_kernel<decltype(sh)::value, decltype(flip)::value>),
                               grid, dim3(256), 0, stream, weight, U, input, V, g, fb);
        };
        using F = std::false_type;
        using T = std::true_type;
        if (PW == 0) flip_filter ? go(std::integral_constant<int, 4>{}, T{}) : go(std::integral_constant<int, 4>{}, F{});
        else if (PW == 1) flip_filter ? go(std::integral_constant<int, 3>{}, T{}) : go(std::integral_constant<int, 3>{}, F{});
        else flip_filter ? go(std::integral_constant<int, 2>{}, T{}) : go(std::integral_constant<int, 2>{}, F{});
        st = hip_error(hipGetLastError(), "wino_filter_input_v4_kernel launch");
    } else {
        if (flip_filter)
            hipLaunchKernelGGL(wino_filter_kernel<true>, dim3(blocks_for(OC * IC)), dim3(256), 0,
                               stream, weight, U, OC, IC);
        else
            hipLaunchKernelGGL(wino_filter_kernel<false>, dim3(blocks_for(OC * IC)), dim3(256), 0,
                               stream, weight, U, OC, IC);
        st = hip_error(hipGetLastError(), "wino_filter_kernel launch");
        if (st) return st;
        hipLaunchKernelGGL(wino_input_kernel, dim3(blocks_for(IC * g.NT)), dim3(256), 0, stream,
                           input, V, g);
        st = hip_error(hipGetLastError(), "wino_input_kernel launch");
    }
    if (st) return st;

    // 36 GEMMs M_a[OC, NT] = U_a[OC, IC] * V_a[IC, NT] in one batched launch
    GemmArgs ga{CDX_OP_N, CDX_OP_N, OC, g.NT, IC, U, IC, V, g.NT, Mm, g.NT, 0, 0,
                nullptr, CDX_BIAS_NONE, CDX_EPI_NONE};
    ga.batch = 36;
    ga.stride_a = OC * IC;
    ga.stride_b = IC * g.NT;
    ga.stride_c = OC * g.NT;
    if (precision == CDX_PREC_FP32) st = launch_gemm_f32(ga, stream);
    else st = launch_gemm_bf16x3(ga, precision == CDX_PREC_TF32MODE4 ? 4 : 3, stream);
    if (st) return st;

    hipLaunchKernelGGL(wino_output_kernel, dim3(blocks_for(OC * g.NT)), dim3(256), 0, stream,
                       Mm, bias, output, g);
    return hip_error(hipGetLastError(), "wino_output_kernel launch");
}

}  // namespace cdx
