// Conv2d forward as an implicit GEMM on gfx950 (FP32 MFMA), no column buffer:
//
//   y[b, oc, s] = bias[oc] + sum_k W[oc, k] * x[b, ic, oh*SH - PH + kh, ow*SW - PW + kw]
//   k = (ic*KH + kh)*KW + kw,  s = oh*OW + ow,  zero outside the image
//
// -- the reference's implicit_gemm_conv2d_kernel (src/kernels/conv_kernel.cu:
// 172-215), which its forward dispatcher takes for layers whose im2col buffer
// would exceed 4 MiB outside 3x3 stride 1 (:263-275).  The reference runs one
// thread per output with a scalar loop over (ic, kh, kw); here it is the
// GEMM weight[OC, Kc] x col[Kc, B*S] of the im2col route, with the column
// tile gathered from the NCHW input while each k-tile is staged into LDS, so
// nothing of the Kc x B*S column matrix (1.26 GB for a 7x7 layer at
// 32 x 64 x 56^2) is ever materialised.
//
// Tile: 64 (OC) x 128 (output pixels n = b*S + s) x 16 (k); 4 waves of
// 32 x 64, v_mfma_f32_16x16x4_f32 with the library's k-permutation (lane
// group g feeds MFMA q with k = 4g + q, so each operand fragment is one
// 16-byte LDS read).  Per k-tile a thread stages one 16-byte run of a filter
// row and gathers 8 consecutive k of one output pixel:
//  * the pixel's (b, oh, ow) is decoded once per kernel (multiply-high
//    divisions), giving its image base and window origin (ih0, iw0);
//  * the 8 taps' (ic, kh, kw) are decoded once per k-tile from a k that is
//    uniform across the wave, then stepped (kw, then kh, then ic), so the
//    per-element work is two bounds tests and one load; consecutive lanes
//    hold consecutive pixels, so each load instruction reads along an input
//    row.
// Both operands sit k-contiguous in LDS ([row][16 + 4]), double buffered; the
// next k-tile's loads are issued before the current k-tile's MFMAs.
// FP32 products in every precision mode, as the reference's kernel.
#include "cdx_internal.hpp"

namespace cdx {
namespace {

constexpr int CF_BM = 64, CF_BN = 128, CF_BK = 16, CF_NT = 256;
constexpr int CF_STRIDE = CF_BK + 4;   // LDS row pitch (floats)

struct CfArgs {
    const float* x;      // [B][IC][IH][IW]
    const float* w;      // [OC][Kc]
    const float* bias;   // [OC] or null
    float* y;            // [B][OC][S]
    int OC, Kc, N, S;    // N = B*S
    int OW, IH, IW, plane, KH, KW, SH, SW, PH, PW;
    int64_t img_x, img_y;                // IC*IH*IW, OC*S
    DivMagic div_s, div_ow, div_khw, div_kw;
    int vec_w;                           // Kc % 4 == 0 and w 16-byte aligned
};

struct CfStage {
    float4 a;       // filter row ra, k columns ca .. ca+3
    float g[8];     // gathered column: pixel gn, 8 consecutive k
};

__global__ __launch_bounds__(CF_NT)
void conv_fwd_implicit_kernel(CfArgs p) {
    __shared__ __attribute__((aligned(16))) float lds[2][(CF_BM + CF_BN) * CF_STRIDE];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lq = lane >> 4;
    const int wm0 = (wave >> 1) * 32, wn0 = (wave & 1) * 64;
    const int n0 = blockIdx.x * CF_BN, oc0 = blockIdx.y * CF_BM;

    // filter staging slot
    const int ra = tid >> 2, ca = (tid & 3) * 4;
    const bool a_ok = oc0 + ra < p.OC;
    const float* wrow = p.w + (int64_t)(a_ok ? oc0 + ra : 0) * p.Kc;   // (this launch's channels)

    // gather slot: pixel gn of the tile, k offsets 8*kg .. 8*kg + 7
    const int gn = tid & (CF_BN - 1);
    const int kg = __builtin_amdgcn_readfirstlane(tid >> 7);   // wave-uniform
    const int n = n0 + gn;
    const bool n_ok = n < p.N;
    const uint32_t nn = n_ok ? (uint32_t)n : 0u;
    const uint32_t b = div_u31(nn, p.div_s);
    const uint32_t s = nn - b * (uint32_t)p.S;
    const uint32_t oh = div_u31(s, p.div_ow);
    const uint32_t ow = s - oh * (uint32_t)p.OW;
    const int ih0 = (int)oh * p.SH - p.PH, iw0 = (int)ow * p.SW - p.PW;
    const float* ximg = p.x + (int64_t)b * p.img_x;

    auto load = [&](CfStage& st, int k0) {
        const int ka = k0 + ca;
        if (p.vec_w && a_ok && ka + 3 < p.Kc) {
            st.a = *reinterpret_cast<const float4*>(wrow + ka);
        } else {
            st.a.x = a_ok && ka + 0 < p.Kc ? wrow[ka + 0] : 0.0f;
            st.a.y = a_ok && ka + 1 < p.Kc ? wrow[ka + 1] : 0.0f;
            st.a.z = a_ok && ka + 2 < p.Kc ? wrow[ka + 2] : 0.0f;
            st.a.w = a_ok && ka + 3 < p.Kc ? wrow[ka + 3] : 0.0f;
        }
        // taps k .. k+7, k uniform across the wave
        const int k = k0 + 8 * kg;
        const uint32_t ku = k < p.Kc ? (uint32_t)k : 0u;
        int ic = (int)div_u31(ku, p.div_khw);
        const int r = (int)ku - ic * p.KH * p.KW;
        int kh = (int)div_u31((uint32_t)r, p.div_kw);
        int kw = r - kh * p.KW;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int ih = ih0 + kh, iw = iw0 + kw;
            const bool ok = n_ok && k + e < p.Kc && (unsigned)ih < (unsigned)p.IH &&
                            (unsigned)iw < (unsigned)p.IW;
            st.g[e] = ok ? ximg[ic * p.plane + ih * p.IW + iw] : 0.0f;
            if (++kw == p.KW) {
                kw = 0;
                if (++kh == p.KH) {
                    kh = 0;
                    ++ic;
                }
            }
        }
    };
    auto store = [&](const CfStage& st, int buf) {
        float* sA = lds[buf];
        float* sB = sA + CF_BM * CF_STRIDE;
        *reinterpret_cast<float4*>(sA + ra * CF_STRIDE + ca) = st.a;
        float* dst = sB + gn * CF_STRIDE + 8 * kg;
        *reinterpret_cast<float4*>(dst) = make_float4(st.g[0], st.g[1], st.g[2], st.g[3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(st.g[4], st.g[5], st.g[6], st.g[7]);
    };

    floatx4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int buf) {
        const float* sA = lds[buf];
        const float* sB = sA + CF_BM * CF_STRIDE;
        float4 a[2], bq[4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            a[i] = *reinterpret_cast<const float4*>(sA + (wm0 + i * 16 + l16) * CF_STRIDE + 4 * lq);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            bq[j] = *reinterpret_cast<const float4*>(sB + (wn0 + j * 16 + l16) * CF_STRIDE + 4 * lq);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float av = q == 0 ? a[i].x : q == 1 ? a[i].y : q == 2 ? a[i].z : a[i].w;
                    const float bv = q == 0 ? bq[j].x : q == 1 ? bq[j].y : q == 2 ? bq[j].z : bq[j].w;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[i][j], 0, 0, 0);
                }
    };

    const int nk = (int)ceil_div(p.Kc, CF_BK);
    CfStage st;
    load(st, 0);
    store(st, 0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const bool more = kt + 1 < nk;
        if (more) load(st, (kt + 1) * CF_BK);
        compute(kt & 1);
        if (more) store(st, (kt + 1) & 1);
        __syncthreads();
    }

    // D layout of a 16x16 block: register r of lane l is row 4*(l/16) + r,
    // column l % 16; output (oc, n) -> y[b][oc][s] + bias[oc]
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int on = n0 + wn0 + j * 16 + l16;
        if (on >= p.N) continue;
        const uint32_t ob = div_u31((uint32_t)on, p.div_s);
        float* ycol = p.y + (int64_t)ob * p.img_y + (on - (int)ob * p.S);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int oc = oc0 + wm0 + i * 16 + 4 * lq + r;
                if (oc < p.OC)
                    ycol[(int64_t)oc * p.S] = acc[i][j][r] + (p.bias ? p.bias[oc] : 0.0f);
            }
    }
}

}  // namespace

bool conv_fwd_implicit_ok(int64_t batch, int64_t IC, int64_t IH, int64_t IW, int64_t KH,
                          int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    const int64_t OH = (IH + 2 * PH - KH) / SH + 1, OW = (IW + 2 * PW - KW) / SW + 1;
    const int64_t lim = INT32_MAX / 2;
    // 32-bit pixel, in-image and tap indices; window origins within int range
    return OH >= 1 && OW >= 1 && batch * OH * OW < lim && IC * IH * IW < lim &&
           IC * KH * KW < lim && OH * SH + KH + IH < lim && OW * SW + KW + IW < lim &&
           PH < lim && PW < lim;
}

int launch_conv_fwd_implicit_f32(const float* x, const float* w, const float* bias, float* y,
                                 int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                                 int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                                 int64_t PW, hipStream_t stream) {
    if (!conv_fwd_implicit_ok(batch, IC, IH, IW, KH, KW, SH, SW, PH, PW))
        return set_error(CDX_ERR_UNSUPPORTED, "conv implicit forward: geometry beyond 32-bit indices");
    const int64_t OH = (IH + 2 * PH - KH) / SH + 1, OW = (IW + 2 * PW - KW) / SW + 1;
    CfArgs p;
    p.x = x;
    p.Kc = (int)(IC * KH * KW); p.S = (int)(OH * OW); p.N = (int)(batch * OH * OW);
    p.OW = (int)OW; p.IH = (int)IH; p.IW = (int)IW; p.plane = (int)(IH * IW);
    p.KH = (int)KH; p.KW = (int)KW; p.SH = (int)SH; p.SW = (int)SW; p.PH = (int)PH; p.PW = (int)PW;
    p.img_x = IC * IH * IW; p.img_y = OC * OH * OW;
    p.div_s = div_magic(p.S); p.div_ow = div_magic(OW);
    p.div_khw = div_magic(KH * KW); p.div_kw = div_magic(KW);
    p.vec_w = p.Kc % 4 == 0 && (uintptr_t)w % 16 == 0;
    // output channels in launches of at most 65535 tiles (grid y)
    const int64_t chunk = (int64_t)65535 * CF_BM;
    for (int64_t oc0 = 0; oc0 < OC; oc0 += chunk) {
        const int64_t oc_n = OC - oc0 < chunk ? OC - oc0 : chunk;
        p.OC = (int)oc_n;
        p.w = w + oc0 * p.Kc;
        p.bias = bias ? bias + oc0 : nullptr;
        p.y = y + oc0 * p.S;
        const dim3 grid((unsigned)ceil_div(p.N, CF_BN), (unsigned)ceil_div(oc_n, CF_BM));
        hipLaunchKernelGGL(conv_fwd_implicit_kernel, grid, dim3(CF_NT), 0, stream, p);
        const int st = hip_error(hipGetLastError(), "conv_fwd_implicit_kernel launch");
        if (st) return st;
    }
    return CDX_OK;
}

}  // namespace cdx
