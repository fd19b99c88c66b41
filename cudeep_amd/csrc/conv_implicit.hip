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
//  * the 8 taps (ic, kh, kw) of a k-tile are the same for every lane of a
//    wave: eight lanes decode one each and the wave reads them back with
//    readlane, so the per-element work is two bounds tests, one add and one
//    load; consecutive lanes hold consecutive pixels, so each load
//    instruction reads along an input row.
// Both operands sit k-contiguous in LDS ([row][16 + 4]), double buffered; the
// next k-tile's loads are issued before the current k-tile's MFMAs and
// stored after them.  (Measured on MI355X: 32-deep k-tiles, or k ordered by
// 32-channel chunks of one tap, were slower -- fewer resident waves, and in
// the channel order every filter element of a k-tile sits on its own cache
// line.)
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
    int OW, IH, IW, plane, KH, KW, KHW, SH, SW, PH, PW;
    int64_t img_x, img_y;                // IC*IH*IW, OC*S
    DivMagic div_s, div_ow, div_khw, div_kw;
    int vec_w;                           // Kc % 4 == 0 and w 16-byte aligned
};

struct CfStage {
    float4 a;       // filter row ra, k columns ca .. ca+3
    float g[8];     // gathered column: pixel gn, 8 consecutive k
    uint32_t ok;    // bit e: g[e] in range; bits 8-11: a's components
};

// Keeps a loaded value opaque to the compiler, so the select that zeroes an
// out-of-range slot (applied when the stage is stored, after the MFMAs)
// cannot be folded back into a conditional load at the load site, which
// would split the loop into branches and wait for each load at once.
__device__ __forceinline__ float opaque(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// VECW: Kc % 4 == 0 and a 16-byte-aligned filter, so each filter run of 4
// k is wholly inside or outside its row (one 16-byte load).
template <bool VECW>
__global__ __launch_bounds__(CF_NT)
void conv_fwd_implicit_kernel(CfArgs p) {
    __shared__ __attribute__((aligned(16))) float lds[2][(CF_BM + CF_BN) * CF_STRIDE];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lq = lane >> 4;
    const int wm0 = (wave >> 1) * 32, wn0 = (wave & 1) * 64;
    const int n0 = blockIdx.x * CF_BN, oc0 = blockIdx.y * CF_BM;

    // filter staging slot (this launch's channels)
    const int ra = tid >> 2, ca = (tid & 3) * 4;
    const bool a_ok = oc0 + ra < p.OC;
    const float* wrow = p.w + (int64_t)(a_ok ? oc0 + ra : 0) * p.Kc;

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
    const int pix0 = ih0 * p.IW + iw0;   // in-plane offset of tap (0, 0)
    const float* ximg = p.x + (int64_t)b * p.img_x;

    // Per k-tile, lane e < 8 of each wave decodes tap k + e of the wave's
    // 8 k (ic, kh, kw -> in-image offset ic*IH*IW + kh*IW + kw, and kh, kw;
    // -1 past Kc), and the wave reads the 8 taps back as scalars with
    // readlane: the tap walk costs a few vector instructions per k-tile
    // instead of a chain of scalar ones per element.  Every load is issued
    // from an in-bounds address (out-of-range slots read element 0 of their
    // row or image) and store() zeroes those slots.
    auto load = [&](CfStage& st, int k0) {
        const int ka = k0 + ca;
        uint32_t ok = 0;
        if constexpr (VECW) {
            const bool in = a_ok & (ka < p.Kc);
            st.a = *reinterpret_cast<const float4*>(wrow + (in ? ka : 0));
            ok |= in ? 0xF00u : 0u;
        } else {
            float e[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const bool in = a_ok & (ka + c < p.Kc);
                e[c] = wrow[in ? ka + c : 0];
                ok |= in ? 1u << (8 + c) : 0u;
            }
            st.a = make_float4(e[0], e[1], e[2], e[3]);
        }
        const int kt = k0 + 8 * kg + (lane & 7);
        const bool t_ok = kt < p.Kc;
        const uint32_t ku = t_ok ? (uint32_t)kt : 0u;
        const uint32_t ic = div_u31(ku, p.div_khw);
        const uint32_t r = ku - ic * (uint32_t)p.KHW;
        const uint32_t kh = div_u31(r, p.div_kw);
        const uint32_t kw = r - kh * (uint32_t)p.KW;
        const int t_off = (int)(ic * (uint32_t)p.plane + kh * (uint32_t)p.IW + kw);
        const int t_hw = t_ok ? (int)((kh << 16) | kw) : -1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int off = __builtin_amdgcn_readlane(t_off, e);
            const int hw = __builtin_amdgcn_readlane(t_hw, e);
            const int ih = ih0 + (hw >> 16), iw = iw0 + (hw & 0xFFFF);
            const bool in = n_ok & (hw >= 0) & ((unsigned)ih < (unsigned)p.IH) &
                            ((unsigned)iw < (unsigned)p.IW);
            st.g[e] = ximg[in ? pix0 + off : 0];
            ok |= in ? 1u << e : 0u;
        }
        st.ok = ok;
    };
    auto store = [&](const CfStage& st, int buf) {
        float* sA = lds[buf];
        float* sB = sA + CF_BM * CF_STRIDE;
        auto z = [&](float v, int bit) {
            const float o = opaque(v);
            return (st.ok >> bit) & 1u ? o : 0.0f;
        };
        *reinterpret_cast<float4*>(sA + ra * CF_STRIDE + ca) =
            make_float4(z(st.a.x, 8), z(st.a.y, 9), z(st.a.z, 10), z(st.a.w, 11));
        float* dst = sB + gn * CF_STRIDE + 8 * kg;
        *reinterpret_cast<float4*>(dst) =
            make_float4(z(st.g[0], 0), z(st.g[1], 1), z(st.g[2], 2), z(st.g[3], 3));
        *reinterpret_cast<float4*>(dst + 4) =
            make_float4(z(st.g[4], 4), z(st.g[5], 5), z(st.g[6], 6), z(st.g[7], 7));
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

    // one barrier per k-tile; the next k-tile's loads are in flight during
    // this one's MFMAs (a scheduling barrier keeps the LDS stores, which wait
    // for them, after the MFMAs); the last k-tile is peeled
    const int nk = (int)ceil_div(p.Kc, CF_BK);
    CfStage st;
    load(st, 0);
    store(st, 0);
    __syncthreads();
    int kt = 0;
    for (; kt + 1 < nk; ++kt) {
        load(st, (kt + 1) * CF_BK);
        compute(kt & 1);
        __builtin_amdgcn_sched_barrier(0);
        store(st, (kt + 1) & 1);
        __syncthreads();
    }
    compute(kt & 1);

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
           PH < lim && PW < lim && KH < 32768 && KW < 32768;   // (kh, kw) packed in 16 bits
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
    p.KH = (int)KH; p.KW = (int)KW; p.KHW = (int)(KH * KW); p.SH = (int)SH; p.SW = (int)SW; p.PH = (int)PH; p.PW = (int)PW;
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
        if (p.vec_w)
            hipLaunchKernelGGL(conv_fwd_implicit_kernel<true>, grid, dim3(CF_NT), 0, stream, p);
        else
            hipLaunchKernelGGL(conv_fwd_implicit_kernel<false>, grid, dim3(CF_NT), 0, stream, p);
        const int st = hip_error(hipGetLastError(), "conv_fwd_implicit_kernel launch");
        if (st) return st;
    }
    return CDX_OK;
}

}  // namespace cdx
