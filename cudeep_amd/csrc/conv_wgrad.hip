// Conv backward weight as an implicit GEMM on gfx950 (FP32 MFMA):
//
//   dW[oc, n] = sum over b, s of dY[b, oc, s] * x[b, ic, oh*SH - PH + kh, ow*SW - PW + kw]
//   n = (ic*KH + kh)*KW + kw,  s = oh*OW + ow
//
// -- the reference's dW = dY_flat[OC, B*S] * col^T (src/kernels/conv_kernel.cu:
// 486-545, col as built by im2col_kernel :32-65), without the column buffer
// or the dY reshape: both GEMM operands are gathered from the NCHW tensors
// while the k-tiles are staged into LDS.
//
// Shape of the problem: M = OC and N = IC*KH*KW are small (64 x 576 at
// ResNet-like layers), K = B*OH*OW is long (100352).  One workgroup owns a
// 64 x BN tile of dW and one slice of K; the slices' partial tiles are summed
// in slice order by the split-K reduction (deterministic).
//
// A gathered element is x[b, ic, oh*SH + kh - PH, ow*SW + kw - PW], zero
// outside the image: (oh, ow) of a thread's 4 pixels are decoded once per
// k-tile (a multiply-high division by OW) and shared by its rows; each row
// keeps its plane offset and (kh - PH, kw - PW) in registers for the whole
// K loop.  (Materialising a zero-bordered copy of x to drop the bounds
// tests measured slower: 123 against 103 us at the shape below.)
//
// K layout: every image's OH*OW pixels are padded to a whole number of
// BK-wide k-tiles, so a k-tile never straddles two images: its image b and
// first pixel are uniform across the workgroup (scalar registers), pixels
// s >= OH*OW read as zero.
//
// Per k-tile and thread: one 4-pixel column of dY (a 16-byte load when the
// plane allows) and BK/16 4-pixel columns of the gathered input.  LDS holds
// both operands k-contiguous ([row][BK + 4]), double buffered, read as
// 16-byte fragments with the same k-permutation as the library's GEMM: a
// lane feeds MFMA q with k = 4*(lane/16) + q.  Two register staging sets
// keep tile k+2's loads in flight while tile k+1 is written to LDS.
#include "cdx_internal.hpp"

namespace cdx {
namespace {

// Tile: 64 (OC) x BN (filter rows) x BK (pixels); waves of 32 x 32 in a
// 2 x BN/32 grid (4*BN threads).  Measured on MI355X (C5 backward weight,
// 32 x 64 x 56^2, 3x3): BN 192, BK 32 and ~256 workgroups beat BN 128 / 64,
// BK 16 and 512-1024 workgroups.
#ifndef CDX_WGRAD_BN
#define CDX_WGRAD_BN 192
#endif
#ifndef CDX_WGRAD_BK
#define CDX_WGRAD_BK 32
#endif
#ifndef CDX_WGRAD_TARGET_WGS
#define CDX_WGRAD_TARGET_WGS 256
#endif
constexpr int WG_BM = 64, WG_BN = CDX_WGRAD_BN, WG_BK = CDX_WGRAD_BK;
constexpr int WG_WAVES_N = WG_BN / 32;
constexpr int WG_NT = 64 * 2 * WG_WAVES_N;
constexpr int WG_CPR = WG_BK / 4;                         // 4-pixel columns per row
constexpr int WG_RPP = WG_NT / WG_CPR;                    // rows per staging pass
constexpr int WG_BP = WG_BN / WG_RPP;                     // gathered columns per thread
constexpr int WG_STRIDE = WG_BK + 4;                      // LDS row stride (floats)
static_assert(WG_BN % 32 == 0 && WG_BK % 16 == 0 && WG_BN % WG_RPP == 0 && WG_RPP >= WG_BM,
              "tile shape");

// n / d for n < 2^31, d < 2^31: q = (mulhi(n, m) + n) >> l
struct DivMagic {
    uint32_t m;
    int l;
};

DivMagic div_magic(int64_t d) {
    int l = 0;
    while (((int64_t)1 << l) < d) ++l;
    const uint64_t m = ((((uint64_t)1 << 32) * (((uint64_t)1 << l) - (uint64_t)d)) / (uint64_t)d) + 1;
    return {(uint32_t)m, l};
}

__device__ __forceinline__ uint32_t div_u31(uint32_t n, DivMagic g) {
    return (__umulhi(n, g.m) + n) >> g.l;
}

struct WgGeom {
    int64_t B, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, OH, OW;
    int64_t S() const { return OH * OW; }
    int64_t Kc() const { return IC * KH * KW; }
    int64_t tpi() const { return ceil_div(OH * OW, WG_BK); }
    int64_t tiles() const { return ceil_div(OC, WG_BM) * ceil_div(Kc(), WG_BN); }
};

WgGeom make_geom(int64_t B, int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH,
                 int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    WgGeom g{B, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, 0, 0};
    g.OH = (IH + 2 * PH - KH) / SH + 1;
    g.OW = (IW + 2 * PW - KW) / SW + 1;
    return g;
}

int splits_for(const WgGeom& g) {
    const int64_t kt_total = g.B * g.tpi();
    // about CDX_WGRAD_TARGET_WGS workgroups, at least 8 k-tiles per slice
    int64_t s = CDX_WGRAD_TARGET_WGS / g.tiles();
    if (s > kt_total / 8) s = kt_total / 8;
    if (s < 1) s = 1;
    const int64_t chunk = ceil_div(kt_total, s);
    return (int)ceil_div(kt_total, chunk);
}

struct WgArgs {
    const float* dy;   // [B][OC][S]
    const float* x;    // [B][IC][IH][IW]
    float* out;        // [splits][OC][Kc] partials (or dW when one slice)
    int64_t OC, Kc;
    int64_t img_x, img_y;          // IC*IH*IW, OC*S
    int IH, IW, OW, S, plane;      // plane = IH*IW
    int KW, KHW, SH, SW, PH, PW;
    int tpi;                       // k-tiles per image
    int kt_total, kt_chunk;        // k-tiles in all / per slice
    DivMagic div_ow, div_khw, div_kw;
    int vec_dy;                    // S % 4 == 0 and dy 16-byte aligned
};

// Registers staging one k-tile: this thread's dY and gathered columns.
struct WgStage {
    float4 a, b[WG_BP];
};

__global__ __launch_bounds__(WG_NT)
void conv_wgrad_f32_kernel(WgArgs p) {
    __shared__ __attribute__((aligned(16))) float lds[2][(WG_BM + WG_BN) * WG_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lq = lane >> 4;
    const int wm0 = (wave / WG_WAVES_N) * 32, wn0 = (wave % WG_WAVES_N) * 32;

    const int tiles_n = (int)ceil_div(p.Kc, WG_BN);
    const int64_t bm = (int64_t)(blockIdx.x / tiles_n) * WG_BM;
    const int64_t bn = (int64_t)(blockIdx.x % tiles_n) * WG_BN;
    const int kt_begin = blockIdx.y * p.kt_chunk;
    const int kt_end = min(p.kt_total, kt_begin + p.kt_chunk);

    // staging slots: 4-pixel column c of gathered rows rb + i*RPP (and of
    // dY row rb for rb < 64)
    const int c = (tid % WG_CPR) * 4;
    const int rb = tid / WG_CPR;
    const bool has_a = rb < WG_BM;
    const int64_t oc = bm + rb;
    const bool a_ok = has_a && oc < p.OC;

    int64_t b_off[WG_BP];   // ic * IH * IW
    int b_dh[WG_BP], b_dw[WG_BP];
    bool b_ok[WG_BP];
#pragma unroll
    for (int i = 0; i < WG_BP; ++i) {
        const int64_t n = bn + rb + i * WG_RPP;
        b_ok[i] = n < p.Kc;
        const uint32_t nn = b_ok[i] ? (uint32_t)n : 0u;
        const uint32_t ic = div_u31(nn, p.div_khw);
        const uint32_t t = nn - ic * (uint32_t)p.KHW;
        const uint32_t kh = div_u31(t, p.div_kw);
        const uint32_t kw = t - kh * (uint32_t)p.KW;
        b_off[i] = (int64_t)ic * p.plane;
        b_dh[i] = (int)kh - p.PH;
        b_dw[i] = (int)kw - p.PW;
    }

    // the k-tile the next load() reads: image ld_b, tile ld_t of that image
    // (loads run in k order, so a running pair replaces a division per tile)
    int ld_b = kt_begin / p.tpi;
    int ld_t = kt_begin - ld_b * p.tpi;

    auto load = [&](WgStage& st) {
        const int s0 = ld_t * WG_BK + c;
        if (has_a) {   // dY[b, oc, s0 .. s0+3]
            const float* ya = p.dy + (int64_t)ld_b * p.img_y + oc * p.S + s0;
            if (a_ok && p.vec_dy && s0 + 3 < p.S) {
                st.a = *reinterpret_cast<const float4*>(ya);
            } else {
                st.a.x = a_ok && s0 + 0 < p.S ? ya[0] : 0.0f;
                st.a.y = a_ok && s0 + 1 < p.S ? ya[1] : 0.0f;
                st.a.z = a_ok && s0 + 2 < p.S ? ya[2] : 0.0f;
                st.a.w = a_ok && s0 + 3 < p.S ? ya[3] : 0.0f;
            }
        }
        // (oh, ow) of the 4 pixels, shared by the gathered rows
        int oh[4], ow[4];
        oh[0] = (int)div_u31((uint32_t)s0, p.div_ow);
        ow[0] = s0 - oh[0] * p.OW;
#pragma unroll
        for (int j = 1; j < 4; ++j) {
            const bool wrap = ow[j - 1] + 1 == p.OW;
            ow[j] = wrap ? 0 : ow[j - 1] + 1;
            oh[j] = wrap ? oh[j - 1] + 1 : oh[j - 1];
        }
        const float* xb = p.x + (int64_t)ld_b * p.img_x;
#pragma unroll
        for (int i = 0; i < WG_BP; ++i) {
            // x[b, ic, oh*SH + kh - PH, ow*SW + kw - PW]
            const float* xr = xb + b_off[i];
            float e[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ih = oh[j] * p.SH + b_dh[i];
                const int iw = ow[j] * p.SW + b_dw[i];
                const bool ok = b_ok[i] && s0 + j < p.S && (unsigned)ih < (unsigned)p.IH &&
                                (unsigned)iw < (unsigned)p.IW;
                e[j] = ok ? xr[ih * p.IW + iw] : 0.0f;
            }
            st.b[i] = make_float4(e[0], e[1], e[2], e[3]);
        }
        if (++ld_t == p.tpi) {
            ld_t = 0;
            ++ld_b;
        }
    };
    auto store = [&](const WgStage& st, int buf) {
        float* sA = lds[buf];
        float* sB = sA + WG_BM * WG_STRIDE;
        if (has_a) *reinterpret_cast<float4*>(sA + rb * WG_STRIDE + c) = st.a;
#pragma unroll
        for (int i = 0; i < WG_BP; ++i)
            *reinterpret_cast<float4*>(sB + (rb + i * WG_RPP) * WG_STRIDE + c) = st.b[i];
    };

    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int buf) {
        const float* sA = lds[buf];
        const float* sB = sA + WG_BM * WG_STRIDE;
#pragma unroll
        for (int kk = 0; kk < WG_BK; kk += 16) {
            float a[2][4], bq[2][4];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float4 t = *reinterpret_cast<const float4*>(
                    sA + (wm0 + i * 16 + l16) * WG_STRIDE + kk + 4 * lq);
                a[i][0] = t.x; a[i][1] = t.y; a[i][2] = t.z; a[i][3] = t.w;
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float4 t = *reinterpret_cast<const float4*>(
                    sB + (wn0 + j * 16 + l16) * WG_STRIDE + kk + 4 * lq);
                bq[j][0] = t.x; bq[j][1] = t.y; bq[j][2] = t.z; bq[j][3] = t.w;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][q], bq[j][q],
                                                                         acc[i][j], 0, 0, 0);
        }
    };

    const int nk = kt_end - kt_begin;
    if (nk > 0) {
        WgStage s0, s1;
        load(s0);
        if (nk > 1) load(s1);
        store(s0, 0);
        __syncthreads();
        int k = 0;
        for (; k + 3 < nk; k += 2) {        // stage 0 holds tile k, set 1 tile k+1
            load(s0);                       // tile k+2
            compute(0);
            store(s1, 1);
            __syncthreads();
            load(s1);                       // tile k+3
            compute(1);
            store(s0, 0);
            __syncthreads();
        }
        if (k + 2 < nk) {                   // three tiles left
            load(s0);
            compute(0);
            store(s1, 1);
            __syncthreads();
            compute(1);
            store(s0, 0);
            __syncthreads();
            compute(0);
        } else if (k + 1 < nk) {            // two tiles left
            compute(0);
            store(s1, 1);
            __syncthreads();
            compute(1);
        } else {                            // one tile
            compute(0);
        }
    }

    // D layout of a 16x16 block: register r of lane l is row 4*(l/16) + r,
    // column l % 16
    float* out = p.out + (int64_t)blockIdx.y * p.OC * p.Kc;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t nn = bn + wn0 + j * 16 + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = bm + wm0 + i * 16 + 4 * lq + r;
                if (m < p.OC && nn < p.Kc) out[m * p.Kc + nn] = acc[i][j][r];
            }
        }
}

}  // namespace

bool conv_wgrad_implicit_ok(int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                            int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                            int64_t PW) {
    const WgGeom g = make_geom(batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW);
    const int64_t lim = (int64_t)1 << 30;
    // 32-bit in-kernel index math: plane offsets, pixels, k-tiles, filter
    // rows, input coordinates
    return batch > 0 && OC > 0 && g.S() > 0 && g.Kc() > 0 && IH * IW < lim && g.S() < lim &&
           batch * g.tpi() < lim && g.Kc() < lim && g.tiles() < lim &&
           g.OH * SH + KH < lim && g.OW * SW + KW < lim && PH < lim && PW < lim;
}

size_t conv_wgrad_implicit_floats(int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                                  int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                                  int64_t PW) {
    const WgGeom g = make_geom(batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW);
    const int s = splits_for(g);
    return s > 1 ? (size_t)s * (size_t)OC * (size_t)g.Kc() : 0;
}

int launch_conv_wgrad_f32(const float* dy, const float* x, float* dw, float* ws, int64_t batch,
                          int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                          int64_t SH, int64_t SW, int64_t PH, int64_t PW, hipStream_t stream) {
    const WgGeom g = make_geom(batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW);
    const int splits = splits_for(g);
    WgArgs p;
    p.dy = dy; p.x = x;
    p.out = splits > 1 ? ws : dw;
    p.OC = OC; p.Kc = g.Kc();
    p.img_x = IC * IH * IW; p.img_y = OC * g.S();
    p.IH = (int)IH; p.IW = (int)IW; p.OW = (int)g.OW; p.S = (int)g.S(); p.plane = (int)(IH * IW);
    p.KW = (int)KW; p.KHW = (int)(KH * KW);
    p.SH = (int)SH; p.SW = (int)SW; p.PH = (int)PH; p.PW = (int)PW;
    p.tpi = (int)g.tpi();
    p.kt_total = (int)(batch * p.tpi);
    p.kt_chunk = (int)ceil_div(p.kt_total, splits);
    p.div_ow = div_magic(g.OW);
    p.div_khw = div_magic(KH * KW);
    p.div_kw = div_magic(KW);
    p.vec_dy = (p.S % 4 == 0) && ((uintptr_t)dy % 16 == 0);
    hipLaunchKernelGGL(conv_wgrad_f32_kernel, dim3((unsigned)g.tiles(), (unsigned)splits),
                       dim3(WG_NT), 0, stream, p);
    int st = hip_error(hipGetLastError(), "conv_wgrad_f32_kernel launch");
    if (st || splits == 1) return st;
    GemmArgs r{CDX_OP_N, CDX_OP_N, OC, p.Kc, 0, nullptr, 1, nullptr, 1, dw, p.Kc, 0, 0,
               nullptr, CDX_BIAS_NONE, CDX_EPI_NONE};
    return launch_splitk_reduce(ws, splits, r, stream);
}

}  // namespace cdx
