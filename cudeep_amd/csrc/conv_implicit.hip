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
// Two forms: the row-window form further down (the input window of a tile
// staged in LDS per channel chunk; every layer whose window fits, and the
// stride-1 backward-data route) and, for the rest, the gather form:
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
#include <algorithm>
#include <type_traits>

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

// ---------------------------------------------------------------------------
// Row-window form: every kernel size and stride whose input window fits in LDS.
//
// A workgroup owns 64 output channels x TN (80, 112 or 128) consecutive
// output pixels s of one image.  Those pixels lie in at most R output rows
// starting at oh_lo, which read the input rows ih = oh_lo*SH - PH + r,
// r < NR = (R-1)*SH + KH, and the columns iw = c - PW, c < WP = (OW-1)*SW +
// KW.  Per chunk of ICT input channels the workgroup stages that window of
// each channel into LDS once, zero outside the image (the padding is
// materialised), so every column-matrix element of the tile is one LDS read:
//
//   col[(ic, kh, kw), s] = win[ic - ic0][(oh(s) - oh_lo)*SH + kh][ow(s)*SW + kw]
//                        = win_flat[base(s) + off(k)]
//   base(s) = (oh(s) - oh_lo)*SH*WP + ow(s)*SW            (per lane, fixed)
//   off(k)  = (ic - ic0)*NR*WP + kh*WP + kw               (table built once)
//
// An input element is fetched about NR / R times per 64 output channels
// (C5 with 112-pixel tiles: 5 rows staged per 2 output rows) instead of
// KH*KW times, and the k-loop has no bounds tests.  Each of the 4 waves
// computes 16 output channels x the whole tile: per 16 k one 16-byte read of
// four tap offsets, 4*FN LDS reads of B and 4*FN v_mfma_f32_16x16x4_f32 (the
// library's k-permutation: lane group g feeds MFMA q with k = 4g + q).  The
// filter comes straight from L2 into registers two 16-k groups ahead; the
// next chunk's window is staged through registers a slice per group (both
// described at the loop below).  A chunk holds ICT*KH*KW taps padded to a
// multiple of 16; padded taps read a zero channel plane kept at the end of
// each window buffer (never a staged value, so an Inf input cannot turn a
// padded 0 * x into NaN).  rowwin_plan() picks TN and ICT.
//
// TWO_LEVEL: the FP32 backward-data route's two-level k sum -- each run of
// 32 consecutive k is summed from zero, then added to the total.

constexpr int RF_BM = 64, RF_NT = 256;
constexpr int RF_KCP_MAX = 1024;   // taps per chunk (padded): the offset table's size
constexpr int RF_CPG = 2;          // window channels staged per 16-k group
constexpr int RF_LDS_MAX = 64 * 1024;

struct RfArgs {
    const float* x;      // [B][IC][IH][IW]
    const float* w;      // [OC][Kc]
    const float* bias;   // [OC] or null
    float* y;            // [B][OC][S]
    int IC, OC, IH, IW, OW, S, KW, KHW, SH, SW, PH, PW, Kc, plane;
    int ICT, NR, WP, CP;      // channels per chunk, staged rows, row pitch, channel pitch
    int kc_real, KCP;         // ICT*KHW taps per chunk, padded to a multiple of 16
    int EB;                   // window buffer: ICT + 1 channel planes, the last all zero
    int nchunks, tiles_img;
    int64_t img_x, img_y;     // IC*IH*IW, OC*S
    DivMagic div_ow, div_wp, div_tiles, div_khw, div_kw;
    int IW4;    // IW / 4 (vector staging)
    // split last round (RUN forms, one channel block): workgroups
    // [0, n_full) take whole tiles, [n_full, n_full + n_half) half tiles
    // (tile n_full + h/2, output channels 32 (h%2) .. +32); n_full = 0: off
    uint32_t n_full, n_half;
};

// PP: window positions per thread (CP <= 256 PP).  MASKED: a chunk has
// padded taps or the last chunk has fewer than ICT channels, so some filter
// values read are zeroed; otherwise every filter element read is in range
// and used as loaded.  RUN (stride-1 columns, FN dividing OW): column n of
// pixel block j is pixel s0 + FN*n + j instead of s0 + 16*j + n, so a
// lane's FN pixels are consecutive in one output row and their window
// addresses are one per-tap base plus the constants 4*j (the LDS reads'
// immediate offsets): 4 address adds per 16-k group instead of 4*FN.
//
// HALF: the workgroup takes half a tile -- output channels 32 * oc_half ..
// +32 -- and its waves split each 16-k group's four MFMA k-steps: wave w
// computes channels 16 (w & 1) .. +16 over k-steps 2 (w >> 1) and
// 2 (w >> 1) + 1, and the two halves of every output are added in the
// epilogue (k-steps 0-1 + k-steps 2-3).  A last round of 2r half tiles
// instead of r whole ones puts 3.5 tiles' MFMA work on every CU at C5
// (896 tiles on 256 CUs) where whole tiles put 4 on half of them.
template <int FN, int PP, bool VECW, bool MASKED, bool TWO_LEVEL, bool RUN, bool VST, bool HALF>
__device__ __forceinline__ void rowwin_body(const RfArgs& p, uint32_t bx, uint32_t by,
                                            int oc_half) {
    constexpr int TN = 16 * FN;   // output pixels per tile
    // LDS: tap byte offsets [KCP] | window buffer 0 [EB] | window buffer 1 [EB]
    extern __shared__ __attribute__((aligned(16))) int rf_smem[];
    int* off = rf_smem;
    float* lf = reinterpret_cast<float*>(rf_smem + p.KCP);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lq = lane >> 4;
    // each wave: 16 output channels x the tile's TN pixels (HALF: over half
    // of the k-steps)
    const int wm0 = HALF ? 32 * oc_half + 16 * (wave & 1) : wave * 16;
    const int hq = HALF ? wave >> 1 : 0;

    const uint32_t b = div_u31(bx, p.div_tiles);
    const int s0 = (int)(bx - b * (uint32_t)p.tiles_img) * TN;
    const int oc0 = by * RF_BM;
    const int oh_lo = (int)div_u31((uint32_t)s0, p.div_ow);
    const float* ximg = p.x + (int64_t)b * p.img_x;

    // tap byte offsets of one chunk (the same for every chunk); padded taps
    // read the zero plane (channel ICT); and the zero planes themselves
    const int zplane = p.ICT * p.CP;
    for (int k = tid; k < p.KCP; k += RF_NT) {
        int o = zplane;
        if (k < p.kc_real) {
            const uint32_t icl = div_u31((uint32_t)k, p.div_khw);
            const uint32_t t = (uint32_t)k - icl * (uint32_t)p.KHW;
            const uint32_t kh = div_u31(t, p.div_kw);
            const uint32_t kw = t - kh * (uint32_t)p.KW;
            o = (int)(icl * (uint32_t)p.CP + kh * (uint32_t)p.WP + kw);
        }
        off[k] = 4 * o;
    }
    if constexpr (VST) {
        // both window buffers all zero: vector staging writes only the
        // input's own columns of in-image rows, so the padding columns,
        // rows outside the image and the zero planes stay zero
        // (16-byte stores: lf is 16-byte aligned, KCP being a multiple of 16)
        const int n4 = (2 * p.EB) >> 2;
        for (int i = tid; i < n4; i += RF_NT)
            reinterpret_cast<floatx4*>(lf)[i] = floatx4{0.f, 0.f, 0.f, 0.f};
        for (int i = 4 * n4 + tid; i < 2 * p.EB; i += RF_NT) lf[i] = 0.0f;
        __syncthreads();
    } else {
        for (int i = tid; i < p.CP; i += RF_NT) {
            lf[zplane + i] = 0.0f;
            lf[p.EB + zplane + i] = 0.0f;
        }
    }

    // this lane's pixel offsets in the window (pixels past the image read
    // the tile's first pixel; their results are not stored)
    // (RUN: a lane's run of FN pixels lies wholly inside or past the image,
    // since S and the run's first pixel are multiples of FN)
    int base[FN];
#pragma unroll
    for (int j = 0; j < (RUN ? 1 : FN); ++j) {
        const int s = RUN ? s0 + FN * l16 : s0 + 16 * j + l16;
        const uint32_t sc = (uint32_t)(s < p.S ? s : s0);
        const uint32_t oh = div_u31(sc, p.div_ow);
        const int ow = (int)(sc - oh * (uint32_t)p.OW);
        base[j] = ((int)oh - oh_lo) * p.SH * p.WP + ow * p.SW;
    }

    // Staging.  This thread's window positions q = tid + 256 m (m < PP) of
    // every channel: in-plane input offset (0 outside the image) and
    // validity, decoded once per workgroup.  The next chunk's window goes
    // through registers RF_CPG channels at a time, one slice per 16-k group:
    // loaded before the group's filter loads and stored into the other
    // window buffer after its MFMAs, so few registers stay live and the
    // filter loads stay in flight.  Loads are issued from in-range addresses;
    // out-of-image positions and channels past IC are zeroed when stored.
    constexpr int SPP = VST ? 1 : PP;   // scalar positions per thread
    int pos[SPP];
    uint32_t pos_ok = 0;
    if constexpr (!VST) {
        const int ih_lo = oh_lo * p.SH - p.PH;
#pragma unroll
        for (int m = 0; m < SPP; ++m) {
            const int q = tid + RF_NT * m;
            const uint32_t qc = (uint32_t)(q < p.CP ? q : 0);
            const uint32_t r = div_u31(qc, p.div_wp);
            const int ih = ih_lo + (int)r, iw = (int)(qc - r * (uint32_t)p.WP) - p.PW;
            const bool ok = q < p.CP && (unsigned)ih < (unsigned)p.IH && (unsigned)iw < (unsigned)p.IW;
            pos[m] = ok ? ih * p.IW + iw : 0;
            pos_ok |= ok ? 1u << m : 0u;
        }
    }
    // Vector staging (VST: stride-1 rows, IW % 4 == 0, 16-byte aligned
    // input): slot t = tid + 256 m of a group covers channel t / (NR*IW4) of
    // the group, window row r and input columns 4 c4 .. 4 c4 + 3 -- one
    // 16-byte load and four LDS stores (the window rows keep their pitch, so
    // the columns are 4-byte aligned only); slots on rows outside the image
    // load from the plane's start and store nothing.
    int vg[VST ? PP : 1], vl[VST ? PP : 1], vh[VST ? PP : 1];
    uint32_t vmask = 0;
    if constexpr (VST) {
        const int per_ch = p.NR * p.IW4;
        const int ih_lo = oh_lo * p.SH - p.PH;
#pragma unroll
        for (int m = 0; m < PP; ++m) {
            const int t = tid + RF_NT * m;
            const int h = t / per_ch, rem = t - h * per_ch;
            const int r = rem / p.IW4, c4 = rem - r * p.IW4;
            const int ih = ih_lo + r;
            const bool act = t < RF_CPG * per_ch && (unsigned)ih < (unsigned)p.IH;
            vg[m] = act ? ih * p.IW + 4 * c4 : 0;
            vl[m] = r * p.WP + p.PW + 4 * c4;
            vh[m] = h < RF_CPG ? h : 0;
            vmask |= act ? 1u << m : 0u;
        }
    }
    using VSlice = floatx4[VST ? PP : 1];
    VSlice vv;
    auto vslice_load_to = [&](VSlice& d, int c, int g) {
#pragma unroll
        for (int m = 0; m < PP; ++m) {
            const int icl = min(RF_CPG * g + vh[m], p.ICT - 1), ic = c * p.ICT + icl;
            const int icc = ic < p.IC ? ic : 0;
            d[m] = *reinterpret_cast<const floatx4*>(ximg + (int64_t)icc * p.plane + vg[m]);
        }
    };
    auto vslice_store_from = [&](const VSlice& sv4, int c, int dst, int g) {
#pragma unroll
        for (int m = 0; m < PP; ++m) {
            const int icl = min(RF_CPG * g + vh[m], p.ICT - 1), ic = c * p.ICT + icl;
            const bool keep = ic < p.IC;
            floatx4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float u = opaque(sv4[m][e]);
                v[e] = keep ? u : 0.0f;
            }
            if ((vmask >> m) & 1) {
                float* d = lf + dst + icl * p.CP + vl[m];
                d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
            }
        }
    };
    auto vslice_load = [&](int c, int g) { vslice_load_to(vv, c, g); };
    auto vslice_store = [&](int c, int dst, int g) { vslice_store_from(vv, c, dst, g); };

    // (groups past the chunk's channels restage its last channel: the same
    // values again, so every group issues the same loads and stores)
    using SSlice = float[RF_CPG][SPP];
    SSlice sv;
    auto sslice_load_to = [&](SSlice& d, int c, int g) {
#pragma unroll
        for (int h = 0; h < RF_CPG; ++h) {
            const int icl = min(RF_CPG * g + h, p.ICT - 1), ic = c * p.ICT + icl;
            const int icc = ic < p.IC ? ic : 0;   // wave-uniform
            const float* src = ximg + icc * p.plane;
#pragma unroll
            for (int m = 0; m < SPP; ++m) d[h][m] = src[pos[m]];
        }
    };
    auto sslice_store_from = [&](const SSlice& sd, int c, int dst, int g) {
#pragma unroll
        for (int h = 0; h < RF_CPG; ++h) {
            const int icl = min(RF_CPG * g + h, p.ICT - 1), ic = c * p.ICT + icl;
            const uint32_t ok = ic < p.IC ? pos_ok : 0u;
            float* d = lf + dst + icl * p.CP + tid;
#pragma unroll
            for (int m = 0; m < SPP; ++m) {
                const float v = opaque(sd[h][m]);
                if (tid + RF_NT * m < p.CP) d[RF_NT * m] = (ok >> m) & 1 ? v : 0.0f;
            }
        }
    };
    auto slice_load = [&](int c, int g) {
        if constexpr (VST) vslice_load(c, g);
        else sslice_load_to(sv, c, g);
    };
    auto slice_store = [&](int c, int dst, int g) {
        if constexpr (VST) vslice_store(c, dst, g);
        else sslice_store_from(sv, c, dst, g);
    };

    // filter fragments for one 16-k group: row oc0 + wm0 + l16 (rows past
    // OC read row 0; their results are not stored), k = 4 lq + q of the
    // group
    const int nkg = p.KCP / 16;
    int ld_c = 0, ld_g = 0;   // the next group to load
    const float* wrow[1];
    {
        const int oc = oc0 + wm0 + l16;
        wrow[0] = p.w + (int64_t)(oc < p.OC ? oc : 0) * p.Kc;
    }
    struct AFrag { float v[1][4]; uint32_t ok; };
    auto a_load = [&](AFrag& a) {
        // prefetches past the last group re-read the last group (unused)
        const int lc = ld_c < p.nchunks ? ld_c : p.nchunks - 1;
        const int kl = 16 * ld_g + 4 * lq;
        const int kg = lc * p.kc_real + kl;
        uint32_t ok = 0xFu;
#pragma unroll
        for (int i = 0; i < 1; ++i) {
            if constexpr (VECW) {
                bool in = true;
                if constexpr (MASKED) in = (kl < p.kc_real) & (kg < p.Kc);
                const float4 t = *reinterpret_cast<const float4*>(wrow[i] + (in ? kg : 0));
                a.v[i][0] = t.x; a.v[i][1] = t.y; a.v[i][2] = t.z; a.v[i][3] = t.w;
                if constexpr (MASKED) ok &= in ? 0xFu : 0u;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    bool in = true;
                    if constexpr (MASKED) in = (kl + q < p.kc_real) & (kg + q < p.Kc);
                    a.v[i][q] = wrow[i][in ? kg + q : 0];
                    if constexpr (MASKED) ok &= in ? 0xFu : ~(1u << q);
                }
            }
        }
        a.ok = ok;
        if (++ld_g == nkg) { ld_g = 0; ++ld_c; }
    };

    floatx4 acc[FN], part[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[j] = part[j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // per chunk: byte address of each pixel block's (0, 0) tap in the
    // chunk's window buffer
    const char* lfb = reinterpret_cast<const char*>(lf);
    int pb[FN];
    auto set_buffer = [&](int buf) {
#pragma unroll
        for (int j = 0; j < (RUN ? 1 : FN); ++j) pb[j] = 4 * (buf + base[j]);
    };
    auto compute_half = [&](const AFrag& a, int g) {
        // k-steps 2 hq and 2 hq + 1 of the group (wave-uniform selects)
        const int4 o = *reinterpret_cast<const int4*>(off + 16 * g + 4 * lq);
        const int oq[2] = {hq ? o.z : o.x, hq ? o.w : o.y};
        float av[2], bv[FN][2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const float v = hq ? a.v[0][2 + q] : a.v[0][q];
            if constexpr (MASKED) {
                const float vo = opaque(v);
                av[q] = (a.ok >> (2 * hq + q)) & 1 ? vo : 0.0f;
            } else {
                av[q] = v;
            }
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const float* src = reinterpret_cast<const float*>(lfb + pb[0] + oq[q]);
#pragma unroll
            for (int j = 0; j < FN; ++j) bv[j][q] = src[j];
        }
        floatx4 (&tgt)[FN] = TWO_LEVEL ? part : acc;
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                tgt[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[q], bv[j][q], tgt[j], 0, 0, 0);
    };
    auto compute = [&](const AFrag& a, int g) {
        const int4 o = *reinterpret_cast<const int4*>(off + 16 * g + 4 * lq);
        const int oq[4] = {o.x, o.y, o.z, o.w};
        float av[4], bv[FN][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (MASKED) {
                const float v = opaque(a.v[0][q]);
                av[q] = (a.ok >> q) & 1 ? v : 0.0f;
            } else {
                av[q] = a.v[0][q];
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (RUN) {
                const float* src = reinterpret_cast<const float*>(lfb + pb[0] + oq[q]);
#pragma unroll
                for (int j = 0; j < FN; ++j) bv[j][q] = src[j];
            } else {
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    bv[j][q] = *reinterpret_cast<const float*>(lfb + pb[j] + oq[q]);
            }
        }
        floatx4 (&tgt)[FN] = TWO_LEVEL ? part : acc;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                tgt[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[q], bv[j][q], tgt[j], 0, 0, 0);
    };
    auto fold = [&]() {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            acc[j] += part[j];
            part[j] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    };

    // Within each loop below every group issues the same loads, so the code
    // is straight-line and each wait covers only the loads it needs.  Two
    // filter fragment sets alternate: a group computes with its set, then
    // refills it with the group two ahead (no register copies, so a refill
    // is waited for only when its group starts).
    const int groups = p.nchunks * nkg;
    AFrag a0, a1;
    a_load(a0);
    a_load(a1);
    {
        // chunk 0's window with NPRO groups' slices in flight at a time (the
        // accumulators and B fragments are not live yet; loads of groups
        // past the chunk's channels are clamped to its last channel)
        constexpr int NPRO = (VST ? PP : SPP) == 1 ? 4 : (VST ? PP : SPP) == 2 ? 2 : 1;
        VSlice pv[VST ? NPRO : 1];
        SSlice ps[VST ? 1 : NPRO];
        for (int g0 = 0; g0 * RF_CPG < p.ICT; g0 += NPRO) {
#pragma unroll
            for (int i = 0; i < NPRO; ++i) {
                if constexpr (VST) vslice_load_to(pv[i], 0, g0 + i);
                else sslice_load_to(ps[i], 0, g0 + i);
            }
#pragma unroll
            for (int i = 0; i < NPRO; ++i) {
                if ((g0 + i) * RF_CPG < p.ICT) {
                    if constexpr (VST) vslice_store_from(pv[i], 0, 0, g0 + i);
                    else sslice_store_from(ps[i], 0, 0, g0 + i);
                }
            }
        }
    }
    __syncthreads();
    int gi = 0, c = 0, g = 0;
    int cb = 0, nb = p.EB;   // window buffer of chunk c, and of chunk c + 1
    set_buffer(cb);
    auto step = [&](AFrag& a, auto stage) {
        // STAGE: stage chunk c + 1's window (every chunk but the last).
        // (scheduling barriers keep the slice loads ahead of the MFMAs and
        // the slice stores, which wait for them, behind)
        // (wave priority 1 from the slice loads through the filter refill,
        // the slice stores at 0: on a SIMD shared with waves storing their
        // slices, this wave's MFMA chain issues first -- C5 forward 72.6 ->
        // 71.5 us, backward data 75.3 -> 73.9, 7x7 380 -> 373, same bits)
        constexpr bool STAGE = decltype(stage)::value;
        __builtin_amdgcn_s_setprio(1);
        if constexpr (STAGE) slice_load(c + 1, g);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (HALF) compute_half(a, g);
        else compute(a, g);
        a_load(a);
        if (TWO_LEVEL && (gi & 1)) fold();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        if constexpr (STAGE) slice_store(c + 1, nb, g);
        ++gi;
        if (++g == nkg) {
            if constexpr (STAGE) {
                // the rest of chunk c + 1's window (chunks with fewer groups
                // than channel pairs: 1x1 taps); then every wave's reads of
                // buffer cb and writes of buffer nb are complete
                for (int h = nkg; h * RF_CPG < p.ICT; ++h) {
                    slice_load(c + 1, h);
                    slice_store(c + 1, nb, h);
                }
                __syncthreads();
            }
            ++c;
            g = 0;
            const int t = cb; cb = nb; nb = t;
            set_buffer(cb);
        }
    };
    // groups of chunks 0 .. nchunks-2 stage the next chunk; the last
    // chunk's do not (group t computes with a0 for even t, a1 for odd t)
    const std::bool_constant<true> staged;
    const std::bool_constant<false> last;
    const int gs = (p.nchunks - 1) * nkg;
    int t = 0;
    for (; t + 1 < gs; t += 2) {
        step(a0, staged);
        step(a1, staged);
    }
    if (gs & 1) {
        step(a0, staged);
        for (t = gs; t + 1 < groups; t += 2) {
            step(a1, last);
            step(a0, last);
        }
        if (t < groups) step(a1, last);
    } else {
        for (t = gs; t + 1 < groups; t += 2) {
            step(a0, last);
            step(a1, last);
        }
        if (t < groups) step(a0, last);
    }
    if (TWO_LEVEL && (groups & 1)) fold();

    // D layout of a 16x16 block: register r of lane l is row 4*(l/16) + r,
    // column l % 16; output (oc, s) -> y[b][oc][s] + bias[oc]
    float* yimg = p.y + (int64_t)b * p.img_y;
    if constexpr (RUN) {
        // (a lane's pixels are FN apart across its 16-lane row: the tile goes
        // through LDS -- [64 channels][TN pixels] at a pitch of TN + 1 -- so
        // that each store instruction writes consecutive pixels of a row)
        // (HALF: rows 0-31 hold k-steps 0-1 of the half tile's 32 channels,
        // rows 32-63 k-steps 2-3)
        constexpr int TP = TN + 1;
        float* tile = reinterpret_cast<float*>(rf_smem);
        __syncthreads();   // every wave's last window reads are done
        const int row0 = HALF ? 32 * hq + 16 * (wave & 1) : wm0;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) tile[(row0 + 4 * lq + r) * TP + FN * l16 + j] = acc[j][r];
        __syncthreads();
        const int npx = p.S - s0 < TN ? p.S - s0 : TN;
        constexpr int ROWS = HALF ? RF_BM / 2 : RF_BM;
        for (int i = tid; i < ROWS * TN; i += RF_NT) {
            const int ocl = i / TN, px = i - ocl * TN;
            const int oc = oc0 + (HALF ? 32 * oc_half : 0) + ocl;
            float v = tile[ocl * TP + px];
            if constexpr (HALF) v += tile[(ocl + 32) * TP + px];
            if (px < npx && oc < p.OC)
                yimg[(int64_t)oc * p.S + s0 + px] = v + (p.bias ? p.bias[oc] : 0.0f);
        }
    } else {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int s = s0 + 16 * j + l16;
            if (s >= p.S) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int oc = oc0 + wm0 + 4 * lq + r;
                if (oc < p.OC)
                    yimg[(int64_t)oc * p.S + s] = acc[j][r] + (p.bias ? p.bias[oc] : 0.0f);
            }
        }
    }
}

template <int FN, int PP, bool VECW, bool MASKED, bool TWO_LEVEL, bool RUN, bool VST>
__global__ __launch_bounds__(RF_NT)
void conv_rowwin_kernel(RfArgs p) {
    // Workgroups go to the 8 XCDs round-robin by linear id; where the grid
    // allows, the ids are renumbered so that consecutive pixel tiles (whose
    // windows share halo rows) run on one XCD and share its L2.
    const uint32_t lin = blockIdx.x + gridDim.x * blockIdx.y;
    auto xcd_order = [](uint32_t i, uint32_t n) {
        return n % 8 == 0 ? (i % 8) * (n / 8) + i / 8 : i;
    };
    if constexpr (RUN) {
        if (p.n_full > 0) {   // one channel block (gridDim.y == 1)
            if (lin < p.n_full) {
                rowwin_body<FN, PP, VECW, MASKED, TWO_LEVEL, RUN, VST, false>(p, xcd_order(lin, p.n_full), 0, 0);
            } else {
                const uint32_t u = xcd_order(lin - p.n_full, p.n_half);
                rowwin_body<FN, PP, VECW, MASKED, TWO_LEVEL, RUN, VST, true>(p, p.n_full + u / 2, 0, (int)(u & 1));
            }
            return;
        }
    }
    const uint32_t l = xcd_order(lin, gridDim.x * gridDim.y);
    rowwin_body<FN, PP, VECW, MASKED, TWO_LEVEL, RUN, VST, false>(p, l % gridDim.x, l / gridDim.x, 0);
}

// Launch plan of the row-window form, or ok = false where no window fits
// (then the gather form above runs).
struct RfPlan {
    bool ok = false;
    int fn = 0, ict = 0, nr = 0, wp = 0, kcp = 0, eb = 0, pp = 0;
    int vpp = 0;     // 16-byte staging slots per thread, 0: scalar staging only
    size_t lds = 0;
};

// Tile width and channel chunk: the choice that gives the busiest CU the
// least work -- ceil(workgroups / 256 CUs) tiles of TN pixels, times the
// padded-tap waste, plus 15 % where those tiles are more than its LDS lets
// one CU hold at once (a partial second round runs a CU at low occupancy);
// near-ties (within 3 %) go to more channels per chunk, then wider tiles.
// (C5, 32 x 64 x 56^2, 3x3: 112-pixel tiles of 16 channels, 896 workgroups
// at 4 per CU; 128-pixel tiles leave 800 workgroups at 3 per CU, 32 of
// them in a second round.)
RfPlan rowwin_plan(int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH,
                   int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW, bool two_level) {
    RfPlan best;
    const int64_t OH = (IH + 2 * PH - KH) / SH + 1, OW = (IW + 2 * PW - KW) / SW + 1;
    const int64_t lim = INT32_MAX / 2;
    const int64_t S = OH * OW, khw = KH * KW;
    // 32-bit in-image, pixel, tap and filter indices
    if (OH < 1 || OW < 1 || S >= lim || IC * IH * IW >= lim || OC * S >= lim ||
        IC * khw >= lim || OC * IC * khw >= lim || batch * S >= lim ||
        PH >= lim || PW >= lim || OH * SH + KH >= lim || OW * SW + KW >= lim)
        return best;
    double best_cost = 0.0;
    for (const int fn : {8, 7, 5}) {
        const int64_t tn = 16 * fn;
        const int64_t rows = std::min<int64_t>(OH, (OW - 1 + tn - 1) / OW + 1);
        const int64_t nr = (rows - 1) * SH + KH, wp0 = (OW - 1) * SW + KW;
        // vector staging: stride-1 rows of whole 16-byte groups
        const bool vst = SW == 1 && OW % fn == 0 && IW % 4 == 0 &&
                         RF_CPG * nr * (IW / 4) <= 4 * RF_NT;
        const int64_t wp = wp0, cp = nr * wp;
        if (cp > 4 * RF_NT) continue;   // at most 4 window positions per thread
        const int pp = cp <= RF_NT ? 1 : cp <= 2 * RF_NT ? 2 : 4;
        const int64_t vslots = ceil_div(RF_CPG * nr * (IW / 4), RF_NT);
        const int vpp = vst ? (vslots <= 1 ? 1 : vslots <= 2 ? 2 : 4) : 0;
        const bool run = SW == 1 && OW % fn == 0;
        // workgroups per CU the registers allow (4 waves each): 4 at <= 128
        // VGPRs -- every one-level form, and the two-level forms with
        // consecutive-pixel lanes except those with 4 slots per thread and
        // FN 8 (scalar staging) or FN >= 7 (vector staging) -- else 3 (the
        // other two-level forms: up to ~152 VGPRs in the gfx950 build)
        const int64_t by_regs =
            !two_level ? 4
            : !run     ? 3
            : vst      ? (vpp == 4 && fn >= 7 ? 3 : 4)
                       : (fn <= 7 || pp <= 2 ? 4 : 3);
        const int64_t wgs = batch * ceil_div(S, tn) * ceil_div(OC, RF_BM);
        const int64_t per_cu = ceil_div(wgs, 256);
        int64_t ict = 16;
        while (ict > 1 && ict / 2 >= IC) ict /= 2;
        for (; ict >= 1; ict /= 2) {
            const int64_t kcp = ceil_div(ict * khw, 16) * 16;
            // (consecutive-pixel lanes stage the output tile through LDS too)
            const int64_t lds = std::max<int64_t>((kcp + 2 * (ict + 1) * cp) * 4,
                                                  run ? (int64_t)RF_BM * (tn + 1) * 4 : 0);
            if (lds > RF_LDS_MAX || kcp > RF_KCP_MAX) continue;
            const int64_t resident = std::min<int64_t>(by_regs, (160 * 1024) / lds);
            const double cost = (double)per_cu * tn * ((double)kcp / (double)(ict * khw)) *
                                (per_cu > resident ? 1.15 : 1.0);
            if (!best.ok || cost < best_cost * 0.97) {
                best.ok = true;
                best_cost = cost;
                best.fn = fn; best.ict = (int)ict; best.nr = (int)nr; best.wp = (int)wp;
                best.kcp = (int)kcp; best.eb = (int)((ict + 1) * cp);
                best.pp = pp;
                best.vpp = vpp;
                best.lds = (size_t)lds;
            }
        }
    }
    return best;
}

template <int FN, int PP, bool VECW, bool MASKED, bool RUN, bool VST>
void rowwin_go_run(const RfArgs& p, bool two_level, dim3 grid, size_t lds, hipStream_t stream) {
    if (two_level)
        hipLaunchKernelGGL((conv_rowwin_kernel<FN, PP, VECW, MASKED, true, RUN, VST>), grid, dim3(RF_NT), lds, stream, p);
    else
        hipLaunchKernelGGL((conv_rowwin_kernel<FN, PP, VECW, MASKED, false, RUN, VST>), grid, dim3(RF_NT), lds, stream, p);
}

// vst: vector staging (PP then counts 16-byte slots per thread)
template <int FN, int PP, bool VECW, bool MASKED>
void rowwin_go(const RfArgs& p, bool two_level, bool vst, dim3 grid, size_t lds, hipStream_t stream) {
    if (vst)
        rowwin_go_run<FN, PP, VECW, MASKED, true, true>(p, two_level, grid, lds, stream);
    else if (p.SW == 1 && p.OW % FN == 0)
        rowwin_go_run<FN, PP, VECW, MASKED, true, false>(p, two_level, grid, lds, stream);
    else
        rowwin_go_run<FN, PP, VECW, MASKED, false, false>(p, two_level, grid, lds, stream);
}

template <int FN, int PP>
void rowwin_go_pp(const RfArgs& p, bool vecw, bool masked, bool two_level, bool vst, dim3 grid,
                  size_t lds, hipStream_t stream) {
    if (vecw) {
        if (masked) rowwin_go<FN, PP, true, true>(p, two_level, vst, grid, lds, stream);
        else rowwin_go<FN, PP, true, false>(p, two_level, vst, grid, lds, stream);
    } else {
        if (masked) rowwin_go<FN, PP, false, true>(p, two_level, vst, grid, lds, stream);
        else rowwin_go<FN, PP, false, false>(p, two_level, vst, grid, lds, stream);
    }
}

template <int FN>
void rowwin_go_fn(const RfArgs& p, int pp, bool vecw, bool masked, bool two_level, bool vst,
                  dim3 grid, size_t lds, hipStream_t stream) {
    if (pp == 1) rowwin_go_pp<FN, 1>(p, vecw, masked, two_level, vst, grid, lds, stream);
    else if (pp == 2) rowwin_go_pp<FN, 2>(p, vecw, masked, two_level, vst, grid, lds, stream);
    else rowwin_go_pp<FN, 4>(p, vecw, masked, two_level, vst, grid, lds, stream);
}

int launch_rowwin(const float* x, const float* w, const float* bias, float* y, int64_t batch,
                  int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                  int64_t SH, int64_t SW, int64_t PH, int64_t PW, const RfPlan& pl,
                  bool two_level, hipStream_t stream) {
    const int64_t OH = (IH + 2 * PH - KH) / SH + 1, OW = (IW + 2 * PW - KW) / SW + 1;
    RfArgs p;
    p.x = x;
    p.IC = (int)IC; p.IH = (int)IH; p.IW = (int)IW; p.OW = (int)OW; p.S = (int)(OH * OW);
    p.KW = (int)KW; p.KHW = (int)(KH * KW); p.SH = (int)SH; p.SW = (int)SW;
    p.PH = (int)PH; p.PW = (int)PW; p.Kc = (int)(IC * KH * KW); p.plane = (int)(IH * IW);
    p.ICT = pl.ict; p.NR = pl.nr; p.WP = pl.wp; p.CP = pl.nr * pl.wp;
    p.IW4 = (int)(IW / 4);
    // vector staging where the rows allow it and the input is 16-byte
    // aligned
    const bool vst = pl.vpp > 0 && (uintptr_t)x % 16 == 0;
    const int pp = vst ? pl.vpp : pl.pp;
    p.kc_real = pl.ict * p.KHW; p.KCP = pl.kcp; p.EB = pl.eb;
    p.nchunks = (int)ceil_div(IC, pl.ict);
    p.tiles_img = (int)ceil_div(p.S, 16 * pl.fn);
    p.img_x = IC * IH * IW; p.img_y = OC * OH * OW;
    p.div_ow = div_magic(OW); p.div_wp = div_magic(p.WP);
    p.div_tiles = div_magic(p.tiles_img); p.div_khw = div_magic(p.KHW); p.div_kw = div_magic(KW);
    const bool vecw = p.Kc % 4 == 0 && p.kc_real % 4 == 0 && (uintptr_t)w % 16 == 0;
    const bool masked = IC % pl.ict != 0 || p.kc_real != p.KCP;
    // Split last round (consecutive-pixel forms with one channel block, at
    // most four tiles per CU so that all are resident at once): whole tiles
    // for the whole rounds of 256 CUs, the remaining r <= 128 tiles as 2r
    // half tiles, so no CU holds more than half a tile above the average.
    p.n_full = p.n_half = 0;
    {
        const int64_t T = batch * p.tiles_img, rem = T % 256;
        if (SW == 1 && OW % pl.fn == 0 && OC <= RF_BM && T > 256 && T <= 4 * 256 && rem > 0 &&
            rem <= 128) {
            p.n_full = (uint32_t)(T - rem);
            p.n_half = (uint32_t)(2 * rem);
        }
    }
    const int64_t chunk = (int64_t)65535 * RF_BM;   // output channels per launch (grid y)
    for (int64_t oc0 = 0; oc0 < OC; oc0 += chunk) {
        const int64_t oc_n = OC - oc0 < chunk ? OC - oc0 : chunk;
        p.OC = (int)oc_n;
        p.w = w + oc0 * p.Kc;
        p.bias = bias ? bias + oc0 : nullptr;
        p.y = y + oc0 * p.S;
        const dim3 grid = p.n_full > 0 ? dim3(p.n_full + p.n_half, 1u)
                                       : dim3((unsigned)(batch * p.tiles_img), (unsigned)ceil_div(oc_n, RF_BM));
        if (pl.fn == 8) rowwin_go_fn<8>(p, pp, vecw, masked, two_level, vst, grid, pl.lds, stream);
        else if (pl.fn == 7) rowwin_go_fn<7>(p, pp, vecw, masked, two_level, vst, grid, pl.lds, stream);
        else rowwin_go_fn<5>(p, pp, vecw, masked, two_level, vst, grid, pl.lds, stream);
        const int st = hip_error(hipGetLastError(), "conv_rowwin_kernel launch");
        if (st) return st;
    }
    return CDX_OK;
}

}  // namespace

bool conv_rowwin_ok(int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH,
                    int64_t KW, int64_t SH, int64_t SW, int64_t PH, int64_t PW) {
    return rowwin_plan(batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, true).ok;
}

int launch_conv_rowwin_f32(const float* x, const float* w, const float* bias, float* y,
                           int64_t batch, int64_t IC, int64_t OC, int64_t IH, int64_t IW,
                           int64_t KH, int64_t KW, int64_t SH, int64_t SW, int64_t PH,
                           int64_t PW, bool two_level, hipStream_t stream) {
    const RfPlan pl = rowwin_plan(batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, two_level);
    if (!pl.ok)
        return set_error(CDX_ERR_UNSUPPORTED, "conv row-window kernel: window does not fit in LDS");
    return launch_rowwin(x, w, bias, y, batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, pl,
                         two_level, stream);
}

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
    // the row-window form wherever its input window fits in LDS
    const RfPlan pl = rowwin_plan(batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, false);
    if (pl.ok)
        return launch_rowwin(x, w, bias, y, batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW, pl,
                             false, stream);
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
