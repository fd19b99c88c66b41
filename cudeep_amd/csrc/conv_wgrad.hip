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
#ifndef CDX_WGRAD_ROWS_WGS
#define CDX_WGRAD_ROWS_WGS 256
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

// ---- Row-window form for 3x3, stride-1 layers ---------------------------
//
// With stride 1 the im2col rows of one input channel ic and filter row kh are
// shifts of a single input row: for the output-row segment (b, oh, ow0 ..
// ow0 + BKP) the gathered element is
//   col[(ic, kh, kw)][p] = x[b, ic, oh + kh - PH, ow0 + p + kw - PW].
// So a k-tile here is one such segment of BKP pixels (BKP = 32, 56 or 64: the
// output width rounded up, segments of 64 beyond that).  Per k-tile the
// workgroup stages into LDS the 64 dY rows of its output channels and the 3
// input rows of each of its 16 input channels -- whole-row 16-byte loads, no
// per-element index math or bounds test beyond the row and its two halo
// columns -- and a lane reads its B operand at row (ic, kh), column p + kw.
//
// Tile: 64 (OC) x 144 (16 channels x 9 taps) outputs, 12 waves of 16 x 48 (three
// per SIMD: a 6-wave workgroup of 32 x 48 leaves two SIMDs with twice the
// MFMA work of the other two, and measured slower).
// MFMA step t of a k-tile: lane (l16, lq) feeds pixel KQ*lq + t (KQ = BKP/4),
// for A and B alike, so the four lane groups together cover each pixel once.
// In LDS each input row is split into four blocks, one per lane group: block
// g holds row positions KQ*g .. KQ*g + KQ + 1 (its pixels plus the two
// columns the kw shift reaches; those are stored twice), at a pitch XB of 16
// floats (48 when KQ + 2 > 16).  Rows sit at a pitch of 3 (mod 32) floats.  A
// B read for filter row n = (ic*3 + kh)*3 + kw then lands on bank
// (n + XB*lq + t) mod 64: 16 consecutive filter rows hit 16 consecutive banks
// and the four lane groups disjoint quarters.  (Rows kept whole, the groups
// 14 pixels apart overlapped on two banks each: 48 % of LDS-active cycles
// were bank conflicts, 25 % with the blocks -- the C5 time did not change.)
// Two register staging sets keep tile k+2's loads in flight; one workgroup
// per CU (about 256 in all; two per CU with twice the slices measured slower).
// Measured on MI355X at C5 (32 x 64 x 56^2, OC 64): 84.5 us per launch plus
// the slice reduction, against 100+ us for conv_wgrad_f32_kernel.
constexpr int RW_BM = 64;
#ifndef RW_SEGS16
#define RW_SEGS16 2
#endif

// Input-channel tile ICT and wave layout.  16 channels: 12 waves of 16 x 48
// (three per SIMD; see above).  64 channels (the whole dW row of a 64-channel
// layer, so each dY row is fetched by one workgroup instead of four): 16
// waves of 16 x 144 (four per SIMD), each k-tile 126 MFMAs per wave against
// 42, so a barrier and the staging stores are spread over three times the
// work; rows of at most 56 pixels (two LDS stages of 64 x 56 dY and 192 x 56
// input values: 131 KiB).
template <int ICT> struct RwTile;
template <> struct RwTile<16> { static constexpr int NT = 768, WAVES_N = 3, FMW = 1, JB = 3; };
template <> struct RwTile<64> { static constexpr int NT = 512, WAVES_N = 4, FMW = 2, JB = 9; };

template <int BKP, int ICT>
struct RwShape {
    static constexpr int KQ = BKP / 4;                       // MFMA steps per k-tile
    static constexpr int A_STRIDE = BKP + 4;                 // dY row pitch (floats)
    static constexpr int XB = KQ + 2 <= 16 ? 16 : 48;        // x block pitch per lane group
    static constexpr int X_LEN = 3 * XB + KQ + 2;            // floats used per x row
    static constexpr int X_RS = ((X_LEN - 3 + 31) / 32) * 32 + 3;   // >= X_LEN, = 3 mod 32
    static constexpr int NT = RwTile<ICT>::NT;
    static constexpr int X_ROWS = ICT * 3;
    static constexpr int STAGE = RW_BM * A_STRIDE + X_ROWS * X_RS;
    static constexpr int NA = (RW_BM * KQ + NT - 1) / NT;       // dY float4 per thread
    static constexpr int NX = (X_ROWS * KQ + NT - 1) / NT;      // x float4 per thread
    static_assert(KQ % 2 == 0 && X_RS >= X_LEN && X_RS % 32 == 3, "row-window shape");
    // LDS column(s) of row position P (0 .. BKP+1): its own block, and the
    // previous block too for the first two positions of a block (c2 = c1 when
    // there is no second copy, so both stores can be made unconditionally)
    __device__ __forceinline__ static void cols_of(int P, int& c1, int& c2) {
        const int b = P / KQ < 3 ? P / KQ : 3;
        c1 = XB * b + P - KQ * b;
        c2 = (b >= 1 && P - KQ * (b - 1) < KQ + 2) ? XB * (b - 1) + P - KQ * (b - 1) : c1;
    }
};

struct RwArgs {
    const float* dy;   // [B][OC][OH][OW]
    const float* x;    // [B][IC][IH][IW]
    float* out;        // [splits][OC][Kc] partials (or dW when one slice)
    int64_t OC, IC, Kc;
    int IH, IW, OH, OW, PH, PW, nseg;
    int rows_total, rows_chunk;    // k-tiles (row segments) in all / per slice
    int vec_dy, vec_x;             // 16-byte loads allowed
};

// SEGS: row segments per k-tile (1, or 2 to double the MFMA work between
// barriers and the distance the register prefetch runs ahead).  WHOLE: every
// segment lies inside its dY and input rows with 16-byte loads allowed (the
// host checks OW % BKP == 0, IW >= OW and alignment), so the loads are one
// straight-line sequence: the compiler can then wait for exactly the tile
// being stored instead of for every load in flight.
template <int BKP, int ICT, int SEGS, bool WHOLE>
__global__ __launch_bounds__(RwTile<ICT>::NT)
void conv_wgrad_rows_kernel(RwArgs p) {
    using SH_ = RwShape<BKP, ICT>;
    using TL = RwTile<ICT>;
    constexpr int RW_NT = TL::NT, FMW = TL::FMW, JB = TL::JB;
    constexpr int KQ = SH_::KQ, A_STRIDE = SH_::A_STRIDE, X_RS = SH_::X_RS;
    constexpr int STAGE = SH_::STAGE, NA = SH_::NA, NX = SH_::NX;
    // (+ one slot per thread: where threads without a halo column write, so
    // the halo store is not a divergent branch)
    __shared__ __attribute__((aligned(16))) float lds[2 * SEGS * STAGE + RW_NT];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lq = lane >> 4;
    const int wm0 = (wave / TL::WAVES_N) * 16 * FMW, wn0 = (wave % TL::WAVES_N) * 16 * JB;

    const int tiles_n = (int)ceil_div(p.IC, ICT);
    // Workgroups go to the 8 XCDs round-robin by linear id.  Where the grid
    // allows, the ids are renumbered so that every tile of a k-slice runs on
    // one XCD: the tiles of a slice read the same dY rows, which its L2 then
    // fetches once instead of once per tile.
    uint32_t tile = blockIdx.x, slice = blockIdx.y;
    {
        const uint32_t total = gridDim.x * gridDim.y, per_xcd = total / 8;
        if (total % 8 == 0 && per_xcd % gridDim.x == 0) {
            const uint32_t lin = blockIdx.x + gridDim.x * blockIdx.y;
            const uint32_t l = (lin % 8) * per_xcd + lin / 8;
            tile = l % gridDim.x;
            slice = l / gridDim.x;
        }
    }
    const int64_t bm = (int64_t)(tile / tiles_n) * RW_BM;
    const int64_t bic = (int64_t)(tile % tiles_n) * ICT;
    const int r_begin = slice * p.rows_chunk;
    const int r_end = min(p.rows_total, r_begin + p.rows_chunk);
    const int nk = r_end - r_begin;

    // the row segment the next load() reads (running counters in k order)
    int ld_seg = r_begin % p.nseg;
    int ld_oh = (r_begin / p.nseg) % p.OH;
    int ld_b = r_begin / (p.nseg * p.OH);

    // This thread's staging slots are the same for every k-tile: element
    // offsets from a wave-uniform per-k-tile base, validity of the row, and
    // the LDS destination.  dY slot u: row (output channel) idx / KQ, 4-pixel
    // column q = idx % KQ; x slot u: row (channel, kh) idx / KQ, column q.
    int a_src[NA], a_dst[NA], a_q4[NA];
    bool a_ok[NA];
#pragma unroll
    for (int u = 0; u < NA; ++u) {
        const int idx = tid + u * RW_NT;
        const int row = idx / KQ, q = idx - (idx / KQ) * KQ;
        a_ok[u] = idx < RW_BM * KQ && bm + row < p.OC;
        a_src[u] = a_ok[u] ? row * p.OH * p.OW + 4 * q : 0;   // within one image's dY block
        a_dst[u] = row * A_STRIDE + 4 * q;
        a_q4[u] = 4 * q;
    }
    int x_src[NX], x_row[NX], x_q4[NX], x_kh[NX];
    bool x_ok[NX];
#pragma unroll
    for (int u = 0; u < NX; ++u) {
        const int idx = tid + u * RW_NT;
        const int row = idx / KQ, q = idx - (idx / KQ) * KQ;   // row = icl * 3 + kh
        const int icl = row / 3, kh = row - (row / 3) * 3;
        x_ok[u] = idx < SH_::X_ROWS * KQ && bic + icl < p.IC;
        x_src[u] = x_ok[u] ? icl * p.IH * p.IW + kh * p.IW + 4 * q : 0;
        x_row[u] = row * X_RS;
        x_q4[u] = 4 * q;
        x_kh[u] = kh;
    }
    // halo column hp of row tid/2 (threads 0 .. 2*X_ROWS-1): LDS position hp
    // (left of the segment) when hp < PW, else BKP + hp (right of it); input
    // column ow0 - PW + pos
    const bool h_thread = tid < 2 * SH_::X_ROWS;
    // waves holding halo threads (wave-uniform): only they load and store halo columns
    const bool h_wave = __builtin_amdgcn_readfirstlane(tid >> 6) < (2 * SH_::X_ROWS + 63) / 64;
    int h_src = 0, h_row = 0, h_c1 = 0, h_c2 = 0, h_kh = 0, h_col = 0;
    bool h_ok = false;
    if (h_thread) {
        const int row = tid >> 1, hp = tid & 1;
        const int icl = row / 3, kh = row - (row / 3) * 3;
        const int pos = hp < p.PW ? hp : BKP + hp;
        h_ok = bic + icl < p.IC;
        h_col = pos - p.PW;
        h_src = h_ok ? icl * p.IH * p.IW + kh * p.IW + h_col : 0;
        h_row = row * X_RS;
        SH_::cols_of(pos, h_c1, h_c2);
        h_kh = kh;
    }
    const float* dy_blk = p.dy + bm * p.OH * p.OW;            // this tile's first channel
    const float* x_blk = p.x + bic * p.IH * p.IW;

    // registers staging one k-tile.  ok: bit u -- va[u] is real, bit 8 + u
    // -- vx[u], bit 31 -- vh; the others are zeroed when stored (a select at
    // the load would make every load wait for its data at once).
    static_assert(NA <= 8 && NX <= 16, "ok mask layout");
    struct Stage {
        floatx4 va[NA], vx[NX];
        float vh;
        uint32_t ok;
    };
    // valid = false: a k-tile's missing last segment -- the same loads from
    // the first segment's addresses, every element marked not real (one
    // instruction sequence either way, so the waits stay exact)
    auto load = [&](Stage& st, bool valid) {
        const int l_seg = valid ? ld_seg : 0, l_oh = valid ? ld_oh : 0, l_b = valid ? ld_b : 0;
        const int ow0 = l_seg * BKP;
        // wave-uniform bases: dY row (b, oc = bm, oh) at ow0; x row (b, ic = bic,
        // ih = oh - PH) at ow0
        const float* yk = dy_blk + (int64_t)l_b * p.OC * p.OH * p.OW + (int64_t)l_oh * p.OW + ow0;
        const float* xk = x_blk + (int64_t)l_b * p.IC * p.IH * p.IW +
                          (int64_t)(l_oh - p.PH) * p.IW + ow0;
        if (WHOLE || (p.vec_dy && p.vec_x && ow0 + BKP <= p.OW && ow0 + BKP <= p.IW)) {
            // whole segment inside both rows: 16-byte loads from addresses that
            // are always valid (a skipped row reads the tile's first dY row or
            // the input's first element), zeroed at the store -- no branches
            uint32_t ok = 0;
#pragma unroll
            for (int u = 0; u < NA; ++u) {
                st.va[u] = *reinterpret_cast<const floatx4*>(yk + a_src[u]);
                ok |= (uint32_t)(a_ok[u] && valid) << u;
            }
#pragma unroll
            for (int u = 0; u < NX; ++u) {
                const bool rok = valid && x_ok[u] &&
                                 (unsigned)(l_oh - p.PH + x_kh[u]) < (unsigned)p.IH;
                const float* src = rok ? xk + x_src[u] : p.x;
                st.vx[u] = *reinterpret_cast<const floatx4*>(src);
                ok |= (uint32_t)rok << (8 + u);
            }
            st.ok = ok;
        } else {
            st.ok = 0x7fffffffu;   // elementwise-zeroed below
#pragma unroll
            for (int u = 0; u < NA; ++u) {
                const float* src = yk + a_src[u];
                const int ow = ow0 + a_q4[u];
                const bool aok = valid && a_ok[u];
                if (aok && p.vec_dy && ow + 3 < p.OW) {
                    st.va[u] = *reinterpret_cast<const floatx4*>(src);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) st.va[u][j] = aok && ow + j < p.OW ? src[j] : 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < NX; ++u) {
                const float* src = xk + x_src[u];
                const int iw = ow0 + x_q4[u];
                const bool rok = valid && x_ok[u] &&
                                 (unsigned)(l_oh - p.PH + x_kh[u]) < (unsigned)p.IH;
                if (rok && p.vec_x && iw + 3 < p.IW) {
                    st.vx[u] = *reinterpret_cast<const floatx4*>(src);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) st.vx[u][j] = rok && iw + j < p.IW ? src[j] : 0.0f;
                }
            }
        }
        if (h_wave) {
            // every thread of a halo wave loads (non-halo threads the input's
            // first element); the other waves issue no halo load at all
            const int iw = ow0 + h_col;
            const bool ok = valid && h_thread && h_ok &&
                            (unsigned)(l_oh - p.PH + h_kh) < (unsigned)p.IH &&
                            (unsigned)iw < (unsigned)p.IW;
            st.vh = *(ok ? xk + h_src : p.x);
            st.ok = (st.ok & 0x7fffffffu) | ((uint32_t)ok << 31);
        } else {
            st.vh = 0.0f;
            st.ok &= 0x7fffffffu;
        }
        if (valid && ++ld_seg == p.nseg) {
            ld_seg = 0;
            if (++ld_oh == p.OH) {
                ld_oh = 0;
                ++ld_b;
            }
        }
    };
    // (opaque: keeps the zeroing select here, away from the load)
    auto zsel = [](float v, bool keep) {
        asm volatile("" : "+v"(v));
        return keep ? v : 0.0f;
    };
    auto zsel4 = [&](floatx4 v, bool keep) {
        return floatx4{zsel(v[0], keep), zsel(v[1], keep), zsel(v[2], keep), zsel(v[3], keep)};
    };
    auto store = [&](const Stage& st, int buf) {
        float* sA = lds + buf * STAGE;
        float* sX = sA + RW_BM * A_STRIDE;
#pragma unroll
        for (int u = 0; u < NA; ++u)
            if (tid + u * RW_NT < RW_BM * KQ)
                *reinterpret_cast<floatx4*>(sA + a_dst[u]) = zsel4(st.va[u], (st.ok >> u) & 1u);
#pragma unroll
        for (int u = 0; u < NX; ++u)
            if (tid + u * RW_NT < SH_::X_ROWS * KQ) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    int c1, c2;   // (recomputed: a few integer ops per k-tile)
                    SH_::cols_of(p.PW + x_q4[u] + j, c1, c2);
                    const float v = zsel(st.vx[u][j], (st.ok >> (8 + u)) & 1u);
                    sX[x_row[u] + c1] = v;
                    sX[x_row[u] + c2] = v;
                }
            }
        if (h_wave) {
            const float v = zsel(st.vh, st.ok >> 31);
            float* dummy = lds + 2 * SEGS * STAGE + tid;
            *(h_thread ? sX + h_row + h_c1 : dummy) = v;
            *(h_thread ? sX + h_row + h_c2 : dummy) = v;
        }
    };

    // this lane's B rows: filter row n -> (channel, kh, kw) -> LDS row and shift
    int b_off[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int n = wn0 + j * 16 + l16;          // 0 .. 9 ICT - 1
        const int icl = n / 9, tap = n - (n / 9) * 9;
        const int kh = tap / 3, kw = tap - (tap / 3) * 3;
        b_off[j] = RW_BM * A_STRIDE + (icl * 3 + kh) * X_RS + SH_::XB * lq + kw;
    }
    const int a_off = (wm0 + l16) * A_STRIDE + KQ * lq;

    floatx4 acc[FMW][JB];
#pragma unroll
    for (int i = 0; i < FMW; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // (the 64-channel form steps through the k-tile without unrolling: fully
    // unrolled, the compiler hoists all 140 fragment reads of a k-tile and
    // spills)
    constexpr int T_UNROLL = JB > 3 ? 1 : KQ / 2;
    auto compute = [&](int buf) {
        const float* s = lds + buf * STAGE;
#pragma unroll T_UNROLL
        for (int t0 = 0; t0 < KQ; t0 += 2) {
            float2 a[FMW];
#pragma unroll
            for (int i = 0; i < FMW; ++i)
                a[i] = *reinterpret_cast<const float2*>(s + a_off + 16 * i * A_STRIDE + t0);
            float b[JB][2];
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                b[j][0] = s[b_off[j] + t0];
                b[j][1] = s[b_off[j] + t0 + 1];
            }
#pragma unroll
            for (int i = 0; i < FMW; ++i)
#pragma unroll
                for (int j = 0; j < JB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].x, b[j][0], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < FMW; ++i)
#pragma unroll
                for (int j = 0; j < JB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].y, b[j][1], acc[i][j], 0, 0, 0);
        }
    };

    // A k-tile is SEGS consecutive row segments, each in its own LDS
    // sub-stage (buffer buf, segment s at sub-stage buf * SEGS + s); a
    // missing last segment is staged as zeros (zero dY adds nothing).
    // (Callers load a segment only while ld_left > 0.)
    struct Group {
        Stage s[SEGS];
    };
    int ld_left = nk;   // segments not yet loaded
    auto load_g = [&](Group& gr) {
#pragma unroll
        for (int q = 0; q < SEGS; ++q) {
            load(gr.s[q], ld_left > 0);
            --ld_left;
        }
    };
    auto store_g = [&](const Group& gr, int buf) {
#pragma unroll
        for (int q = 0; q < SEGS; ++q) store(gr.s[q], buf * SEGS + q);
    };
    auto compute_g = [&](int buf) {
#pragma unroll 1
        for (int q = 0; q < SEGS; ++q) compute(buf * SEGS + q);
    };
    const int nkt = (nk + SEGS - 1) / SEGS;   // k-tiles

    // Two register staging sets: tile k+2 is loaded while tile k is
    // multiplied and tile k+1 (loaded an iteration earlier) is written to LDS.
    if ((ICT == 64 || SEGS > 1) && nkt > 0) {
        // One staging set: a k-tile's MFMAs (252 per wave, two waves per
        // SIMD, for 64 channels; 84 per wave, three per SIMD, for two
        // segments of 16 channels) outlast the next tile's loads.  With one
        // set, the wait before a store is for the newest loads only -- with
        // two, the compiler's waits at the stores also waited for the other
        // set's loads just issued.
        Group st;
        load_g(st);
        store_g(st, 0);
        __syncthreads();
        // (wave priority 1 over the MFMAs: on a SIMD shared with waves
        // storing their staging sets, the MFMA chains issue first -- C5
        // 84.9 -> 84.0 us, same bits)
        for (int k = 0; k < nkt; ++k) {
            const bool more = k + 1 < nkt;
            if (more) load_g(st);
            __builtin_amdgcn_s_setprio(1);
            compute_g(k & 1);
            __builtin_amdgcn_s_setprio(0);
            if (more) store_g(st, (k & 1) ^ 1);
            __syncthreads();
        }
    } else if (nkt > 0) {
        Group s0, s1;
        load_g(s0);
        if (nkt > 1) load_g(s1);
        store_g(s0, 0);
        __syncthreads();
        int k = 0;
        for (; k + 1 < nkt; k += 2) {       // LDS stage 0: tile k; s1: tile k+1
            if (k + 2 < nkt) load_g(s0);    // tile k+2
            compute_g(0);
            store_g(s1, 1);
            __syncthreads();
            if (k + 3 < nkt) load_g(s1);    // tile k+3
            compute_g(1);
            if (k + 2 < nkt) store_g(s0, 0);
            __syncthreads();
        }
        if (k < nkt) compute_g(0);          // odd count: the last tile, in stage 0
    }

    // D layout of a 16x16 block: register r of lane l is row 4*(l/16) + r,
    // column l % 16
    float* out = p.out + (int64_t)slice * p.OC * p.Kc;
#pragma unroll
    for (int i = 0; i < FMW; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j) {
            const int64_t nn = bic * 9 + wn0 + j * 16 + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = bm + wm0 + 16 * i + 4 * lq + r;
                if (m < p.OC && nn < p.Kc) out[m * p.Kc + nn] = acc[i][j][r];
            }
        }
}

// Pixels per k-tile: the output width rounded up to 32 / 56 / 64, or 64-pixel
// segments for wider rows.
int rw_bkp(int64_t OW) { return OW <= 32 ? 32 : OW <= 56 ? 56 : 64; }

bool rows_applies(const WgGeom& g) {
    // per-thread element offsets span at most one tile's 64 dY planes or 16
    // input planes, and the row segments are counted in int: 32-bit
    const int64_t lim = (int64_t)1 << 31;
    return g.KH == 3 && g.KW == 3 && g.SH == 1 && g.SW == 1 && g.PW >= 0 && g.PW <= 2 &&
           g.PH >= 0 && RW_BM * g.OH * g.OW < lim && 64 * g.IH * g.IW < lim &&
           g.B * g.OH * ceil_div(g.OW, rw_bkp(g.OW)) < lim;
}

struct RwPlan {
    int bkp, ict, nseg, rows_total, tiles, splits, chunk;
};

RwPlan rw_plan_for(const WgGeom& g, int ict) {
    RwPlan r;
    r.bkp = rw_bkp(g.OW);
    r.ict = ict;
    r.nseg = (int)ceil_div(g.OW, r.bkp);
    r.rows_total = (int)(g.B * g.OH * r.nseg);
    r.tiles = (int)(ceil_div(g.OC, RW_BM) * ceil_div(g.IC, r.ict));
    // about CDX_WGRAD_ROWS_WGS workgroups, at least 4 row segments per slice
    int64_t s = CDX_WGRAD_ROWS_WGS / r.tiles;
    if (s > r.rows_total / 4) s = r.rows_total / 4;
    if (s < 1) s = 1;
    r.chunk = (int)ceil_div(r.rows_total, s);
    r.splits = (int)ceil_div(r.rows_total, r.chunk);
    return r;
}

// The 64-channel tile where it applies (IC a multiple of 64, rows of at
// most 56 pixels) and each slice is at least 16 row segments long: its
// partials are four times the 16-channel form's (the whole 64 x 9 IC tile
// per workgroup), which the slice's work has to outweigh.  Measured on
// MI355X with the reduction: 64 x 128 x 56^2 552 against 626 us, 32 x 512
// x 14^2 704 against 862, 32 x 256 x 28^2 357 against 445; C5 (7 row
// segments per slice) 96 against 93, so C5 keeps the 16-channel tile.
RwPlan rw_plan(const WgGeom& g) {
    if (g.IC % 64 == 0 && rw_bkp(g.OW) <= 56) {
        const RwPlan r = rw_plan_for(g, 64);
        if (r.chunk >= 16) return r;
    }
    return rw_plan_for(g, 16);
}

template <bool WHOLE>
void launch_rows(const RwPlan& r, dim3 grid, dim3 b16, dim3 b64, const RwArgs& p,
                 hipStream_t stream) {
    if (r.ict == 64) {
        if (r.bkp == 32)
            hipLaunchKernelGGL((conv_wgrad_rows_kernel<32, 64, 1, WHOLE>), grid, b64, 0, stream, p);
        else
            hipLaunchKernelGGL((conv_wgrad_rows_kernel<56, 64, 1, WHOLE>), grid, b64, 0, stream, p);
    } else {
        if (r.bkp == 32)
            hipLaunchKernelGGL((conv_wgrad_rows_kernel<32, 16, RW_SEGS16, WHOLE>), grid, b16, 0, stream, p);
        else if (r.bkp == 56)
            hipLaunchKernelGGL((conv_wgrad_rows_kernel<56, 16, RW_SEGS16, WHOLE>), grid, b16, 0, stream, p);
        else
            hipLaunchKernelGGL((conv_wgrad_rows_kernel<64, 16, 1, WHOLE>), grid, b16, 0, stream, p);
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
    const int s = rows_applies(g) ? rw_plan(g).splits : splits_for(g);
    return s > 1 ? (size_t)s * (size_t)OC * (size_t)g.Kc() : 0;
}

int launch_conv_wgrad_f32(const float* dy, const float* x, float* dw, float* ws, int64_t batch,
                          int64_t IC, int64_t OC, int64_t IH, int64_t IW, int64_t KH, int64_t KW,
                          int64_t SH, int64_t SW, int64_t PH, int64_t PW, hipStream_t stream) {
    const WgGeom g = make_geom(batch, IC, OC, IH, IW, KH, KW, SH, SW, PH, PW);
    if (rows_applies(g)) {
        const RwPlan r = rw_plan(g);
        RwArgs p;
        p.dy = dy; p.x = x;
        p.out = r.splits > 1 ? ws : dw;
        p.OC = OC; p.IC = IC; p.Kc = g.Kc();
        p.IH = (int)IH; p.IW = (int)IW; p.OH = (int)g.OH; p.OW = (int)g.OW;
        p.PH = (int)PH; p.PW = (int)PW; p.nseg = r.nseg;
        p.rows_total = r.rows_total; p.rows_chunk = r.chunk;
        p.vec_dy = g.OW % 4 == 0 && (uintptr_t)dy % 16 == 0;
        p.vec_x = IW % 4 == 0 && (uintptr_t)x % 16 == 0;
        const dim3 grid((unsigned)r.tiles, (unsigned)r.splits);
        const dim3 b16(RwTile<16>::NT), b64(RwTile<64>::NT);
        const bool whole = p.vec_dy && p.vec_x && g.OW % r.bkp == 0 && IW >= g.OW;
        if (whole) launch_rows<true>(r, grid, b16, b64, p, stream);
        else launch_rows<false>(r, grid, b16, b64, p, stream);
        int st = hip_error(hipGetLastError(), "conv_wgrad_rows_kernel launch");
        if (st || r.splits == 1) return st;
        GemmArgs red{CDX_OP_N, CDX_OP_N, OC, g.Kc(), 0, nullptr, 1, nullptr, 1, dw, g.Kc(), 0, 0,
                     nullptr, CDX_BIAS_NONE, CDX_EPI_NONE};
        return launch_splitk_reduce(ws, r.splits, red, stream);
    }
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
