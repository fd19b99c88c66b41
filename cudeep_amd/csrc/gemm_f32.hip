// FP32 GEMM on gfx950 matrix cores: v_mfma_f32_16x16x4_f32.
//
// Replaces the reference's CUDA-core SGEMMs (sgemm_fast_kernel /
// sgemm_general_kernel, src/kernels/matmul_kernel.cu:458-689).  The
// reference computes each output as an fp32 FMA chain over k; here each
// output is an fp32 MFMA accumulation (the same fp32 products, summed by
// the matrix core four k at a time), which is what the relative-Frobenius
// parity gate compares against.
//
// Structure (per workgroup, one BM x BN output tile):
//   * A and B k-tiles of depth BK are staged global -> VGPR -> LDS with
//     register double buffering: the loads for tile t+1 are in flight while
//     the waves run the MFMAs of tile t, and one barrier per k-tile
//     separates the two LDS buffers.
//   * LDS keeps each operand in its global orientation (k-contiguous or
//     m/n-contiguous), so the staging copy is a plain 16-byte copy.  Row
//     strides are padded by 4 floats, which makes both the 16-byte stores
//     and the fragment reads bank-conflict free.
//   * Each wave owns a WM x WN sub-tile = (WM/16) x (WN/16) MFMA blocks of
//     16x16, accumulated in 4 fp32 registers per lane each.
//   * k is consumed 16 at a time: a lane feeds MFMA j (j = 0..3) with
//     k = k0 + 4*(lane/16) + j, for A and B alike, so a k-contiguous operand
//     is read with one 16-byte LDS read per fragment and the four MFMAs
//     together cover k0..k0+15 exactly once.
//   * The epilogue adds an optional per-row / per-column bias, applies
//     ReLU / GELU, and writes through the output map (plain row-major, or
//     the conv map that lands the [OC, B*S] result directly in NCHW).
//   * Workgroup -> tile order is XCD-aware: consecutive dispatch slots go
//     round-robin over the 8 XCDs, so the block id is remapped to give each
//     XCD a contiguous run of tiles, walked in GROUP_M-row groups so the
//     A row-panels and B column-panels of a run share that XCD's L2.
#include "cdx_internal.hpp"

namespace cdx {
namespace {

constexpr int kLoadAlignedVec = 0;  // every tile in bounds, 16-byte loads
constexpr int kLoadChecked = 1;     // bounds-checked; 16-byte loads where whole and the
                                    // operand allows them (per-operand flag), else scalar

struct KParams {
    const float* A; const float* B; float* C; const float* bias;
    int64_t M, N, K, lda, ldb, ldc, n_split, ldc_split;
    int bias_mode, epilogue;
    int64_t k_chunk;    // split-K: k-range per blockIdx.y slice (gridDim.y > 1)
    int64_t sa, sb, sc; // batch strides (elements) for blockIdx.z
    int64_t batch;      // gridDim.z
    int vec_a, vec_b;   // kLoadChecked: operand base, ld and batch stride allow 16-byte loads
    const float* aux;   // activation-backward epilogues: aux [M, N], leading dim ldaux
    int64_t ldaux;
    // op(B)'s own column count and the virtual ones column: with ones >= 0
    // (= nb) op(B)(k, nb) reads as 1 (checked loads only) and the kernel's N
    // is nb + 1; colsum receives that column's results.
    int64_t nb, ones;
    float* colsum;
    int interior;   // kLoadChecked: whole tiles may take the unchecked path
};

// Loads a ROWS x COLS tile (COLS contiguous in memory) starting at (r0, c0)
// of a matrix with leading dimension ld and extent (rmax, cmax) into
// registers; NT threads, each holding NV float4.
template <int ROWS, int COLS, int NT, int MODE>
struct TileLoader {
    static constexpr int C4 = COLS / 4;
    static constexpr int TOTAL = ROWS * C4;           // float4 slots in the tile
    static constexpr int NV = (TOTAL + NT - 1) / NT;
    static constexpr bool PARTIAL = TOTAL % NT != 0;  // last pass: some threads idle
    float4 v[NV];

    // ones_row / ones_col >= 0: that row / column (one past the matrix)
    // reads as 1 within the other dimension's bounds (checked mode only)
    __device__ __forceinline__ void load(const float* __restrict__ X, int64_t ld,
                                         int64_t r0, int64_t c0, int64_t rmax,
                                         int64_t cmax, bool vec, int tid,
                                         int64_t ones_row = -1, int64_t ones_col = -1) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            int idx = tid + i * NT;
            if (PARTIAL && idx >= TOTAL) break;
            int r = idx / C4, c = (idx % C4) * 4;
            int64_t gr = r0 + r, gc = c0 + c;
            const float* p = X + gr * ld + gc;
            if (MODE == kLoadAlignedVec) {
                v[i] = *reinterpret_cast<const float4*>(p);
            } else if (vec && gr < rmax && gc + 3 < cmax) {
                v[i] = *reinterpret_cast<const float4*>(p);
            } else {
                bool rok = gr < rmax;
                v[i].x = (rok && gc + 0 < cmax) ? p[0] : 0.0f;
                v[i].y = (rok && gc + 1 < cmax) ? p[1] : 0.0f;
                v[i].z = (rok && gc + 2 < cmax) ? p[2] : 0.0f;
                v[i].w = (rok && gc + 3 < cmax) ? p[3] : 0.0f;
                if (ones_col >= 0 && rok) {
                    if (gc + 0 == ones_col) v[i].x = 1.0f;
                    if (gc + 1 == ones_col) v[i].y = 1.0f;
                    if (gc + 2 == ones_col) v[i].z = 1.0f;
                    if (gc + 3 == ones_col) v[i].w = 1.0f;
                }
                if (ones_row >= 0 && gr == ones_row) {
                    v[i].x = gc + 0 < cmax ? 1.0f : 0.0f;
                    v[i].y = gc + 1 < cmax ? 1.0f : 0.0f;
                    v[i].z = gc + 2 < cmax ? 1.0f : 0.0f;
                    v[i].w = gc + 3 < cmax ? 1.0f : 0.0f;
                }
            }
        }
    }

    template <int LDS_STRIDE>
    __device__ __forceinline__ void store(float* __restrict__ s, int tid) const {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            int idx = tid + i * NT;
            if (PARTIAL && idx >= TOTAL) break;
            int r = idx / C4, c = (idx % C4) * 4;
            *reinterpret_cast<float4*>(s + r * LDS_STRIDE + c) = v[i];
        }
    }
};

// PIPE: 1 = one register staging set; 2 = two sets (tile k+2 loads while
// tile k+1 is written to LDS).
template <int BM_, int BN_, int BK_, int WM_, int WN_, int GROUP_M_, int PIPE_ = 1>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int GROUP_M = GROUP_M_;
    static constexpr int PIPE = PIPE_;
    static constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
    static constexpr int NT = WAVES_M * WAVES_N * 64;
    static constexpr int FM = WM / 16, FN = WN / 16;
};

// Maps the linear workgroup id to an output tile (tm, tn): XCD-contiguous
// runs, then GROUP_M-row groups within the run.
__device__ __forceinline__ void tile_of_block(int tiles_m, int tiles_n, int group_m,
                                              int& tm, int& tn) {
    int nb = gridDim.x;
    int bid = blockIdx.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    int per_group = group_m * tiles_n;
    int g = bid / per_group;
    int first_m = g * group_m;
    int gsize = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
    int in_g = bid - g * per_group;
    tm = first_m + in_g % gsize;
    tn = in_g / gsize;
}

// Reads V consecutive floats of one LDS row (V = 1, 2 or 4: one 4-, 8- or
// 16-byte read) into fragment slots f[blk0 .. blk0 + V - 1][j].
template <int V, int F>
__device__ __forceinline__ void read_rows(const float* p, float (&f)[F][4], int blk0, int j) {
    if constexpr (V == 4) {
        const float4 t = *reinterpret_cast<const float4*>(p);
        f[blk0][j] = t.x; f[blk0 + 1][j] = t.y; f[blk0 + 2][j] = t.z; f[blk0 + 3][j] = t.w;
    } else if constexpr (V == 2) {
        const float2 t = *reinterpret_cast<const float2*>(p);
        f[blk0][j] = t.x; f[blk0 + 1][j] = t.y;
    } else {
        f[blk0][j] = *p;
    }
}

// LDS geometry and fragment-read widths of one configuration.
//  * m/n-contiguous operands are read V consecutive rows (columns) per lane
//    with one LDS read, feeding V MFMAs whose blocks are interleaved
//    (blk_pos); k-contiguous operands keep the plain layout.  (Measured on
//    MI355X: 16-byte reads gain 1-4 %; 8-byte reads gain only on A when B is
//    read 16 bytes at a time too -- 2048^3 TN 141 -> 132 us -- and lose
//    elsewhere: 2048^3 TT 132 -> 138 us, 8192 x 784 x 256 NN on 64 x 64
//    tiles 44 -> 45 us.)
//  * k-contiguous operands are [mn][BK+4], m/n-contiguous ones [BK][mn+4]:
//    with 4-byte reads, lane groups lq = 0..3 read rows 4 apart, 16 banks
//    apart with the pad; wider reads take one contiguous row segment per
//    16 lanes.
template <class CF, int OPA, int OPB>
struct Geo {
    static constexpr int BM = CF::BM, BN = CF::BN, BK = CF::BK;
    static constexpr int VB = OPB == CDX_OP_T ? 1 : (CF::FN % 4 == 0 ? 4 : 1);
    static constexpr int VA = OPA == CDX_OP_N ? 1 : (CF::FM % 4 == 0 ? 4 : CF::FM % 2 == 0 && VB == 4 ? 2 : 1);
    static constexpr int A_STRIDE = OPA == CDX_OP_N ? BK + 4 : BM + 4;
    static constexpr int A_ELEMS = OPA == CDX_OP_N ? BM * A_STRIDE : BK * A_STRIDE;
    static constexpr int B_STRIDE = OPB == CDX_OP_N ? BN + 4 : BK + 4;
    static constexpr int B_ELEMS = OPB == CDX_OP_N ? BK * B_STRIDE : BN * B_STRIDE;
    static constexpr int LDS_FLOATS = 2 * (A_ELEMS + B_ELEMS);
};

// One workgroup's output tile (top-left (bm, bn)) over the k-range of p.
// BLK: two-level k sum -- each pair of k-tiles (32 k) is summed from zero in
// `part`, then added to `acc` (a rounding chain of ~32 + K/32 additions).
template <class CF, int OPA, int OPB, int MODE, bool SPLITN, bool BLK>
__device__ __forceinline__ void gemm_tile(const KParams& p, int64_t bm, int64_t bn, float* lds) {
    using G = Geo<CF, OPA, OPB>;
    constexpr int BK = CF::BK;
    constexpr int NT = CF::NT, FM = CF::FM, FN = CF::FN;
    constexpr int VA = G::VA, VB = G::VB;
    constexpr int A_STRIDE = G::A_STRIDE, A_ELEMS = G::A_ELEMS;
    constexpr int B_STRIDE = G::B_STRIDE, B_ELEMS = G::B_ELEMS;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave / CF::WAVES_N) * CF::WM;
    const int wn0 = (wave % CF::WAVES_N) * CF::WN;
    const int l16 = lane & 15;
    const int lq = lane >> 4;   // 0..3

    constexpr int BM = CF::BM, BN = CF::BN;
// Global tile loaders in memory orientation.
    using LA = TileLoader<OPA == CDX_OP_N ? BM : BK, OPA == CDX_OP_N ? BK : BM, NT, MODE>;
    using LB = TileLoader<OPB == CDX_OP_N ? BK : BN, OPB == CDX_OP_N ? BN : BK, NT, MODE>;
    LA la;
    LB lb;

    auto load_into = [&](LA& a, LB& b, int64_t k0) {
        if (OPA == CDX_OP_N) a.load(p.A, p.lda, bm, k0, p.M, p.K, p.vec_a, tid);
        else                 a.load(p.A, p.lda, k0, bm, p.K, p.M, p.vec_a, tid);
        // op(B)'s own columns, plus the ones column when p.ones >= 0
        if (OPB == CDX_OP_N) b.load(p.B, p.ldb, k0, bn, p.K, p.nb, p.vec_b, tid, -1, p.ones);
        else                 b.load(p.B, p.ldb, bn, k0, p.nb, p.K, p.vec_b, tid, p.ones, -1);
    };
    auto store_from = [&](const LA& a, const LB& b, int buf) {
        float* sA = lds + buf * (A_ELEMS + B_ELEMS);
        float* sB = sA + A_ELEMS;
        a.template store<A_STRIDE>(sA, tid);
        b.template store<B_STRIDE>(sB, tid);
    };

    floatx4 acc[FM][FN], part[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
            part[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    floatx4 (&tgt)[FM][FN] = BLK ? part : acc;
    // BLK: fold the partial sum into the total and restart it
    auto flush = [&]() {
        if (!BLK) return;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                acc[i][j] += part[i][j];
                part[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
    };

    // MFMAs over the k-tile held in LDS stage `buf`, into `tgt`
    auto compute = [&](int buf) {
        const float* sA = lds + buf * (A_ELEMS + B_ELEMS);
        const float* sB = sA + A_ELEMS;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            float a[FM][4], b[FN][4];
            if constexpr (OPA == CDX_OP_N) {
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    const int m = wm0 + i * 16 + l16;
                    float4 t = *reinterpret_cast<const float4*>(sA + m * A_STRIDE + kk + 4 * lq);
                    a[i][0] = t.x; a[i][1] = t.y; a[i][2] = t.z; a[i][3] = t.w;
                }
            } else {
#pragma unroll
                for (int g = 0; g < FM / VA; ++g)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        read_rows<VA>(sA + (kk + 4 * lq + j) * A_STRIDE + wm0 + 16 * VA * g + VA * l16,
                                      a, g * VA, j);
            }
            if constexpr (OPB == CDX_OP_T) {
#pragma unroll
                for (int jn = 0; jn < FN; ++jn) {
                    const int n = wn0 + jn * 16 + l16;
                    float4 t = *reinterpret_cast<const float4*>(sB + n * B_STRIDE + kk + 4 * lq);
                    b[jn][0] = t.x; b[jn][1] = t.y; b[jn][2] = t.z; b[jn][3] = t.w;
                }
            } else {
#pragma unroll
                for (int g = 0; g < FN / VB; ++g)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        read_rows<VB>(sB + (kk + 4 * lq + j) * B_STRIDE + wn0 + 16 * VB * g + VB * l16,
                                      b, g * VB, j);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int jn = 0; jn < FN; ++jn)
                        tgt[i][jn] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][j], b[jn][j],
                                                                         tgt[i][jn], 0, 0, 0);
        }
    };

    const int64_t nk = ceil_div(p.K, BK);
    if (CF::PIPE == 2 && nk >= 2) {
        // Two register staging sets: tile k+2 is loaded while tile k+1 is
        // written to LDS from the set loaded one iteration earlier, so the
        // LDS stores never wait on global memory.
        LA la1;
        LB lb1;
        load_into(la, lb, 0);
        load_into(la1, lb1, BK);
        store_from(la, lb, 0);
        __syncthreads();
        int64_t kt = 0;
        // loop invariant (kt even): stage 0 holds tile kt, set 1 tile kt+1
        for (; kt + 3 < nk; kt += 2) {
            load_into(la, lb, (kt + 2) * BK);
            compute(0);
            store_from(la1, lb1, 1);
            __syncthreads();
            load_into(la1, lb1, (kt + 3) * BK);
            compute(1);
            store_from(la, lb, 0);
            __syncthreads();
            flush();
        }
        if (kt + 2 < nk) {            // three tiles left
            load_into(la, lb, (kt + 2) * BK);
            compute(0);
            store_from(la1, lb1, 1);
            __syncthreads();
            compute(1);
            store_from(la, lb, 0);
            __syncthreads();
            flush();
            compute(0);
        } else {                      // two tiles left
            compute(0);
            store_from(la1, lb1, 1);
            __syncthreads();
            compute(1);
        }
        flush();
    } else {
        // One staging set: tile k+1 is in flight during the MFMAs of tile k.
        load_into(la, lb, 0);
        store_from(la, lb, 0);
        __syncthreads();
        for (int64_t kt = 0; kt < nk; ++kt) {
            const int buf = (int)(kt & 1);
            const bool has_next = kt + 1 < nk;
            if (has_next) load_into(la, lb, (kt + 1) * BK);
            compute(buf);
            if (has_next) store_from(la, lb, buf ^ 1);
            __syncthreads();
            if (kt & 1) flush();
        }
        flush();
    }

    // epilogue: bias, activation and the output map, straight from the
    // accumulators
    const EpiArgs epi{p.C, p.ldc, p.M, p.N, p.n_split, p.ldc_split,
                      p.bias, p.bias_mode, p.epilogue, p.aux, p.ldaux, p.colsum, p.nb};
    write_acc<FM, FN, MODE != kLoadAlignedVec, SPLITN, VA, VB>(acc, epi, bm + wm0, bn + wn0, lane);
}

// MODE kLoadChecked launches (ragged M / N, unaligned operands, the ones
// column) run their interior tiles -- clear of the edges and of the ones
// column -- through the unchecked 16-byte loads and epilogue when
// p.interior allows (both operands 16-byte loadable, K and the split-K
// chunk whole k-tiles): 8192 x 784 x 256 NN has 12 of every 13 tile
// columns interior (44 -> 40 us).
template <class CF, int OPA, int OPB, int MODE, bool SPLITN, bool BLK>
__global__ __launch_bounds__(CF::NT)
void gemm_f32_mfma_kernel(KParams p) {
    constexpr int BM = CF::BM, BN = CF::BN, BK = CF::BK;
    static_assert(BK % 16 == 0, "BK must be a multiple of 16");
    __shared__ __attribute__((aligned(16))) float lds[Geo<CF, OPA, OPB>::LDS_FLOATS];

    int tiles_m = (int)ceil_div(p.M, BM), tiles_n = (int)ceil_div(p.N, BN);
    int tm, tn;
    tile_of_block(tiles_m, tiles_n, CF::GROUP_M, tm, tn);
    const int64_t bm = (int64_t)tm * BM, bn = (int64_t)tn * BN;

    // Split-K slice: blockIdx.y owns k in [y*k_chunk, min(K, (y+1)*k_chunk))
    // and writes a plain [M, N] partial (the reduction applies the epilogue).
    if (gridDim.y > 1) {
        const int64_t k0 = (int64_t)blockIdx.y * p.k_chunk;
        p.A += OPA == CDX_OP_N ? k0 : k0 * p.lda;
        p.B += OPB == CDX_OP_N ? k0 * p.ldb : k0;
        p.K = p.K - k0 < p.k_chunk ? p.K - k0 : p.k_chunk;
        p.C += (int64_t)blockIdx.y * p.M * p.N;
    }
    if (gridDim.z > 1) {
        p.A += (int64_t)blockIdx.z * p.sa;
        p.B += (int64_t)blockIdx.z * p.sb;
        p.C += (int64_t)blockIdx.z * p.sc;
    }
    if constexpr (MODE == kLoadChecked) {
        // p.nb: op(B)'s own columns, so the ones column stays on the checked path
        if (p.interior && bm + BM <= p.M && bn + BN <= p.nb) {
            gemm_tile<CF, OPA, OPB, kLoadAlignedVec, SPLITN, BLK>(p, bm, bn, lds);
            return;
        }
    }
    gemm_tile<CF, OPA, OPB, MODE, SPLITN, BLK>(p, bm, bn, lds);
}

template <class CF, int OPA, int OPB, int MODE, bool SPLITN, bool BLK>
int launch_cfg(const KParams& kp, int splits, hipStream_t stream) {
    int64_t tiles = ceil_div(kp.M, CF::BM) * ceil_div(kp.N, CF::BN);
    if (tiles > INT32_MAX) return set_error(CDX_ERR_UNSUPPORTED, "gemm: too many tiles");
    if (kp.batch < 1 || kp.batch > 65535) return set_error(CDX_ERR_UNSUPPORTED, "gemm: batch out of range");
    hipLaunchKernelGGL((gemm_f32_mfma_kernel<CF, OPA, OPB, MODE, SPLITN, BLK>),
                       dim3((unsigned)tiles, (unsigned)splits, (unsigned)kp.batch), dim3(CF::NT), 0, stream, kp);
    return hip_error(hipGetLastError(), "gemm_f32_mfma_kernel launch");
}

KParams kparams_of(const GemmArgs& g, int64_t k_chunk) {
    KParams kp{static_cast<const float*>(g.A), static_cast<const float*>(g.B), g.C, g.bias,
               g.M, g.N, g.K, g.lda, g.ldb, g.ldc,
               g.n_split, g.ldc_split, g.bias_mode, g.epilogue, k_chunk,
               g.stride_a, g.stride_b, g.stride_c, g.batch, 0, 0, g.aux, g.ldaux,
               g.ones_col >= 0 ? g.ones_col : g.N, g.ones_col, g.colsum};
    // 16-byte loads need 16-byte aligned bases, leading dimensions and batch
    // strides, decided per operand (a 10-column operand no longer sends the
    // other one down the scalar path: C4's dW2 = dY2^T H, 10 x 256 x 8192,
    // 14 us with both operands scalar)
    kp.vec_a = ((uintptr_t)g.A % 16 == 0) && g.lda % 4 == 0 && g.stride_a % 4 == 0;
    kp.vec_b = ((uintptr_t)g.B % 16 == 0) && g.ldb % 4 == 0 && g.stride_b % 4 == 0;
    return kp;
}

template <class CF, int OPA, int OPB, bool BLK>
int launch_mode(const GemmArgs& g, int splits, int64_t k_chunk, hipStream_t stream) {
    KParams kp = kparams_of(g, k_chunk);
    bool aligned = g.ones_col < 0 && kp.vec_a && kp.vec_b && g.K > 0 && g.M % CF::BM == 0 &&
                   g.N % CF::BN == 0 &&
                   g.K % CF::BK == 0 && k_chunk % CF::BK == 0;
    bool split = g.n_split > 0;
    kp.interior = kp.vec_a && kp.vec_b && g.K % CF::BK == 0 && k_chunk % CF::BK == 0;
    if (aligned) {
        return split ? launch_cfg<CF, OPA, OPB, kLoadAlignedVec, true, BLK>(kp, splits, stream)
                     : launch_cfg<CF, OPA, OPB, kLoadAlignedVec, false, BLK>(kp, splits, stream);
    }
    return split ? launch_cfg<CF, OPA, OPB, kLoadChecked, true, BLK>(kp, splits, stream)
                 : launch_cfg<CF, OPA, OPB, kLoadChecked, false, BLK>(kp, splits, stream);
}

template <class CF>
int launch_ops(const GemmArgs& g0, hipStream_t stream) {
    const int64_t tiles = ceil_div(g0.M, CF::BM) * ceil_div(g0.N, CF::BN);
    return with_splitk(g0, tiles, CF::BK, stream,
                       [&](const GemmArgs& g, int splits, int64_t k_chunk) {
        if (g.opA == CDX_OP_N && g.opB == CDX_OP_N) return launch_mode<CF, CDX_OP_N, CDX_OP_N, false>(g, splits, k_chunk, stream);
        if (g.opA == CDX_OP_N && g.opB == CDX_OP_T) return launch_mode<CF, CDX_OP_N, CDX_OP_T, false>(g, splits, k_chunk, stream);
        if (g.opA == CDX_OP_T && g.opB == CDX_OP_N) return launch_mode<CF, CDX_OP_T, CDX_OP_N, false>(g, splits, k_chunk, stream);
        return launch_mode<CF, CDX_OP_T, CDX_OP_T, false>(g, splits, k_chunk, stream);
    });
}

// Two-level k sum (GemmArgs::blocked_sum), NN products only, no split-K
// (a split already sums in two levels).
template <class CF>
int launch_blocked(const GemmArgs& g, hipStream_t stream) {
    return launch_mode<CF, CDX_OP_N, CDX_OP_N, true>(g, 1, g.K, stream);
}

// Tile configurations (chosen by measurement on MI355X).  All use the two-set
// register pipeline, which measured 4-12 % faster everywhere (4096^3: 138
// against 133 TFLOP/s; 2048^3: 130 against 114).
//  * Huge: 128x128x16, 4 waves of 64x32 (one per SIMD; several workgroups
//    per CU), for problems with at least two 128x128 tiles per CU: 4096^3
//    in 977-983 us against 997-1000 with Large (64x32 wave tiles read A
//    with four 16-byte fragment reads and B with eight 4-byte reads per 16
//    k for 32 MFMAs).  With one tile per CU (2048^3) one wave per SIMD
//    hides less latency: 133.5 against 131.4 us, so Large stays there.
//    (Measured slower: 256x128 tiles of 16 waves of 64x32 at 2048^3, 64x64
//    wave tiles (spills), 8-byte B reads, one register staging set.)
//  * Large: 128x128x16, 8 waves of 32x64 -> 2 waves per SIMD, 32 fp32
//    accumulators per lane.
//  * Medium: 64x64x16, 4 waves of 16x64, for problems whose 128x128 tiles
//    would spread unevenly over the 256 CUs, for the split-K slices of
//    products with M < 128 and for small problems.  Against 4 waves of 32x32
//    on the same tile: 3072^3 447 against 458 us, 4100^3 1358 against 1385,
//    8192 x 256 x 784 (NT) 31.6 against 32.5; 4 waves of 64x16 about the
//    same, 64x128 / 128x64 tiles of 64x32 / 32x64 waves 1.3-1.8x slower.
//    (8 waves of 16x32 measured slower than 4 of 32x32 earlier: 2048^3 141
//    against 157 us.)
//  * SkinnyM: M <= 64 with a long N (the conv GEMM, M = out channels):
//    64x64x16, 4 waves of 16x64 (16-byte B fragment reads), XCD groups of
//    one tile row: 64 x 100352 x 576 in 70-72 us, against 73-74 with 4
//    waves of 32x32, 81 with 8 waves of 16x32 or 32x16, 81 with 64x128
//    tiles of 8 waves of 16x64, 79-84 with 64x32 / 32x64 tiles, 123-125
//    with 64x128 / 64x256 tiles of 32x64 waves, 218 with BK = 32.  A short
//    last round of tiles runs as 64x32 / 64x16 tiles (gemm_f32_skinny_rem_kernel).
//  * NarrowN: N <= 16 (the MLP's 10-class layer): 32x16 tiles, 2 waves, and
//    a deep k-tile (64): such products read A once and are bound by the
//    latency of their k-loop, so each workgroup takes few, large k-steps and
//    twice as many workgroups share the GPU (64x16x16 tiles: 8192 x 10 x
//    256 in 9.5 us, against 13.4 for mostly-empty 64x64 ones).  A 16-row
//    tile for M <= 16 measured no faster than Medium.
//  * W112: N a multiple of 112 but not of 64 (C4's 784-wide backward-data
//    product): 128x112x16, 8 waves of 16x112, so no tile column is ragged
//    (8192 x 784 x 256 NN: 35.5 us, against 40.0 on 64x64 tiles with a
//    16-wide edge column, 57 with 4 waves of 32x112, 52 with 256x112).
//  * SplitTall: split-K slices of products with M >= 128: 128x64x16, 8
//    waves of 32x32 (C4's weight + bias gradient 256 x 785 x 8192: 48.4 us
//    against 54.5 on 64x64 slices; 128x128: 51.5; any BK = 32 slice: 58-79).
using CfgLarge = Cfg<128, 128, 16, 32, 64, 8, 2>;
using CfgHuge = Cfg<128, 128, 16, 64, 32, 8, 2>;
using CfgMedium = Cfg<64, 64, 16, 16, 64, 8, 2>;
using CfgSkinnyM = Cfg<64, 64, 16, 16, 64, 1, 2>;
using CfgNarrowN = Cfg<32, 16, 64, 16, 16, 8, 2>;
using CfgW112 = Cfg<128, 112, 16, 16, 112, 8, 2>;
using CfgSplitTall = Cfg<128, 64, 16, 32, 32, 8, 2>;
using CfgSkinnyHalf = Cfg<64, 32, 16, 16, 32, 1, 2>;
using CfgSkinnyQuarter = Cfg<64, 16, 16, 16, 16, 1, 2>;

// SkinnyM products whose 64-column tiles leave a last round over the 256 CUs
// well short of full: those last tiles run as f = 2 or 4 times as many
// 64 x (64 / f) tiles (same 256 threads, waves of 16 x 64 / f) after the full
// ones, so the busiest CU's share of the last round drops from one tile to
// ceil(rem * f / 256) / f of one.  C5's im2col rounds, 882 and 686 tiles: 4
// -> 3.5 tiles, 42.1 -> 39.3 us, and 3 -> 2.75 tiles, unchanged at 33.3 us;
// the whole batch, 1568 tiles: 7 -> 6.25, 70.8 -> 64.4 us.  Every output
// keeps its k order: the sums are the same bits as on 64 x 64 tiles.  NN,
// whole tiles only.
template <class CFR, bool SPLITN, bool BLK>
__global__ __launch_bounds__(CfgSkinnyM::NT)
void gemm_f32_skinny_rem_kernel(KParams p, int full_tiles) {
    static_assert(CfgSkinnyM::NT == CFR::NT && CFR::BM == CfgSkinnyM::BM, "same block, same rows");
    constexpr int L1 = Geo<CfgSkinnyM, CDX_OP_N, CDX_OP_N>::LDS_FLOATS;
    constexpr int L2 = Geo<CFR, CDX_OP_N, CDX_OP_N>::LDS_FLOATS;
    __shared__ __attribute__((aligned(16))) float lds[L1 > L2 ? L1 : L2];
    const int b = blockIdx.x;
    if (b < full_tiles)
        gemm_tile<CfgSkinnyM, CDX_OP_N, CDX_OP_N, kLoadAlignedVec, SPLITN, BLK>(
            p, 0, (int64_t)b * CfgSkinnyM::BN, lds);
    else
        gemm_tile<CFR, CDX_OP_N, CDX_OP_N, kLoadAlignedVec, SPLITN, BLK>(
            p, 0, (int64_t)full_tiles * CfgSkinnyM::BN + (int64_t)(b - full_tiles) * CFR::BN, lds);
}

// Full tile count and split factor f of the last round when the split launch
// applies: an unsplit NN product of exactly one 64-row tile, whole 64-column
// tiles, whole k-tiles, 16-byte loadable operands, and a last round of rem
// tiles that f splits to less than one tile per CU: f = 4 for rem <= 64
// (1/4) and 128 < rem <= 192 (3/4), f = 2 for 64 < rem <= 128 (1/2).
bool skinny_rem_plan(const GemmArgs& g, int64_t& full, int& f) {
    const KParams kp = kparams_of(g, g.K);
    if (g.M != CfgSkinnyM::BM || g.N % CfgSkinnyM::BN != 0 || g.K <= 0 ||
        g.K % CfgSkinnyM::BK != 0 || g.batch != 1 || g.ones_col >= 0 || !kp.vec_a ||
        !kp.vec_b || g.opA != CDX_OP_N || g.opB != CDX_OP_N)
        return false;
    const int64_t tiles = g.N / CfgSkinnyM::BN, rem = tiles % 256;
    if (rem == 0 || rem > 192 || tiles + 3 * rem > INT32_MAX) return false;
    full = tiles - rem;
    f = rem > 64 && rem <= 128 ? 2 : 4;
    return true;
}

template <bool BLK>
int launch_skinny_rem(const GemmArgs& g, int64_t full, int f, hipStream_t stream) {
    const KParams kp = kparams_of(g, g.K);
    const int64_t rem = g.N / CfgSkinnyM::BN - full;
    const dim3 grid((unsigned)(full + f * rem)), block(CfgSkinnyM::NT);
    const bool sn = g.n_split > 0;
    if (f == 2 && sn)
        hipLaunchKernelGGL((gemm_f32_skinny_rem_kernel<CfgSkinnyHalf, true, BLK>), grid, block, 0, stream, kp, (int)full);
    else if (f == 2)
        hipLaunchKernelGGL((gemm_f32_skinny_rem_kernel<CfgSkinnyHalf, false, BLK>), grid, block, 0, stream, kp, (int)full);
    else if (sn)
        hipLaunchKernelGGL((gemm_f32_skinny_rem_kernel<CfgSkinnyQuarter, true, BLK>), grid, block, 0, stream, kp, (int)full);
    else
        hipLaunchKernelGGL((gemm_f32_skinny_rem_kernel<CfgSkinnyQuarter, false, BLK>), grid, block, 0, stream, kp, (int)full);
    return hip_error(hipGetLastError(), "gemm_f32_skinny_rem_kernel launch");
}

// Configuration choice, shared by the launcher and the workspace query.
enum class F32Cfg { NarrowN, SkinnyM, Huge, Large, Medium, W112, SplitTall };

// Large tiles are ~8 % faster per tile, but a CU's time is set by its largest
// share of tiles: Large is taken when its busiest-CU share (rounded up to
// whole tiles per CU over the 256 CUs) is within 5 % of Medium's.  (2048^3,
// 256 tiles: 130 against 141 us; 3072^3, 576 tiles: 561 against 459.)
bool large_balanced(int64_t M, int64_t N) {
    const int64_t tl = ceil_div(M, 128) * ceil_div(N, 128);
    const int64_t tm = ceil_div(M, 64) * ceil_div(N, 64);
    const int64_t cus = 256;
    if (tl < cus) return false;
    // ceil(tl/cus)/(tl/cus) <= 1.05 * ceil(tm/cus)/(tm/cus)
    return ceil_div(tl, cus) * tm * 100 <= 105 * ceil_div(tm, cus) * tl;
}

F32Cfg choose_f32(const GemmArgs& g, bool& blocked) {
    const bool split = g.batch == 1 && splitk_applies(ceil_div(g.M, 64) * ceil_div(g.N, 64), g.K);
    blocked = g.blocked_sum && !split && g.opA == CDX_OP_N && g.opB == CDX_OP_N;
    if (g.N <= 16) return F32Cfg::NarrowN;
    if (split && !blocked) return g.M >= 128 ? F32Cfg::SplitTall : F32Cfg::Medium;
    if (!blocked && !split && g.N % 112 == 0 && g.N % 64 != 0 &&
        ceil_div(g.M, 128) * (g.N / 112) >= 256)
        return F32Cfg::W112;
    if (g.M <= 64 && g.N >= 4096) return F32Cfg::SkinnyM;
    if (large_balanced(g.M, g.N))
        return ceil_div(g.M, 128) * ceil_div(g.N, 128) >= 512 ? F32Cfg::Huge : F32Cfg::Large;
    return F32Cfg::Medium;
}

template <class CF>
size_t ws_of(const GemmArgs& g) {
    return splitk_bytes(g, ceil_div(g.M, CF::BM) * ceil_div(g.N, CF::BN), CF::BK);
}

}  // namespace

bool f32_takes_w112(const GemmArgs& g) {
    bool blocked;
    return choose_f32(g, blocked) == F32Cfg::W112;
}

size_t gemm_f32_workspace(const GemmArgs& g) {
    if (const int nk = narrow_kind(g)) return nk == 3 ? skinny_m_workspace(g) : 0;
    bool blocked;
    const F32Cfg c = choose_f32(g, blocked);
    if (blocked) return 0;
    switch (c) {
        case F32Cfg::NarrowN: return ws_of<CfgNarrowN>(g);
        case F32Cfg::SkinnyM: return ws_of<CfgSkinnyM>(g);
        case F32Cfg::Large: return ws_of<CfgLarge>(g);
        case F32Cfg::Huge: return ws_of<CfgHuge>(g);
        case F32Cfg::W112: return ws_of<CfgW112>(g);
        case F32Cfg::SplitTall: return ws_of<CfgSplitTall>(g);
        default: return ws_of<CfgMedium>(g);
    }
}

int launch_gemm_f32(const GemmArgs& g, hipStream_t stream) {
    if (narrow_kind(g)) return launch_gemm_narrow(g, stream);
    bool blocked;
    const F32Cfg c = choose_f32(g, blocked);
    int64_t full = 0;
    int f = 1;
    if (c == F32Cfg::SkinnyM && skinny_rem_plan(g, full, f))
        return blocked ? launch_skinny_rem<true>(g, full, f, stream)
                       : launch_skinny_rem<false>(g, full, f, stream);
    if (blocked) {
        switch (c) {
            case F32Cfg::NarrowN: return launch_blocked<CfgNarrowN>(g, stream);
            case F32Cfg::SkinnyM: return launch_blocked<CfgSkinnyM>(g, stream);
            case F32Cfg::Large: return launch_blocked<CfgLarge>(g, stream);
            case F32Cfg::Huge: return launch_blocked<CfgHuge>(g, stream);
            default: return launch_blocked<CfgMedium>(g, stream);
        }
    }
    switch (c) {
        case F32Cfg::NarrowN: return launch_ops<CfgNarrowN>(g, stream);
        case F32Cfg::SkinnyM: return launch_ops<CfgSkinnyM>(g, stream);
        case F32Cfg::Large: return launch_ops<CfgLarge>(g, stream);
        case F32Cfg::Huge: return launch_ops<CfgHuge>(g, stream);
        case F32Cfg::W112: return launch_ops<CfgW112>(g, stream);
        case F32Cfg::SplitTall: return launch_ops<CfgSplitTall>(g, stream);
        default: return launch_ops<CfgMedium>(g, stream);
    }
}

}  // namespace cdx
