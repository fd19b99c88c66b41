// GEMMs with a tiny inner or output dimension, which the tiled MFMA kernels
// run at a few percent of their rate because a k-loop of a handful of steps
// is all latency (the MLP's 10-wide layer: C4's 8192 x 10 x 256 forward and
// 8192 x 256 x 10 hidden-layer gradient).  Both are bound by the bytes they
// move, so each is organised around one pass over memory:
//
//  * tiny K (K <= 16): each thread forms 4 consecutive outputs of a few rows
//    as fp32 FMA chains over k ascending -- the reference SGEMM's own
//    arithmetic (sgemm_general_kernel, src/kernels/matmul_kernel.cu:632-647)
//    -- reading op(A)'s rows and op(B)'s 4 columns (cached; tiny) and
//    writing C through the epilogue.  Traffic: C written once (plus aux read
//    once for the activation-backward epilogues).
//  * narrow N (N <= 16): a workgroup owns 16 rows; its four waves split K in
//    four contiguous quarters, each running v_mfma_f32_16x16x4_f32 on
//    operands read straight from global memory (no LDS staging: op(A)'s rows
//    are read once, op(B) is a few KB and stays in cache), with the library's
//    k-permutation (lane group g feeds MFMA q with k = 4g + q, so a
//    k-contiguous operand is one 16-byte load per 16 k).  The four partial
//    16 x 16 tiles are summed in LDS in wave order (deterministic) and
//    written through the epilogue.  Traffic: op(A) read once, C written once.
//  * skinny M (M <= 16, op(B) = B, long K: the MLP's 10-wide weight
//    gradient dW2 = dY2^T H, 10 x 256 x 8192, its bias gradient as the ones
//    column): K in slices of >= 128 rows; a workgroup owns 64 columns of one
//    slice, each thread 4 columns (one 16-byte op(B) load per row) of 8 rows
//    per step, with 16 x 4 fp32 FMA chains over its rows; the 4 lane groups
//    of a wave are summed by shuffles and the 4 waves in LDS, in a fixed
//    order, into a [slices][M][N] partial.  A second kernel sums the slices
//    (4 waves per output row and 64 columns, slices dealt round-robin, the
//    waves combined in order) through the epilogue.  Traffic: op(B) read
//    once, the partials (<= 16 MB) written and read once.
//
// All compute fp32 products in every precision mode (exact products: inside
// the TF32-mode error bar, as for the other FP32-routed shapes).  Plain
// row-major output map only, no batch, no ones column (skinny M: with the
// ones column); everything else goes to the tiled kernels.
#include <type_traits>

#include "cdx_internal.hpp"

namespace cdx {
namespace {

struct NarrowArgs {
    const float* A; const float* B; float* C; const float* bias;
    int64_t M, N, K, lda, ldb, ldc;
    int bias_mode, epilogue;
    const float* aux; int64_t ldaux;
    int opA, opB;
    int vec_a, vec_b;   // 16-byte loads allowed (aligned base and leading dim)
};

// (narrow-N kernel: transposition chosen at run time)
__device__ __forceinline__ float opa(const NarrowArgs& p, int64_t m, int64_t k) {
    return p.opA == CDX_OP_N ? p.A[m * p.lda + k] : p.A[k * p.lda + m];
}
__device__ __forceinline__ float opb(const NarrowArgs& p, int64_t k, int64_t n) {
    return p.opB == CDX_OP_N ? p.B[k * p.ldb + n] : p.B[n * p.ldb + k];
}

// One thread: row m, columns n0 .. n0+3.  OPA / OPB / ACT fixed at compile
// time (straight-line code); VEC: 16-byte accesses to op(B) (OPB = N), aux
// and C where a thread's 4 columns are whole.
// rows per thread: op(B)'s 4 columns stay in registers across them (C4's
// 8192 x 256 x 10 hidden gradient: 1, 2, 4 and 8 rows measured 6.7, 7.3,
// 6.4 and 9.8 us -- op(B) re-reads through L1 against fewer threads in
// flight; a plain copy of the same 8.4 MB takes 3.4 us)
constexpr int TK_ROWS = 4;

// WAVE_ROWS: ceil(N / 4) is a multiple of 64, so the 64 threads of a wave
// share their rows m0 .. m0 + 3; the wave then loads those rows' op(A)
// elements once (lane 16 i + k holds row m0 + i, column k) and every lane
// takes them with readlane, instead of 16 uniform loads per row per lane
// (C4's 8192 x 256 x 10 masked dH: 7.7 -> 4.x us).
template <int OPA, int OPB, int ACT, bool VEC, bool WAVE_ROWS>
__global__ __launch_bounds__(256)
void gemm_tinyk_kernel(NarrowArgs p) {
    const int64_t ngroups = ceil_div(p.N, 4);
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= ceil_div(p.M, TK_ROWS) * ngroups) return;
    const int64_t m0 = (t / ngroups) * TK_ROWS, n0 = (t % ngroups) * 4;
    constexpr bool BWD = ACT >= CDX_EPI_BWD_RELU;
    static_assert(TK_ROWS * 16 == 64, "one op(A) element per lane");
    int aw = 0;
    if constexpr (WAVE_ROWS) {
        const int lane = threadIdx.x & 63;
        int64_t ma = m0 + (lane >> 4);
        if (ma >= p.M) ma = m0;
        const int64_t ka = (lane & 15) < p.K ? (lane & 15) : 0;
        aw = __float_as_int(OPA == CDX_OP_N ? p.A[ma * p.lda + ka] : p.A[ka * p.lda + ma]);
    }
    // WH: this thread's 4 columns are whole (16-byte accesses); one branch
    // here, straight-line code below
    auto run = [&](auto wh_c) {
        constexpr bool WH = decltype(wh_c)::value;
        // op(B)'s 4 columns for all 16 k, loaded once for TK_ROWS rows (k >= K
        // clamped to k = 0, always in range, so the loads issue together;
        // the chains stop at K)
        float bv[16][4];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int64_t kk = k < p.K ? k : 0;
            if constexpr (OPB == CDX_OP_N && WH) {
                const float4 v = *reinterpret_cast<const float4*>(p.B + kk * p.ldb + n0);
                bv[k][0] = v.x; bv[k][1] = v.y; bv[k][2] = v.z; bv[k][3] = v.w;
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int64_t n = n0 + c < p.N ? n0 + c : n0;
                    bv[k][c] = OPB == CDX_OP_N ? p.B[kk * p.ldb + n] : p.B[n * p.ldb + kk];
                }
            }
        }
        float bcol[4] = {0.f, 0.f, 0.f, 0.f};
        if (!BWD && p.bias_mode == CDX_BIAS_COL) {
#pragma unroll
            for (int c = 0; c < 4; ++c) bcol[c] = p.bias[n0 + c < p.N ? n0 + c : n0];
        }
#pragma unroll
        for (int i = 0; i < TK_ROWS; ++i) {
            const int64_t m = m0 + i;
            if (m >= p.M) break;
            // the activation input first: its load overlaps the operand loads
            float x[4] = {0.f, 0.f, 0.f, 0.f};
            if constexpr (BWD) {
                const float* ax = p.aux + m * p.ldaux + n0;
                if constexpr (WH) {
                    const float4 v = *reinterpret_cast<const float4*>(ax);
                    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) x[c] = ax[n0 + c < p.N ? c : 0];
                }
            }
            float av[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                if constexpr (WAVE_ROWS) {
                    av[k] = __int_as_float(__builtin_amdgcn_readlane(aw, 16 * i + k));
                } else {
                    const int64_t kk = k < p.K ? k : 0;
                    av[k] = OPA == CDX_OP_N ? p.A[m * p.lda + kk] : p.A[kk * p.lda + m];
                }
            }
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                if (k >= p.K) break;   // K is uniform: a scalar branch
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[c] = fmaf(av[k], bv[k][c], acc[c]);
            }
            float r[4];
            if constexpr (BWD) {
#pragma unroll
                for (int c = 0; c < 4; ++c) r[c] = bwd_fixed<ACT>(acc[c], x[c]);
            } else {
                const float brow = p.bias_mode == CDX_BIAS_ROW ? p.bias[m] : 0.0f;
#pragma unroll
                for (int c = 0; c < 4; ++c) r[c] = act_fixed<ACT>(acc[c] + bcol[c] + brow);
            }
            float* cr = p.C + m * p.ldc + n0;
            if constexpr (WH) {
                *reinterpret_cast<float4*>(cr) = make_float4(r[0], r[1], r[2], r[3]);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (n0 + c < p.N) cr[c] = r[c];
            }
        }
    };
    if (VEC && n0 + 3 < p.N) run(std::true_type{});
    else run(std::false_type{});
}

template <int OPA, int OPB, int ACT>
int launch_tinyk3(const NarrowArgs& p, bool vec, dim3 grid, hipStream_t stream) {
    const bool wave_rows = ceil_div(p.N, 4) % 64 == 0;
    if (vec && wave_rows)
        hipLaunchKernelGGL((gemm_tinyk_kernel<OPA, OPB, ACT, true, true>), grid, dim3(256), 0, stream, p);
    else if (vec)
        hipLaunchKernelGGL((gemm_tinyk_kernel<OPA, OPB, ACT, true, false>), grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((gemm_tinyk_kernel<OPA, OPB, ACT, false, false>), grid, dim3(256), 0, stream, p);
    return hip_error(hipGetLastError(), "gemm_tinyk_kernel launch");
}

template <int OPA, int OPB>
int launch_tinyk2(const NarrowArgs& p, bool vec, dim3 grid, hipStream_t stream) {
    switch (p.epilogue) {
        case CDX_EPI_RELU: return launch_tinyk3<OPA, OPB, CDX_EPI_RELU>(p, vec, grid, stream);
        case CDX_EPI_GELU: return launch_tinyk3<OPA, OPB, CDX_EPI_GELU>(p, vec, grid, stream);
        case CDX_EPI_SILU: return launch_tinyk3<OPA, OPB, CDX_EPI_SILU>(p, vec, grid, stream);
        case CDX_EPI_SIGMOID: return launch_tinyk3<OPA, OPB, CDX_EPI_SIGMOID>(p, vec, grid, stream);
        case CDX_EPI_BWD_RELU: return launch_tinyk3<OPA, OPB, CDX_EPI_BWD_RELU>(p, vec, grid, stream);
        case CDX_EPI_BWD_GELU: return launch_tinyk3<OPA, OPB, CDX_EPI_BWD_GELU>(p, vec, grid, stream);
        case CDX_EPI_BWD_SILU: return launch_tinyk3<OPA, OPB, CDX_EPI_BWD_SILU>(p, vec, grid, stream);
        case CDX_EPI_BWD_SIGMOID: return launch_tinyk3<OPA, OPB, CDX_EPI_BWD_SIGMOID>(p, vec, grid, stream);
        default: return launch_tinyk3<OPA, OPB, CDX_EPI_NONE>(p, vec, grid, stream);
    }
}

// Four waves per workgroup, one 16-row tile, K in four quarters.
__global__ __launch_bounds__(256)
void gemm_narrow_n_kernel(NarrowArgs p, int64_t kq) {
    __shared__ float red[4][16][17];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lq = lane >> 4;
    const int64_t m0 = (int64_t)blockIdx.x * 16;
    const int64_t m = m0 + l16;
    const bool m_ok = m < p.M, n_ok = l16 < p.N;
    const int64_t kb = wave * kq, ke = kb + kq < p.K ? kb + kq : p.K;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    // A row m (this lane's MFMA row) and B column n = l16
    const bool va = p.vec_a && p.opA == CDX_OP_N && m_ok;
    const bool vb = p.vec_b && p.opB == CDX_OP_T && n_ok;
    for (int64_t k0 = kb; k0 < ke; k0 += 16) {
        const int64_t k = k0 + 4 * lq;   // this lane's 4 k
        float a[4], b[4];
        if (va && k + 3 < ke) {
            const float4 v = *reinterpret_cast<const float4*>(p.A + m * p.lda + k);
            a[0] = v.x; a[1] = v.y; a[2] = v.z; a[3] = v.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) a[q] = (m_ok && k + q < ke) ? opa(p, m, k + q) : 0.0f;
        }
        if (vb && k + 3 < ke) {
            const float4 v = *reinterpret_cast<const float4*>(p.B + (int64_t)l16 * p.ldb + k);
            b[0] = v.x; b[1] = v.y; b[2] = v.z; b[3] = v.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) b[q] = (n_ok && k + q < ke) ? opb(p, k + q, l16) : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], b[q], acc, 0, 0, 0);
    }
    // D layout: register r of lane l is row 4*(l/16) + r, column l % 16
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * lq + r][l16] = acc[r];
    __syncthreads();
    const int row = tid >> 4, col = tid & 15;
    if (m0 + row < p.M && col < p.N) {
        const float v = ((red[0][row][col] + red[1][row][col]) + red[2][row][col]) + red[3][row][col];
        const EpiArgs e{p.C, p.ldc, p.M, p.N, 0, 0, p.bias, p.bias_mode, p.epilogue, p.aux, p.ldaux};
        store_one(e, m0 + row, col, v);
    }
}

// ---- skinny M ----
constexpr int SM_COLS = 64;          // columns per workgroup
constexpr int SM_KC_MIN = 128;       // k rows per slice, at least (16 row groups x 8)
constexpr int64_t SM_SLICES_MAX = 256;
constexpr int64_t SM_PART_MAX = int64_t(4) << 20;   // partial floats, at most (16 MB)

struct SkinnyPlan { int64_t kc; int slices; };

// g.N counts the ones column when there is one.
SkinnyPlan skinny_plan(const GemmArgs& g) {
    int64_t smax = SM_PART_MAX / (g.M * g.N);
    if (smax > SM_SLICES_MAX) smax = SM_SLICES_MAX;
    if (smax < 1) smax = 1;
    const int64_t kc = ceil_div(ceil_div(g.K, smax), SM_KC_MIN) * SM_KC_MIN;
    return {kc, (int)ceil_div(g.K, kc)};
}

// Grid (column blocks, slices).  Thread: column quad c4 = tid % 16, row
// group rg = tid / 16 (a 16-lane DPP row); it takes rows kb + rg + 16 u +
// 128 j of its slice (k ascending) and op(B)'s columns n0 .. n0+3 (nb real
// columns; column ones_col, if any, is all ones).  op(A) costs one load per
// row: lane c4 of the row group holds element (min(c4, M-1), k) and each
// element reaches the whole row group by a DPP row broadcast (16 uniform
// loads per row per lane before: 12.7 us for C4's dW2 partials).  Rows past
// the slice contribute exact zeros (both factors zeroed, so no Inf * 0).
constexpr int SM_U = 8;   // rows per thread in flight

// acc[m][c] += op(A)(m, k) * b[c] for m = M .. MT-1, op(A)(m, k) taken from
// lane m of this lane's 16-lane row (DPP row_newbcast:m, control 0x150 + m).
template <int M, int MT>
__device__ __forceinline__ void skinny_fma_rows(float (&acc)[MT][4], int a_bits, const float (&b)[4]) {
    if constexpr (M < MT) {
        const float am = __int_as_float(__builtin_amdgcn_update_dpp(0, a_bits, 0x150 + M, 0xf, 0xf, false));
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[M][c] = fmaf(am, b[c], acc[M][c]);
        skinny_fma_rows<M + 1, MT>(acc, a_bits, b);
    }
}
// MT: rows computed, M rounded up to 4, 8, 12 or 16 (rows past M are
// computed from row M-1 and never stored).
template <int OPA, int MT>
__global__ __launch_bounds__(256)
void gemm_skinny_m_partial_kernel(NarrowArgs p, int64_t nb, int64_t ones_col, int64_t kc,
                                  float* __restrict__ P) {
    __shared__ float red[4][MT][SM_COLS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c4 = tid & 15, rg = tid >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * SM_COLS + 4 * c4;
    const int64_t kb = (int64_t)blockIdx.y * kc;
    const int64_t ke = kb + kc < p.K ? kb + kc : p.K;
    const int64_t ma = c4 < p.M ? c4 : p.M - 1;
    const bool whole = p.vec_b && n0 + 3 < nb;
    float acc[MT][4];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;
    for (int64_t k0 = kb + rg; k0 < ke; k0 += 16 * SM_U) {
        float a[SM_U], b[SM_U][4];
#pragma unroll
        for (int u = 0; u < SM_U; ++u) {
            const int64_t k = k0 + 16 * u;
            const bool ok = k < ke;
            const int64_t kk = ok ? k : kb;
            if (whole) {
                const float4 v = *reinterpret_cast<const float4*>(p.B + kk * p.ldb + n0);
                b[u][0] = v.x; b[u][1] = v.y; b[u][2] = v.z; b[u][3] = v.w;
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int64_t n = n0 + c;
                    b[u][c] = n < nb ? p.B[kk * p.ldb + n] : (n == ones_col ? 1.0f : 0.0f);
                }
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) b[u][c] = ok ? b[u][c] : 0.0f;
            const float av = OPA == CDX_OP_N ? p.A[ma * p.lda + kk] : p.A[kk * p.lda + ma];
            a[u] = ok ? av : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < SM_U; ++u) skinny_fma_rows<0, MT>(acc, __float_as_int(a[u]), b[u]);
    }
    // the wave's 4 row groups (lanes 16 apart hold the same columns)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float v = acc[m][c];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            acc[m][c] = v;
        }
    if (lane < 16) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (m < p.M) {
#pragma unroll
                for (int c = 0; c < 4; ++c) red[wave][m][4 * lane + c] = acc[m][c];
            }
    }
    __syncthreads();
    float* ps = P + (int64_t)blockIdx.y * p.M * p.N;
    for (int i = tid; i < p.M * SM_COLS; i += 256) {
        const int m = i / SM_COLS, col = i % SM_COLS;
        const int64_t n = (int64_t)blockIdx.x * SM_COLS + col;
        if (n < p.N)
            ps[m * p.N + n] = ((red[0][m][col] + red[1][m][col]) + red[2][m][col]) + red[3][m][col];
    }
}

// Grid (column blocks, M): wave w sums slices w, w + 4, ... of 64 columns of
// one row (16 loads in flight), the 4 waves are combined in order and the
// result goes through the epilogue.
__global__ __launch_bounds__(256)
void gemm_skinny_m_reduce_kernel(const float* __restrict__ P, int slices, EpiArgs e) {
    __shared__ float red[4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t m = blockIdx.y, n = (int64_t)blockIdx.x * 64 + lane;
    const int64_t MN = e.M * e.N;
    const float* q = P + m * e.N + (n < e.N ? n : 0);
    float v = 0.0f;
    int s = wave;
    for (; s + 60 < slices; s += 64) {
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) t[u] = q[(int64_t)(s + 4 * u) * MN];
#pragma unroll
        for (int u = 0; u < 16; ++u) v += t[u];
    }
    for (; s + 12 < slices; s += 16) {
        float t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) t[u] = q[(int64_t)(s + 4 * u) * MN];
#pragma unroll
        for (int u = 0; u < 4; ++u) v += t[u];
    }
    for (; s < slices; s += 4) v += q[(int64_t)s * MN];
    red[wave][lane] = v;
    __syncthreads();
    if (wave == 0 && n < e.N)
        store_one(e, m, n, ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane]);
}

NarrowArgs args_of(const GemmArgs& g) {
    NarrowArgs p{static_cast<const float*>(g.A), static_cast<const float*>(g.B), g.C, g.bias,
                 g.M, g.N, g.K, g.lda, g.ldb, g.ldc, g.bias_mode, g.epilogue, g.aux, g.ldaux,
                 g.opA, g.opB, 0, 0};
    p.vec_a = (uintptr_t)g.A % 16 == 0 && g.lda % 4 == 0;
    p.vec_b = (uintptr_t)g.B % 16 == 0 && g.ldb % 4 == 0;
    return p;
}

}  // namespace

int narrow_kind(const GemmArgs& g) {
    if (g.batch != 1 || g.n_split > 0 || g.M <= 0 || g.N <= 0) return 0;
    if (g.M <= 16 && g.opB == CDX_OP_N && g.K >= 1024 && g.N <= 4097) return 3;   // skinny M
    if (g.colsum || g.ones_col >= 0) return 0;
    if (g.K >= 1 && g.K <= 16) return 1;                    // tiny K
    if (g.N <= 16 && g.K >= 64 && g.M >= 64) return 2;      // narrow N
    return 0;
}

namespace {

// the partial kernel for M rounded up to mt rows
template <int OPA>
void skinny_partial_go(int mt, dim3 grid, hipStream_t stream, const NarrowArgs& p, int64_t nb,
                       int64_t ones_col, int64_t kc, float* part) {
    if (mt == 4)
        hipLaunchKernelGGL((gemm_skinny_m_partial_kernel<OPA, 4>), grid, dim3(256), 0, stream, p, nb, ones_col, kc, part);
    else if (mt == 8)
        hipLaunchKernelGGL((gemm_skinny_m_partial_kernel<OPA, 8>), grid, dim3(256), 0, stream, p, nb, ones_col, kc, part);
    else if (mt == 12)
        hipLaunchKernelGGL((gemm_skinny_m_partial_kernel<OPA, 12>), grid, dim3(256), 0, stream, p, nb, ones_col, kc, part);
    else
        hipLaunchKernelGGL((gemm_skinny_m_partial_kernel<OPA, 16>), grid, dim3(256), 0, stream, p, nb, ones_col, kc, part);
}

}  // namespace

size_t skinny_m_workspace(const GemmArgs& g) {
    return (size_t)skinny_plan(g).slices * (size_t)g.M * (size_t)g.N * sizeof(float);
}

static int launch_skinny_m(const GemmArgs& g, const NarrowArgs& p, hipStream_t stream) {
    const SkinnyPlan sp = skinny_plan(g);
    const int64_t nb = g.ones_col >= 0 ? g.ones_col : g.N;
    const dim3 grid1((unsigned)ceil_div(g.N, SM_COLS), (unsigned)sp.slices);
    const dim3 grid2((unsigned)ceil_div(g.N, 64), (unsigned)g.M);
    const size_t bytes = skinny_m_workspace(g);
    float* part = static_cast<float*>(g.ws);
    int st = CDX_OK;
    if (part) {
        if (g.ws_bytes < bytes) return set_error(CDX_ERR_WORKSPACE, "gemm: workspace too small");
    } else {
        st = stream_alloc(reinterpret_cast<void**>(&part), bytes, stream, "gemm skinny-M scratch");
        if (st) return st;
    }
    const int mt = g.M <= 4 ? 4 : g.M <= 8 ? 8 : g.M <= 12 ? 12 : 16;
    if (g.opA == CDX_OP_N) skinny_partial_go<CDX_OP_N>(mt, grid1, stream, p, nb, g.ones_col, sp.kc, part);
    else skinny_partial_go<CDX_OP_T>(mt, grid1, stream, p, nb, g.ones_col, sp.kc, part);
    st = hip_error(hipGetLastError(), "gemm_skinny_m_partial_kernel launch");
    if (!st) {
        const EpiArgs e{g.C, g.ldc, g.M, g.N, g.n_split, g.ldc_split, g.bias, g.bias_mode,
                        g.epilogue, g.aux, g.ldaux, g.colsum, g.ones_col};
        hipLaunchKernelGGL(gemm_skinny_m_reduce_kernel, grid2, dim3(256), 0, stream, part,
                           sp.slices, e);
        st = hip_error(hipGetLastError(), "gemm_skinny_m_reduce_kernel launch");
    }
    if (!g.ws) {
        const int st2 = stream_free(part, stream, "gemm skinny-M scratch");
        if (!st) st = st2;
    }
    return st;
}

int launch_gemm_narrow(const GemmArgs& g, hipStream_t stream) {
    const NarrowArgs p = args_of(g);
    if (narrow_kind(g) == 3) return launch_skinny_m(g, p, stream);
    if (narrow_kind(g) == 1) {
        const int64_t threads = ceil_div(g.M, TK_ROWS) * ceil_div(g.N, 4);
        const int64_t blocks = ceil_div(threads, 256);
        if (blocks > INT32_MAX) return set_error(CDX_ERR_UNSUPPORTED, "gemm: too many rows");
        // 16-byte accesses: C (and aux, and op(B) when not transposed)
        // 16-byte aligned with 4-element leading dimensions
        const bool bwd = g.epilogue >= CDX_EPI_BWD_RELU && g.epilogue <= CDX_EPI_BWD_SIGMOID;
        const bool vec = (uintptr_t)g.C % 16 == 0 && g.ldc % 4 == 0 &&
                         (g.opB == CDX_OP_T || (p.vec_b != 0)) &&
                         (!bwd || ((uintptr_t)g.aux % 16 == 0 && g.ldaux % 4 == 0));
        const dim3 grid((unsigned)blocks);
        if (g.opA == CDX_OP_N && g.opB == CDX_OP_N) return launch_tinyk2<CDX_OP_N, CDX_OP_N>(p, vec, grid, stream);
        if (g.opA == CDX_OP_N && g.opB == CDX_OP_T) return launch_tinyk2<CDX_OP_N, CDX_OP_T>(p, vec, grid, stream);
        if (g.opA == CDX_OP_T && g.opB == CDX_OP_N) return launch_tinyk2<CDX_OP_T, CDX_OP_N>(p, vec, grid, stream);
        return launch_tinyk2<CDX_OP_T, CDX_OP_T>(p, vec, grid, stream);
    }
    const int64_t blocks = ceil_div(g.M, 16);
    if (blocks > INT32_MAX) return set_error(CDX_ERR_UNSUPPORTED, "gemm: too many rows");
    const int64_t kq = ceil_div(ceil_div(g.K, 4), 16) * 16;   // whole 16-k steps per wave
    hipLaunchKernelGGL(gemm_narrow_n_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p, kq);
    return hip_error(hipGetLastError(), "gemm_narrow_n_kernel launch");
}

}  // namespace cdx
