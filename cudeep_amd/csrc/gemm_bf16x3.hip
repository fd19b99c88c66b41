// "TF32-mode" (bf16x3 / bf16x4 split-precision) and 16-bit-operand GEMMs:
// configuration choice and the library entry points.  The kernels and their
// launchers are in gemm_split.hpp; their instantiations in gemm_split_*.hip.
//
// Replaces the reference's TF32 tensor-core dispatcher
// (launch_matmul_kernel<float>, src/kernels/matmul_kernel.cu:1785-1841) and
// its FP16 launcher (launch_matmul_kernel_fp16, :1926-1943).
#include "gemm_split.hpp"

namespace cdx {
namespace {

using namespace split;

// Configuration choice, shared by the launcher and the workspace query.
enum class BfCfg { SkinnyM, Huge, KAlt, Large, Small };

BfCfg choose_bf(const GemmArgs& g, int terms) {
    if (g.M <= 64 && g.N >= 4096) return BfCfg::SkinnyM;
    // Huge holds 128 accumulators per lane: only its unchecked three-term
    // form fits in 256 registers without spilling.
    if (terms == 3 && ceil_div(g.M, 256) * ceil_div(g.N, 256) >= 256 && aligned_for<CfgHuge>(g))
        return BfCfg::Huge;
    const int64_t tiles128 = ceil_div(g.M, 128) * ceil_div(g.N, 128);
    if (tiles128 >= 256 && kalt_fits(g)) return BfCfg::KAlt;
    if (tiles128 >= 256) return BfCfg::Large;
    return BfCfg::Small;
}

template <class CF>
size_t ws_of(const GemmArgs& g) {
    return splitk_bytes(g, ceil_div(g.M, CF::BM) * ceil_div(g.N, CF::BN), CF::BK, kSplitMinK);
}

template <int TERMS>
int dispatch(const GemmArgs& g, hipStream_t stream) {
    switch (choose_bf(g, TERMS)) {
        case BfCfg::SkinnyM: return launch_ops<CfgSkinnyM, TERMS>(g, stream);
        case BfCfg::Huge:
            if constexpr (TERMS == 3) {
                if (pingpong_fits(g)) return launch_pingpong_ops<kInF32>(g, stream);
                return launch_ops<CfgHuge, TERMS>(g, stream);
            }
            return set_error(CDX_ERR_UNSUPPORTED, "gemm: no four-term Huge configuration");
        case BfCfg::KAlt: return launch_kalt_ops<TERMS>(g, stream);
        case BfCfg::Large: return launch_ops<CfgLarge, TERMS>(g, stream);
        default: return launch_ops<CfgSmall, TERMS>(g, stream);
    }
}

// Weight-gradient-shaped products -- A transposed, too few output tiles to
// fill the GPU, long K (split-K) -- run on the FP32 kernel in the TF32
// modes: there both bf16x3 operands would be transposed in registers on the
// way into LDS over short k slices, and FP32 measured faster (256 x 784 x
// 8192: 52 us against 66 us at bf16x3's best split) with exact products,
// which is inside the TF32-mode error bar.
bool tn_split_to_f32(const GemmArgs& g, int terms) {
    return g.opA == CDX_OP_T && g.batch == 1 && choose_bf(g, terms) == BfCfg::Small &&
           splitk_applies(ceil_div(g.M, CfgSmall::BM) * ceil_div(g.N, CfgSmall::BN), g.K);
}

// The 16-bit kernels' unchecked loads move 16 bytes (8 elements) per lane,
// so their rows and batch strides must start at 8-element multiples (else
// the checked in-step forms run, 4 elements per load).
bool rows_of_8(const GemmArgs& g) {
    return g.lda % 8 == 0 && g.ldb % 8 == 0 && g.stride_a % 8 == 0 && g.stride_b % 8 == 0;
}

template <int IN>
int dispatch16(const GemmArgs& g, hipStream_t stream) {
    if (ceil_div(g.M, 256) * ceil_div(g.N, 256) >= 256 && aligned_for<Cfg16Huge>(g) &&
        rows_of_8(g)) {
        if (pingpong_fits(g)) return launch_pingpong_ops<IN>(g, stream);
        return launch_ops<Cfg16Huge, 1, IN>(g, stream);
    }
    if (ceil_div(g.M, 128) * ceil_div(g.N, 128) >= 256) return launch_ops<Cfg16Large, 1, IN>(g, stream);
    return launch_ops<Cfg16Small, 1, IN>(g, stream);
}

}  // namespace

// Products whose FP32 form runs on 128 x 112 tiles (C4's 8192 x 784 x 256
// dX) take it in the TF32 modes too: 35.5 against 40.2 us there, with exact
// products (inside the TF32-mode error bar).
static bool to_f32(const GemmArgs& g, int terms) {
    return narrow_kind(g) || tn_split_to_f32(g, terms) || f32_takes_w112(g);
}

size_t gemm_bf16x3_workspace(const GemmArgs& g, int terms) {
    if (to_f32(g, terms)) return gemm_f32_workspace(g);
    switch (choose_bf(g, terms)) {
        case BfCfg::SkinnyM: return ws_of<CfgSkinnyM>(g);
        case BfCfg::Huge: return ws_of<CfgHuge>(g);
        case BfCfg::KAlt:
            return splitk_bytes(g, (g.M / 128) * (g.N / 128), 32);   // launch_kalt_ops's policy
        case BfCfg::Large: return ws_of<CfgLarge>(g);
        default: return ws_of<CfgSmall>(g);
    }
}

// Products with K <= 16 or N <= 16 (narrow_kind) take the FP32 narrow
// kernels in the TF32 modes too: they are bound by memory, not by the MFMA
// rate, and their exact fp32 products are inside the TF32-mode error bar.
int launch_gemm_bf16x3(const GemmArgs& g, int terms, hipStream_t stream) {
    if (to_f32(g, terms)) return launch_gemm_f32(g, stream);
    return terms == 4 ? dispatch<4>(g, stream) : dispatch<3>(g, stream);
}

int launch_gemm_16(const GemmArgs& g, int in_dtype, hipStream_t stream) {
    return in_dtype == CDX_DTYPE_BF16 ? dispatch16<kInBF16>(g, stream) : dispatch16<kInF16>(g, stream);
}

}  // namespace cdx
