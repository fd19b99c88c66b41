// Instantiations: three-term (bf16x3) split GEMM, every tile configuration (gemm_split.hpp).
#include "gemm_split.hpp"

namespace cdx {
namespace split {

template int launch_ops<CfgSkinnyM, 3, kInF32>(const GemmArgs&, hipStream_t);
template int launch_ops<CfgHuge, 3, kInF32>(const GemmArgs&, hipStream_t);
template int launch_ops<CfgLarge, 3, kInF32>(const GemmArgs&, hipStream_t);
template int launch_ops<CfgSmall, 3, kInF32>(const GemmArgs&, hipStream_t);

}  // namespace split
}  // namespace cdx
