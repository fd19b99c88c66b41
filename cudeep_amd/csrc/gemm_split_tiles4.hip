// Instantiations: four-term (bf16x4) split GEMM, every tile configuration (gemm_split.hpp).
#include "gemm_split.hpp"

namespace cdx {
namespace split {

template int launch_ops<CfgSkinnyM, 4, kInF32>(const GemmArgs&, hipStream_t);
template int launch_ops<CfgLarge, 4, kInF32>(const GemmArgs&, hipStream_t);
template int launch_ops<CfgSmall, 4, kInF32>(const GemmArgs&, hipStream_t);

}  // namespace split
}  // namespace cdx
