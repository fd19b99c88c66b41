// Instantiations: two-group (ping-pong) 256 x 256 kernel for fp32 (bf16x3), fp16 and bf16 operands (gemm_split.hpp).
#include "gemm_split.hpp"

namespace cdx {
namespace split {

template int launch_pingpong_ops<kInF32>(const GemmArgs&, hipStream_t);
template int launch_pingpong_ops<kInF16>(const GemmArgs&, hipStream_t);
template int launch_pingpong_ops<kInBF16>(const GemmArgs&, hipStream_t);

}  // namespace split
}  // namespace cdx
