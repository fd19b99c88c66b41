// Instantiations: bf16-operand GEMM, tile configurations (gemm_split.hpp).
#include "gemm_split.hpp"

namespace cdx {
namespace split {

template int launch_ops<Cfg16Huge, 1, kInBF16>(const GemmArgs&, hipStream_t);
template int launch_ops<Cfg16Large, 1, kInBF16>(const GemmArgs&, hipStream_t);
template int launch_ops<Cfg16Small, 1, kInBF16>(const GemmArgs&, hipStream_t);

}  // namespace split
}  // namespace cdx
