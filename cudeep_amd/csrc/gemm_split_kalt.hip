// Instantiations: k-alternating two-group 128 x 128 kernel, three and four terms (gemm_split.hpp).
#include "gemm_split.hpp"

namespace cdx {
namespace split {

template int launch_kalt_ops<3>(const GemmArgs&, hipStream_t);
template int launch_kalt_ops<4>(const GemmArgs&, hipStream_t);

}  // namespace split
}  // namespace cdx
