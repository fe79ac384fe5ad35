// Set operation instantiation for f64 keys (four operations, both orders,
// every value width).
#include "set_ops_kernels.hpp"

namespace rccl_hip {
namespace set_ops {
RCCL_SET_DEFINE_KIND(f64, double)
} // namespace set_ops
} // namespace rccl_hip
