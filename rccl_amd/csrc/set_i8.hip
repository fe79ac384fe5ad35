// Set operation instantiation for i8 keys (four operations, both orders,
// every value width).
#include "set_ops_kernels.hpp"

namespace rccl_hip {
namespace set_ops {
RCCL_SET_DEFINE_KIND(i8, int8_t)
} // namespace set_ops
} // namespace rccl_hip
