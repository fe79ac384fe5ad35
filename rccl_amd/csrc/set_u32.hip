// Set operation instantiation for u32 keys (four operations, both orders,
// every value width).
#include "set_ops_kernels.hpp"

namespace rccl_hip {
namespace set_ops {
RCCL_SET_DEFINE_KIND(u32, uint32_t)
} // namespace set_ops
} // namespace rccl_hip
