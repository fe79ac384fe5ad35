// DeviceMerge instantiation for u16 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(u16, uint16_t)
} // namespace merge
} // namespace rccl_hip
