// DeviceMerge instantiation for u32 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(u32, uint32_t)
} // namespace merge
} // namespace rccl_hip
