// DeviceMerge instantiation for u8 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(u8, uint8_t)
} // namespace merge
} // namespace rccl_hip
