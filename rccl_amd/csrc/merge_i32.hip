// DeviceMerge instantiation for i32 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(i32, int32_t)
} // namespace merge
} // namespace rccl_hip
