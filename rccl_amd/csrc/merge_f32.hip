// DeviceMerge instantiation for f32 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(f32, float)
} // namespace merge
} // namespace rccl_hip
