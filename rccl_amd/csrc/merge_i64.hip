// DeviceMerge instantiation for i64 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(i64, int64_t)
} // namespace merge
} // namespace rccl_hip
