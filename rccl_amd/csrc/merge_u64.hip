// DeviceMerge instantiation for u64 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(u64, uint64_t)
} // namespace merge
} // namespace rccl_hip
