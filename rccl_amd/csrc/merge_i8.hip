// DeviceMerge instantiation for i8 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(i8, int8_t)
} // namespace merge
} // namespace rccl_hip
