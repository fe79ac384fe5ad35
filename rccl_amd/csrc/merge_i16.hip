// DeviceMerge instantiation for i16 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(i16, int16_t)
} // namespace merge
} // namespace rccl_hip
