// DeviceMerge instantiation for f64 keys (both orders, every value width).
#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge {
RCCL_MERGE_DEFINE_KIND(f64, double)
} // namespace merge
} // namespace rccl_hip
