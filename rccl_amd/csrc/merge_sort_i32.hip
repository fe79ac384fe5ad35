// DeviceMergeSort instantiation for i32 keys (both orders, every value width).
#include "merge_sort_kernels.hpp"

namespace rccl_hip {
namespace merge_sort {
RCCL_MERGE_SORT_DEFINE_KIND(i32, int32_t)
} // namespace merge_sort
} // namespace rccl_hip
