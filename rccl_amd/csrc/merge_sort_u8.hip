// DeviceMergeSort instantiation for u8 keys (both orders, every value width).
#include "merge_sort_kernels.hpp"

namespace rccl_hip {
namespace merge_sort {
RCCL_MERGE_SORT_DEFINE_KIND(u8, uint8_t)
} // namespace merge_sort
} // namespace rccl_hip
