// Record sort instantiation for [u32; 5] rows (every payload width).
#include "record_sort_kernels.hpp"

namespace rccl_hip {
namespace record_sort {
RCCL_RECORD_SORT_DEFINE_ARITY(5)
} // namespace record_sort
} // namespace rccl_hip
