// Adjacent-run compaction instantiation for row5 keys (unique and the three
// reduce-by-key operators).
#include "group_kernels.hpp"

namespace rccl_hip {
namespace group {
RCCL_GROUP_DEFINE_KEY(row5, record_sort::Row<5>)
} // namespace group
} // namespace rccl_hip
