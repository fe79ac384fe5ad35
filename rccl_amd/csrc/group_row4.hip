// Adjacent-run compaction instantiation for row4 keys (unique and the three
// reduce-by-key operators).
#include "group_kernels.hpp"

namespace rccl_hip {
namespace group {
RCCL_GROUP_DEFINE_KEY(row4, record_sort::Row<4>)
} // namespace group
} // namespace rccl_hip
