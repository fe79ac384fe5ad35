// Adjacent-run compaction instantiation for i64 keys (unique and the three
// reduce-by-key operators).
#include "group_kernels.hpp"

namespace rccl_hip {
namespace group {
RCCL_GROUP_DEFINE_KEY(i64, int64_t)
} // namespace group
} // namespace rccl_hip
