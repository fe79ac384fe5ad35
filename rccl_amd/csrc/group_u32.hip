// Adjacent-run compaction instantiation for u32 keys (unique and the three
// reduce-by-key operators).
#include "group_kernels.hpp"

namespace rccl_hip {
namespace group {
RCCL_GROUP_DEFINE_KEY(u32, uint32_t)
} // namespace group
} // namespace rccl_hip
