// Adjacent-run compaction instantiation for f32 keys (unique and the three
// reduce-by-key operators).
#include "group_kernels.hpp"

namespace rccl_hip {
namespace group {
RCCL_GROUP_DEFINE_KEY(f32, float)
} // namespace group
} // namespace rccl_hip
