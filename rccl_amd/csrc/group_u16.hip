// Adjacent-run compaction instantiation for u16 keys (unique and the three
// reduce-by-key operators).
#include "group_kernels.hpp"

namespace rccl_hip {
namespace group {
RCCL_GROUP_DEFINE_KEY(u16, uint16_t)
} // namespace group
} // namespace rccl_hip
