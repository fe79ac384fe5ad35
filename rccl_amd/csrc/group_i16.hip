// Adjacent-run compaction instantiation for i16 keys (unique and the three
// reduce-by-key operators).
#include "group_kernels.hpp"

namespace rccl_hip {
namespace group {
RCCL_GROUP_DEFINE_KEY(i16, int16_t)
} // namespace group
} // namespace rccl_hip
