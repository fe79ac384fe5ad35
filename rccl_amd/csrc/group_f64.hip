// Adjacent-run compaction instantiation for f64 keys (unique and the three
// reduce-by-key operators).
#include "group_kernels.hpp"

namespace rccl_hip {
namespace group {
RCCL_GROUP_DEFINE_KEY(f64, double)
} // namespace group
} // namespace rccl_hip
