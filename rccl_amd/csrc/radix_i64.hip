// DeviceRadixSort instantiation for i64 keys (both orders, every value width).
#include "radix_kernels.hpp"

namespace rccl_hip {
namespace radix {
RCCL_RADIX_DEFINE_KIND(i64, uint64_t, Signed)
} // namespace radix
} // namespace rccl_hip
