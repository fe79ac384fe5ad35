// DeviceRadixSort instantiation for u64 keys (both orders, every value width).
#include "radix_kernels.hpp"

namespace rccl_hip {
namespace radix {
RCCL_RADIX_DEFINE_KIND(u64, uint64_t, Unsigned)
} // namespace radix
} // namespace rccl_hip
