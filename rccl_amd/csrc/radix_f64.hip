// DeviceRadixSort instantiation for f64 keys (both orders, every value width).
#include "radix_kernels.hpp"

namespace rccl_hip {
namespace radix {
RCCL_RADIX_DEFINE_KIND(f64, uint64_t, Float)
} // namespace radix
} // namespace rccl_hip
