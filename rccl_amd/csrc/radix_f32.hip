// DeviceRadixSort instantiation for f32 keys (both orders, every value width).
#include "radix_kernels.hpp"

namespace rccl_hip {
namespace radix {
RCCL_RADIX_DEFINE_KIND(f32, uint32_t, Float)
} // namespace radix
} // namespace rccl_hip
