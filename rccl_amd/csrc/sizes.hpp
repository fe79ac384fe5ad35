// Size helpers and device constants shared by host and device code, with no
// HIP dependency (the radix plan header and CPU test builds include them).
#pragma once

#include <cstddef>
#include <cstdint>

namespace rccl_hip {

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// XCDs (accelerator complex dies) of a gfx950 device, each with its own L2.
constexpr uint32_t XCDS = 8;

} // namespace rccl_hip
