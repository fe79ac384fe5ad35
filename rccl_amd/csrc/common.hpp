// Shared host/device helpers for the rccl_hip library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "rccl_hip.h"
#include "sizes.hpp"

namespace rccl_hip {

// ---------------------------------------------------------------------------
// Error reporting (host). Mirrors DeviceAlgorithmError's payloads
// (rccl-cub/src/error.rs:3-25); the last error is kept per thread.
// ---------------------------------------------------------------------------
rccl_hip_status set_error(rccl_hip_status status, const char *role = "",
                          uint64_t expected = 0, uint64_t actual = 0);
rccl_hip_status set_bit_range_error(uint32_t begin, uint32_t end, uint32_t key_bits);
rccl_hip_status set_hip_error(rccl_hip_status status, const char *role, hipError_t err);
rccl_hip_status ok();

#define RCCL_HIP_TRY(expr)                                                      \
  do {                                                                         \
    rccl_hip_status rccl_hip_try_status_ = (expr);                             \
    if (rccl_hip_try_status_ != RCCL_HIP_SUCCESS) return rccl_hip_try_status_; \
  } while (0)

// Launch check: reports a launch failure as RCCL_HIP_ERROR_LAUNCH.
rccl_hip_status check_launch(const char *role);

// Per-launch hipEvent timing (rccl_hip_timing_enable). Construct around a
// launch: records a start event now and a stop event when destroyed, on the
// launch's stream, only while timing is enabled.
class KernelTimer {
public:
  KernelTimer(const char *name, hipStream_t stream, uint64_t items);
  ~KernelTimer();
  KernelTimer(const KernelTimer &) = delete;
  KernelTimer &operator=(const KernelTimer &) = delete;

private:
  int slot_ = -1;
  hipStream_t stream_;
};


// Whether the byte ranges [a, a + an) and [b, b + bn) share a byte (empty or
// null ranges share none).
inline bool ranges_overlap(const void *a, size_t an, const void *b, size_t bn) {
  if (!a || !b || an == 0 || bn == 0) return false;
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x >= y ? x - y < bn : y - x < an;  // no sum that could wrap
}

// a * b, or SIZE_MAX where that overflows (byte counts of huge capacities).
inline size_t sat_mul(size_t a, size_t b) { return b && a > SIZE_MAX / b ? SIZE_MAX : a * b; }

// Whether any output range shares a byte with any input range: kernels that
// read their inputs tile by tile while writing their outputs elsewhere
// (merge, set operations) would race on such a call. The reference's borrows
// rule it out; through the C ABI it is rejected before any launch.
struct ByteRange {
  const void *p;
  size_t bytes;
};
template <size_t NO, size_t NI>
inline bool outputs_overlap_inputs(const ByteRange (&outs)[NO], const ByteRange (&ins)[NI]) {
  for (const ByteRange &o : outs)
    for (const ByteRange &i : ins)
      if (ranges_overlap(o.p, o.bytes, i.p, i.bytes)) return true;
  return false;
}

// Buffers of a sort with a key stream and an optional value stream (value
// bytes 0: none), each sorted in place (input == output) or into its own
// output: whether some output shares a byte with an input it is not the
// in-place output of, or with the other output. Passes read their input
// while other blocks already write, so such a call would race.
inline bool sort_streams_overlap(const void *in_keys, const void *out_keys, size_t key_bytes,
                                 const void *in_values, const void *out_values,
                                 size_t value_bytes) {
  return (in_keys != out_keys && ranges_overlap(out_keys, key_bytes, in_keys, key_bytes)) ||
         (in_values != out_values &&
          ranges_overlap(out_values, value_bytes, in_values, value_bytes)) ||
         ranges_overlap(out_keys, key_bytes, in_values, value_bytes) ||
         ranges_overlap(out_values, value_bytes, in_keys, key_bytes) ||
         ranges_overlap(out_keys, key_bytes, out_values, value_bytes);
}

// Blocks of `kernel` (launched with `threads` threads and no dynamic LDS) that
// the current device holds at once: CUs x resident blocks per CU. Cached per
// device and kernel.
rccl_hip_status resident_blocks(const void *kernel, int threads, size_t *blocks);

// The XCD-ordered look-back (xcd_order_tile) needs two rows of XCD runs
// resident at once. Where `kernel` cannot hold them, *nx becomes 1: its blocks
// claim tiles from the atomic ticket instead (a tile is claimed only by a
// started block, so the look-back cannot wait on an unstarted one).
rccl_hip_status fit_tile_order(const void *kernel, int threads, uint32_t run, uint32_t *nx);

// Tile order for the current device: XCDS where its blocks land on the XCDs
// round-robin (XCD-ordered tiles), 1 where tiles must be claimed from an
// atomic ticket (the load-time probe failed, or rccl_hip_radix_configure
// asked for tickets). Fails, before any launch, on a stream under graph
// capture when the device was not probed yet (rccl_hip_program_load probes it).
rccl_hip_status tile_order(uint32_t *nx, hipStream_t stream);

inline size_t key_bytes(rccl_hip_key_kind k) {
  switch (k) {
  case RCCL_HIP_KEY_U32: case RCCL_HIP_KEY_I32: case RCCL_HIP_KEY_F32: return 4;
  case RCCL_HIP_KEY_U64: case RCCL_HIP_KEY_I64: case RCCL_HIP_KEY_F64: return 8;
  case RCCL_HIP_KEY_U8: case RCCL_HIP_KEY_I8: return 1;
  case RCCL_HIP_KEY_U16: case RCCL_HIP_KEY_I16: return 2;
  default: return 0;
  }
}

inline bool valid_value_bytes(size_t v) {
  return v == 0 || v == 1 || v == 2 || v == 4 || v == 8 || v == 16;
}

// Opaque 16-byte value payloads moved alongside keys. Copies are one 16-byte
// vector move: a defaulted copy of the struct becomes a byte copy that the
// compiler leaves in scratch memory when it stages arrays of them between LDS
// and registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
struct alignas(16) Value16 {
  u32x4 w;
  Value16() = default;
  __host__ __device__ Value16(const Value16 &o) : w(o.w) {}
  __host__ __device__ Value16 &operator=(const Value16 &o) {
    w = o.w;
    return *this;
  }
};

// ---------------------------------------------------------------------------
// Device helpers (wave64).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

// Number of set bits of `mask` in lanes below the calling lane.
__device__ __forceinline__ uint32_t popc_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// Workgroup barrier that orders LDS only: global loads and stores issued
// before it stay in flight (__syncthreads would wait for all of them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Device-scope (agent) atomics: visible across all XCDs of the GPU.
template <class T>
__device__ __forceinline__ T load_agent(const T *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void store_agent(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T add_agent(T *p, T v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// gfx950 places the blocks of a launch on its 8 XCDs round-robin (block b on
// XCD b % 8). xcd_order_tile(b) hands runs of RUN consecutive tiles to
// consecutive blocks of one XCD, so neighbouring tiles share an L2. Within
// one XCD, tile numbers rise with block numbers, and each XCD starts its
// blocks in order. So in a decoupled look-back the lowest unfinished tile
// has always been started (every earlier block of its XCD holds an earlier
// tile, hence has finished), and the look-back cannot deadlock. The grid is
// rounded up to whole rows of 8 * RUN blocks (xcd_order_grid); blocks whose
// tile is past the end return.
template <uint32_t RUN>
__device__ __forceinline__ uint32_t xcd_order_tile(uint32_t block) {
  const uint32_t x = block % XCDS, j = block / XCDS;
  return XCDS * RUN * (j / RUN) + RUN * x + j % RUN;
}
inline size_t xcd_order_grid(size_t tiles, uint32_t run) {
  const size_t row = size_t(XCDS) * run;
  return (tiles + row - 1) / row * row;
}

// Inclusive scan across the 64 lanes of a wave.
template <class T>
__device__ __forceinline__ T wave_inclusive_sum(T v, uint32_t lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    T t = __shfl_up(v, off, 64);
    if (lane >= static_cast<uint32_t>(off)) v += t;
  }
  return v;
}

// 32-bit inclusive sum over a full wave64 in DPP moves, with no LDS round
// trip: each row of 16 lanes scans with row shifts of 1, 2, 4 and 8 (lanes
// shifted in from outside the row read 0), row_bcast:15 adds the last lane of
// rows 0 and 2 to rows 1 and 3, and row_bcast:31 adds lane 31 (the total of
// rows 0 and 1) to rows 2 and 3. Every lane of the wave must be active.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v, uint32_t) {
  constexpr int ROW_SHR = 0x110, ROW_BCAST15 = 0x142, ROW_BCAST31 = 0x143;
  int x = static_cast<int>(v);
  x += __builtin_amdgcn_update_dpp(0, x, ROW_SHR + 1, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, ROW_SHR + 2, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, ROW_SHR + 4, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, ROW_SHR + 8, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, ROW_BCAST15, 0xa, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, ROW_BCAST31, 0xc, 0xf, false);
  return static_cast<uint32_t>(x);
}

} // namespace rccl_hip
