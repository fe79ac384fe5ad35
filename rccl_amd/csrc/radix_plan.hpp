// Pass planning and workspace layout of the radix sort: plain host/device
// C++ with no HIP dependency, so that a CPU build (the tests' sanitized plan
// and layout checks) compiles the same code as the library.
#pragma once

#include <cstddef>
#include <cstdint>

#include "sizes.hpp"

#if defined(__HIPCC__)
#define RCCL_RADIX_HD __host__ __device__
#else
#define RCCL_RADIX_HD
#endif

namespace rccl_hip {
namespace radix {

constexpr int BINS = 256;

// Conversion flags of one onesweep launch: its input is raw keys (convert
// after loading), its output must be raw keys (convert before storing).
constexpr uint32_t CONV_IN = 1u, CONV_OUT = 2u;

// ---------------------------------------------------------------------------
// Policy. Tile = threads x items keys, the largest that keeps the staged tile
// in LDS at full wave occupancy (per-tile costs, above all the look-back,
// dominate smaller tiles). Keys-only sorts use two 512-thread blocks per CU;
// pair sorts one 1024-thread block per CU. Items depend on the widest staged
// element (key or value). Overridable at build time for tuning.
// ---------------------------------------------------------------------------
#ifndef RCCL_RADIX_KEYS_THREADS
#define RCCL_RADIX_KEYS_THREADS 512
#endif
#ifndef RCCL_RADIX_KEYS_ITEMS_4B
#define RCCL_RADIX_KEYS_ITEMS_4B 34
#endif
#ifndef RCCL_RADIX_KEYS_ITEMS_8B
#define RCCL_RADIX_KEYS_ITEMS_8B 17
#endif
#ifndef RCCL_RADIX_PAIRS_THREADS
#define RCCL_RADIX_PAIRS_THREADS 1024
#endif
#ifndef RCCL_RADIX_PAIRS_ITEMS_4B
#define RCCL_RADIX_PAIRS_ITEMS_4B 28
#endif
#ifndef RCCL_RADIX_PAIRS_ITEMS_8B
#define RCCL_RADIX_PAIRS_ITEMS_8B 16
#endif
#ifndef RCCL_RADIX_PAIRS_ITEMS_16B
#define RCCL_RADIX_PAIRS_ITEMS_16B 8
#endif
#ifndef RCCL_RADIX_LOOKBACK_WINDOW
#define RCCL_RADIX_LOOKBACK_WINDOW 16
#endif
#ifndef RCCL_RADIX_WAVES_PER_SIMD
#define RCCL_RADIX_WAVES_PER_SIMD 4
#endif
#ifndef RCCL_RADIX_LOOKBACK_GROUP
#define RCCL_RADIX_LOOKBACK_GROUP 16
#endif
#ifndef RCCL_RADIX_LDS_BATCH
#define RCCL_RADIX_LDS_BATCH 8
#endif
#ifndef RCCL_RADIX_GROUP_WINDOW
#define RCCL_RADIX_GROUP_WINDOW 4
#endif
// Tiles per XCD run: consecutive tiles are handed to consecutive blocks of one
// XCD in runs of this many (see onesweep_kernel).
#ifndef RCCL_RADIX_XCD_RUN
#define RCCL_RADIX_XCD_RUN 8
#endif
constexpr int LOOKBACK = RCCL_RADIX_LOOKBACK_WINDOW;
// Tile slots of the look-back window: half as many for 64-bit descriptors,
// which keeps the window at the same registers (the wide window otherwise
// pushes pair sorts past the register budget into scratch).
template <class Desc>
constexpr int lookback_window() {
  return sizeof(Desc) == 8 ? (LOOKBACK + 1) / 2 : LOOKBACK;
}
constexpr int GROUP = RCCL_RADIX_LOOKBACK_GROUP;
constexpr int GWIN = RCCL_RADIX_GROUP_WINDOW;
constexpr uint32_t XCD_RUN = RCCL_RADIX_XCD_RUN;

constexpr int threads_for(size_t value_bytes) {
  return value_bytes ? RCCL_RADIX_PAIRS_THREADS : RCCL_RADIX_KEYS_THREADS;
}
constexpr size_t stage_elem(size_t key_bytes, size_t value_bytes) {
  return key_bytes > value_bytes ? key_bytes : value_bytes;
}
constexpr int items_for(size_t key_bytes, size_t value_bytes) {
  return value_bytes == 0
             ? (key_bytes <= 4 ? RCCL_RADIX_KEYS_ITEMS_4B : RCCL_RADIX_KEYS_ITEMS_8B)
             : (stage_elem(key_bytes, value_bytes) <= 4
                    ? RCCL_RADIX_PAIRS_ITEMS_4B
                    : (stage_elem(key_bytes, value_bytes) <= 8 ? RCCL_RADIX_PAIRS_ITEMS_8B
                                                               : RCCL_RADIX_PAIRS_ITEMS_16B));
}
constexpr size_t tile_items(size_t key_bytes, size_t value_bytes) {
  return size_t(threads_for(value_bytes)) * items_for(key_bytes, value_bytes);
}

// Small-input tiles: inputs of at most RCCL_RADIX_SMALL_MAX_TILES small tiles
// use blocks of SMALL_THREADS threads with half the items, a quarter of a keys
// tile (an eighth of a pairs tile), so that a cache-resident input still
// spreads over every CU: 2^20 u32 keys make 241 tiles instead of 61 (76 -> 66
// us per sort). Measured crossover: small tiles are faster up to 2^21 u32 keys
// and 2^20 u64 + u32 pairs (512 small tiles), slower from 2^22 and 2^21.
// Sorts with a pass plan (the merge-sort lowering) keep the large tiles.
#ifndef RCCL_RADIX_SMALL_THREADS
#define RCCL_RADIX_SMALL_THREADS 256
#endif
#ifndef RCCL_RADIX_SMALL_MAX_TILES
#define RCCL_RADIX_SMALL_MAX_TILES 512
#endif
#ifndef RCCL_RADIX_SMALL_ITEMS_DIV
#define RCCL_RADIX_SMALL_ITEMS_DIV 2
#endif
constexpr int SMALL_THREADS = RCCL_RADIX_SMALL_THREADS;
constexpr int small_items_for(size_t key_bytes, size_t value_bytes) {
  return items_for(key_bytes, value_bytes) / RCCL_RADIX_SMALL_ITEMS_DIV > 0
             ? items_for(key_bytes, value_bytes) / RCCL_RADIX_SMALL_ITEMS_DIV
             : 1;
}
constexpr size_t small_tile_items(size_t key_bytes, size_t value_bytes) {
  return size_t(SMALL_THREADS) * small_items_for(key_bytes, value_bytes);
}
// Whether a sort of n items uses the small tiles (the layout and the launches
// both ask this).
constexpr bool small_tiles(size_t key_bytes, size_t value_bytes, size_t n, bool planned) {
  return !planned && n <= size_t(RCCL_RADIX_SMALL_MAX_TILES) * small_tile_items(key_bytes,
                                                                               value_bytes);
}

// Pass plan of a sort that skips trivial passes (one digit holds every key:
// the pass would not move anything). Buffers: 0 the input, 1 the output,
// 2 the scratch; lb is the look-back buffer of the pass (the active passes
// alternate, starting with buffer 0, which the histogram zeroes).
struct PassPlan {
  uint32_t active, src, dst, lb, conv;  // conv: CONV_IN on the first active pass, CONV_OUT on the last
};

// Plan flags: some stream (keys or values) is sorted in place (input ==
// output), and some stream is not (its output must be written even when no
// pass moves anything).
constexpr uint32_t PLAN_IN_PLACE = 1u, PLAN_COPIES = 2u;

// Thread-serial plan for P passes, `trivial` bit p set when pass p is
// trivial. The active passes alternate between output and scratch so that
// the last one writes the output; the first reads the input. With a stream in
// place the first must write the scratch, so the active count must be even:
// a trivial pass is activated when it is odd (P is even, so one exists). When
// no pass is active and another stream is not in place, two trivial passes
// run (input -> scratch -> output: P >= 2), so that stream's output is
// written too. Entirely out of place, at least one pass runs, a stable copy
// into the output.
RCCL_RADIX_HD inline void assign_plan(int P, uint32_t trivial, uint32_t flags,
                                      PassPlan *__restrict__ plan) {
  uint32_t act = ~trivial & ((P >= 32 ? 0u : (1u << P)) - 1u);
  int k = __builtin_popcount(act);
  if (flags & PLAN_IN_PLACE) {
    if (k & 1) {
      act |= trivial & (0u - trivial);  // the lowest trivial pass
      ++k;
    } else if (k == 0 && (flags & PLAN_COPIES)) {
      act = 3u;  // every pass is trivial: the two lowest
      k = 2;
    }
  } else if (k == 0) {
    act = 1u << (P - 1);
    k = 1;
  }
  uint32_t j = 0, prev = 0;
  for (int p = 0; p < P; ++p) {
    PassPlan e{0u, 0u, 0u, 0u, 0u};
    if (act & (1u << p)) {
      const uint32_t dst = ((uint32_t(k) - 1u - j) & 1u) ? 2u : 1u;
      e = PassPlan{1u, j == 0 ? 0u : prev, dst, j & 1u,
                   (j == 0 ? CONV_IN : 0u) | (j + 1 == uint32_t(k) ? CONV_OUT : 0u)};
      prev = dst;
      ++j;
    }
    plan[p] = e;
  }
}

// Largest item count the control words support: 30-bit look-back counts
// switch to 62-bit descriptors at 2^30; positions are 32-bit.
constexpr uint64_t MAX_ITEMS = 0xffffffffull;

struct Layout {
  size_t tiles = 0;
  size_t groups = 0;
  size_t desc_bytes = 4;
  bool small = false;  // small_tiles()
  size_t bins = 0;
  size_t skew = 0;  // one skew word per pass (bins_scan_kernel)
  // Look-back buffers: tile descriptors, group prefixes, group aggregates and
  // the pass's tile tickets.
  size_t lb[2] = {0, 0};
  size_t lb_ginc = 0, lb_gagg = 0, lb_ticket = 0, lb_bytes = 0;  // within one buffer
  size_t total = 0;
};


// Workspace layout of a sort of n items: the bins, one skew word per pass and
// two look-back buffers (tile descriptors, group prefixes, group aggregates
// and tile tickets), each region aligned to 256 bytes.
inline Layout layout(size_t key_bytes, size_t value_bytes, size_t n, bool planned) {
  Layout l;
  const size_t max_passes = key_bytes;  // 8-bit digits
  l.small = small_tiles(key_bytes, value_bytes, n, planned);
  const size_t tile =
      l.small ? small_tile_items(key_bytes, value_bytes) : tile_items(key_bytes, value_bytes);
  l.tiles = (n + tile - 1) / tile;
  l.desc_bytes = n < (size_t(1) << 30) ? 4 : 8;
  size_t off = 0;
  l.bins = off;
  off += align_up(max_passes * BINS * sizeof(uint32_t), 256);
  l.skew = off;
  off += align_up(max_passes * sizeof(uint32_t), 256);
  l.groups = (l.tiles + GROUP - 1) / GROUP;
  l.lb_ginc = align_up(l.tiles * BINS * l.desc_bytes, 256);
  l.lb_gagg = l.lb_ginc + align_up(l.groups * BINS * l.desc_bytes, 256);
  l.lb_ticket = l.lb_gagg + align_up(l.groups * BINS * sizeof(uint32_t), 256);
  l.lb_bytes = l.lb_ticket + align_up(XCDS * sizeof(uint32_t), 256);
  l.lb[0] = off;
  off += l.lb_bytes;
  l.lb[1] = off;
  off += l.lb_bytes;
  l.total = n == 0 ? 0 : off;
  return l;
}

// Workspace of a planned sort's pass plan (one PassPlan per pass, at most 8),
// after the layout's total.
inline size_t plan_bytes() { return align_up(8 * sizeof(PassPlan), 256); }

} // namespace radix
} // namespace rccl_hip
