// Two-level decoupled look-back over per-tile counts, for kernels whose tiles
// are numbered so that every tile a look-back waits on has been started
// (claim_tile: XCD order or an atomic ticket) and that need each tile's
// exclusive prefix: the set operations' and the compactions' output offsets.
//
// Every tile publishes its count at once (flag AGG) and, after its look-back,
// its inclusive prefix (flag INCL); it also adds (1 << GA_SHIFT) | count to
// its group's aggregate word, which is complete exactly when its top bits
// equal GROUP, and the group's last tile publishes the group's inclusive
// prefix. One wave looks back: lane l polls in-group predecessor l, then
// earlier groups 64 at a time, newest first.
#pragma once

#include <algorithm>

#include "common.hpp"

namespace rccl_hip {
namespace lookback {

constexpr size_t GROUP = 64;  // tiles per group (one wave polls a group)
// Descriptor words: 2 flag bits over a 62-bit count.
constexpr uint64_t F_AGG = 1ull << 62, F_INCL = 2ull << 62, VMASK = (1ull << 62) - 1;
// Group aggregate: tiles counted in the top 16 bits, count below.
constexpr int GA_SHIFT = 48;
constexpr uint64_t GA_MASK = (1ull << GA_SHIFT) - 1;

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Called by the 64 lanes of one wave of tile t (of `tiles`), whose count is
// tile_count. desc holds `tiles` words, gagg and ginc one word per group, all
// zero before the launch. Returns the sum of the counts of tiles 0..t-1 (in
// every lane).
__device__ __forceinline__ uint64_t tile_prefix(size_t t, size_t tiles, uint64_t tile_count,
                                                uint64_t *desc, uint64_t *gagg, uint64_t *ginc,
                                                uint32_t lane) {
  const size_t g = t / GROUP;
  const size_t gfirst = g * GROUP;
  const uint32_t pos = static_cast<uint32_t>(t - gfirst);
  if (lane == 0) {
    store_agent(&desc[t], (t == 0 ? F_INCL : F_AGG) | tile_count);
    add_agent(&gagg[g], uint64_t((1ull << GA_SHIFT) | tile_count));
  }
  uint64_t prefix = 0;
  if (t > 0) {
    bool done = false;
    if (pos > 0) {
      // In-group predecessors: lane l polls tile gfirst + l (l < pos) until
      // every one has published; the sum then runs from the newest inclusive
      // prefix (if any) up to this tile. Lane 63 (never a polling lane) reads
      // the previous group's inclusive prefix in the same round trip: when no
      // in-group predecessor is inclusive yet, that prefix plus all of them
      // completes the sum without a walk over the groups.
      uint64_t d, gw = 0;
      while (true) {
        d = lane < pos ? load_agent(&desc[gfirst + lane]) : F_AGG;
        if (lane == 63 && g > 0) gw = load_agent(&ginc[g - 1]);
        if (__ballot((d >> 62) == 0) == 0) break;
        __builtin_amdgcn_s_sleep(1);
      }
      const uint64_t incl = __ballot(lane < pos && (d >> 62) == 2);
      const int hi = incl ? 63 - __clzll(static_cast<long long>(incl)) : -1;
      prefix = wave_sum_u64((lane < pos && int(lane) >= hi) ? (d & VMASK) : 0);
      done = hi >= 0;
      if (!done) {
        const uint64_t gv = static_cast<uint64_t>(__shfl(static_cast<long long>(gw), 63, 64));
        if ((gv >> 62) == 2) {
          prefix += gv & VMASK;
          done = true;
        }
      }
    }
    // Earlier groups, newest first, 64 at a time: complete aggregates are
    // summed until a group's inclusive prefix (groups before the first are
    // read as an inclusive zero).
    long long gg = static_cast<long long>(g) - 1;
    while (!done) {
      const long long gi = gg - static_cast<long long>(lane);
      const uint64_t inc_w = gi >= 0 ? load_agent(&ginc[gi]) : F_INCL;
      const uint64_t agg_w = gi >= 0 ? load_agent(&gagg[gi]) : 0;
      const uint64_t incl_lanes = __ballot((inc_w >> 62) == 2);
      const uint64_t full_lanes = __ballot((agg_w >> GA_SHIFT) == uint64_t(GROUP));
      // First lane (newest group) holding an inclusive prefix, if any.
      const int first_incl = incl_lanes ? __ffsll(static_cast<long long>(incl_lanes)) - 1 : 64;
      // Groups before it must all be complete to be summed.
      const uint64_t before = first_incl == 64 ? ~0ull : ((1ull << first_incl) - 1);
      const int first_gap =
          (~full_lanes & before) ? __ffsll(static_cast<long long>(~full_lanes & before)) - 1 : 64;
      if (first_gap < first_incl) {
        // Sum the complete groups before the gap and poll again from it.
        prefix += wave_sum_u64(int(lane) < first_gap ? (agg_w & GA_MASK) : 0);
        gg -= first_gap;
        if (first_gap == 0) __builtin_amdgcn_s_sleep(1);
        continue;
      }
      uint64_t v = int(lane) < first_incl ? (agg_w & GA_MASK) : 0;
      if (int(lane) == first_incl) v = inc_w & VMASK;
      prefix += wave_sum_u64(v);
      if (first_incl < 64) break;
      gg -= 64;
    }
    if (lane == 0) store_agent(&desc[t], F_INCL | (prefix + tile_count));
  }
  const size_t glast = std::min(gfirst + GROUP, tiles) - 1;
  if (lane == 0 && t == glast) store_agent(&ginc[g], F_INCL | (prefix + tile_count));
  return prefix;
}

// Look-back state of `tiles` tiles, as word offsets into one span that is
// zeroed before a launch: tile descriptors, a gap of GAP words, group
// aggregates, another gap, group prefixes, the tile ticket. The gaps keep the
// descriptors and group prefixes, which look-backs read, off the cache lines
// of the group aggregates, the targets of every tile's atomics (a read of
// such a line contends with them: 0.0179 -> 0.021 ms for a 2^20-key
// reduce_by_key whose few groups shared one line).
constexpr size_t GAP = 16;  // 128 bytes
struct State {
  size_t gagg, ginc, ticket, words;
};
inline State state_layout(size_t tiles) {
  const size_t groups = (tiles + GROUP - 1) / GROUP;
  State s;
  s.gagg = tiles + GAP;
  s.ginc = s.gagg + groups + GAP;
  s.ticket = s.ginc + groups;
  s.words = s.ticket + 1;
  return s;
}
inline size_t state_words(size_t tiles) { return state_layout(tiles).words; }

// Tile of the calling block. Where the device places the blocks of a launch
// on its XCDs round-robin (nx == XCDS, probed when the program is loaded),
// tiles go in XCD order (xcd_order_tile): neighbouring tiles share an L2 and
// no atomic is taken. Otherwise the block claims its tile from an atomic
// ticket: a tile is only claimed by a started block, so the lowest unfinished
// tile never waits on an unstarted one, whatever the placement. `slot` is a
// __shared__ word; every thread of the block calls this.
template <uint32_t RUN>
__device__ __forceinline__ size_t claim_tile(uint32_t nx, uint64_t *ticket, uint64_t &slot) {
  if (nx == XCDS) return xcd_order_tile<RUN>(blockIdx.x);
  if (threadIdx.x == 0) slot = add_agent(ticket, uint64_t(1));
  __syncthreads();
  return static_cast<size_t>(slot);
}

} // namespace lookback
} // namespace rccl_hip
