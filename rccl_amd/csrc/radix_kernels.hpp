// DeviceRadixSort kernels for gfx950: onesweep LSD radix sort, 8-bit digits.
//
// Reference behaviour: rccl-cub/src/radix.rs:364-876 (validation and pass
// control) and rccl-cub/src/ordering_backend/radix.rs (device agents). The
// kernels are an independent wave64 design:
//   init        zero the per-pass bins and tile counters (one tiny block)
//   histogram   one read of all keys builds every pass's 256-bin histogram in
//               LDS (per-wave private counters) and adds them to the bins; it
//               also zeroes look-back buffer 0
//   onesweep    one launch per pass; persistent blocks claim tiles in order,
//               rank them with wave64 LDS match masks, run a windowed
//               decoupled look-back on agent-scope atomics, and scatter
//               through LDS so HBM writes coalesce
#pragma once

#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace rccl_hip {
namespace radix {

constexpr int BINS = 256;

struct NoValue {};

enum class KeyClass { Unsigned, Signed, Float };

// Order-preserving bit image of a key, with the float +-0 collapse applied
// for digit extraction. Transforms: rccl-cub/src/ordering_backend/radix.rs:75-235
// (unsigned identity, signed sign flip, float: negative -> all bits inverted,
// otherwise sign flipped; descending = complement); collapse: :257-337 (the
// ordered value 0x7f..f is read as 0x80..0, so -0.0 and +0.0 share every
// digit). Stored keys are never rewritten.
template <class Bits, KeyClass KC, bool DESC>
struct KeyOps {
  using SBits = typename std::make_signed<Bits>::type;
  static constexpr int NBITS = int(sizeof(Bits) * 8);
  static constexpr Bits SIGN = Bits(1) << (NBITS - 1);

  __device__ static __forceinline__ Bits digit_source(Bits raw) {
    Bits x = raw;
    if constexpr (KC == KeyClass::Signed) x ^= SIGN;
    if constexpr (KC == KeyClass::Float)
      x ^= static_cast<Bits>(static_cast<SBits>(raw) >> (NBITS - 1)) | SIGN;
    if constexpr (DESC) x = ~x;
    if constexpr (KC == KeyClass::Float) x = (x == SIGN - 1) ? SIGN : x;
    return x;
  }

  __device__ static __forceinline__ uint32_t digit(Bits raw, uint32_t bit, uint32_t mask) {
    return static_cast<uint32_t>(digit_source(raw) >> bit) & mask;
  }
};

// Look-back descriptor: 2 flag bits over a count.
template <class Desc> struct DescInfo;
// Flag 3 never appears in memory: it marks a window slot before the start of
// the tile's look-back group.
template <> struct DescInfo<uint32_t> {
  static constexpr int SHIFT = 30;
  static constexpr uint32_t AGG = 1u << 30, INCL = 2u << 30, BOUNDARY = 3u << 30,
                            MASK = (1u << 30) - 1;
};
template <> struct DescInfo<uint64_t> {
  static constexpr int SHIFT = 62;
  static constexpr uint64_t AGG = 1ull << 62, INCL = 2ull << 62, BOUNDARY = 3ull << 62,
                            MASK = (1ull << 62) - 1;
};

// Two-level look-back state of one pass. Tiles form groups of GROUP; besides
// its own descriptor, every tile adds (1 << GAGG_SHIFT) | count to its
// group's per-digit aggregate word, which is therefore complete exactly when
// its top byte equals the group size. The group's last tile also publishes
// the inclusive prefix through the group. A look-back sums in-group
// predecessors tile by tile and earlier groups whole, so the prefix chain
// advances a group per step instead of a tile.
constexpr int GAGG_SHIFT = 24;
constexpr uint32_t GAGG_MASK = (1u << GAGG_SHIFT) - 1;
template <class Desc> struct LookbackBuf {
  Desc *tile;      // tiles x BINS descriptors
  Desc *ginc;      // groups x BINS inclusive prefixes through each group
  uint32_t *gagg;  // groups x BINS packed (tiles counted, count)
};

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
#define RCCL_RADIX_PAIRS_ITEMS_8B 14
#endif
#ifndef RCCL_RADIX_PAIRS_ITEMS_16B
#define RCCL_RADIX_PAIRS_ITEMS_16B 7
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
// Where the next tile is claimed: 0 at the start of a tile, 1 after its
// ranking, 2 at its staging (the prefetch of the next tile's keys then
// follows the look-back).
#ifndef RCCL_RADIX_CLAIM_POINT
#define RCCL_RADIX_CLAIM_POINT 1
#endif
// 1: a persistent grid whose blocks loop over tiles, claiming the next tile
// one ahead and prefetching its keys; 0: one tile per block.
#ifndef RCCL_RADIX_PERSISTENT
#define RCCL_RADIX_PERSISTENT 0
#endif
#ifndef RCCL_RADIX_LDS_BATCH
#define RCCL_RADIX_LDS_BATCH 8
#endif
#ifndef RCCL_RADIX_GROUP_WINDOW
#define RCCL_RADIX_GROUP_WINDOW 4
#endif
constexpr int LOOKBACK = RCCL_RADIX_LOOKBACK_WINDOW;
constexpr int GROUP = RCCL_RADIX_LOOKBACK_GROUP;
constexpr int GWIN = RCCL_RADIX_GROUP_WINDOW;

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

// ---------------------------------------------------------------------------
// init: zero bins and tile counters. (Internal linkage: every translation
// unit that launches it carries its own copy.)
// ---------------------------------------------------------------------------
namespace {
__global__ void __launch_bounds__(256) init_kernel(uint32_t *bins, uint32_t *counters,
                                                   uint32_t passes) {
  for (uint32_t i = threadIdx.x; i < passes * BINS; i += 256) bins[i] = 0;
  if (threadIdx.x < passes) counters[threadIdx.x] = 0;
}
} // namespace

// ---------------------------------------------------------------------------
// histogram: every pass's digit counts from one read of the keys.
// ---------------------------------------------------------------------------
constexpr int HIST_THREADS = 512;
constexpr int HIST_ITEMS = 16;

template <class Bits, class Ops>
__global__ void __launch_bounds__(HIST_THREADS)
histogram_kernel(const Bits *__restrict__ keys, size_t n, uint32_t *__restrict__ bins,
                 uint32_t begin_bit, uint32_t end_bit, uint32_t passes,
                 uint32_t *__restrict__ zero_words, size_t zero_count) {
  constexpr int WAVES = HIST_THREADS / 64;
  constexpr int PMAX = sizeof(Bits);
  __shared__ uint32_t hist[WAVES][PMAX * BINS];
  const uint32_t tid = threadIdx.x;
  for (uint32_t i = tid; i < WAVES * PMAX * BINS; i += HIST_THREADS) (&hist[0][0])[i] = 0;
  for (size_t i = size_t(blockIdx.x) * HIST_THREADS + tid; i < zero_count;
       i += size_t(gridDim.x) * HIST_THREADS)
    zero_words[i] = 0;
  __syncthreads();

  uint32_t *my = hist[tid >> 6];
  constexpr size_t CHUNK = size_t(HIST_THREADS) * HIST_ITEMS;
  for (size_t base = size_t(blockIdx.x) * CHUNK; base < n; base += size_t(gridDim.x) * CHUNK) {
    Bits k[HIST_ITEMS];
    const uint32_t avail = static_cast<uint32_t>(min<size_t>(n - base, CHUNK));
#pragma unroll
    for (int j = 0; j < HIST_ITEMS; ++j) {
      const uint32_t i = uint32_t(j) * HIST_THREADS + tid;
      k[j] = i < avail ? keys[base + i] : Bits(0);
    }
#pragma unroll
    for (int j = 0; j < HIST_ITEMS; ++j) {
      if (uint32_t(j) * HIST_THREADS + tid >= avail) continue;
      const Bits s = Ops::digit_source(k[j]);
      for (uint32_t p = 0; p < passes; ++p) {
        const uint32_t bit = begin_bit + 8u * p;
        const uint32_t width = min(8u, end_bit - bit);
        const uint32_t d = static_cast<uint32_t>(s >> bit) & ((1u << width) - 1u);
        atomicAdd(&my[p * BINS + d], 1u);
      }
    }
  }
  __syncthreads();
  for (uint32_t i = tid; i < passes * BINS; i += HIST_THREADS) {
    uint32_t sum = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) sum += hist[w][i];
    if (sum) add_agent(&bins[i], sum);
  }
}

// Turn every pass's digit counts into exclusive offsets (the first output
// position of each digit), once, so the onesweep blocks read them instead of
// each scanning the bins. One block of BINS threads. (Internal linkage, like
// init_kernel.)
namespace {
__global__ void __launch_bounds__(BINS) bins_scan_kernel(uint32_t *bins, uint32_t passes) {
  __shared__ uint32_t s_wave[BINS / 64];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  for (uint32_t p = 0; p < passes; ++p) {
    const uint32_t c = bins[p * BINS + tid];
    const uint32_t inc = wave_inclusive_sum(c, lane);
    if (lane == 63) s_wave[tid >> 6] = inc;
    __syncthreads();
    uint32_t excl = inc - c;
    for (uint32_t w = 0; w < (tid >> 6); ++w) excl += s_wave[w];
    bins[p * BINS + tid] = excl;
    __syncthreads();
  }
}
} // namespace

// ---------------------------------------------------------------------------
// onesweep: one stable counting-sort pass. Persistent blocks claim tiles of
// THREADS*ITEMS keys in order from an atomic counter and software-pipeline
// them: the look-back window for tile t is issued right after t's aggregate
// is published, and the keys of the next tile are loaded before t's
// look-back is consumed.
// ---------------------------------------------------------------------------
template <class Bits, class Val, class Ops, int ITEMS, class Desc, int THREADS>
__global__ void __launch_bounds__(THREADS, RCCL_RADIX_WAVES_PER_SIMD)
onesweep_kernel(const Bits *__restrict__ keys_in, Bits *__restrict__ keys_out,
                const Val *__restrict__ vals_in, Val *__restrict__ vals_out, size_t n,
                uint32_t num_tiles, const uint32_t *__restrict__ pass_bins,
                LookbackBuf<Desc> lbuf, LookbackBuf<Desc> lbuf_next, uint32_t *tile_counter,
                uint32_t bit, uint32_t mask) {
  constexpr bool PAIRS = !std::is_same<Val, NoValue>::value;
  constexpr int WAVES = THREADS / 64;
  // Ranking works on 32-lane halves of each wave ("sub-waves"), each owning a
  // contiguous chunk of 32 * ITEMS keys.
  constexpr int SUBS = 2 * WAVES;
  constexpr int TILE = THREADS * ITEMS;
  constexpr int SUB_ITEMS = 32 * ITEMS;
  // LDS reads issued back to back before their results are used.
  constexpr int BATCH = RCCL_RADIX_LDS_BATCH;
  // Items past the end of the input (last tile only) rank in an extra
  // dummy bin and stage into one spare slot, so the loops need no branches.
  constexpr int NB = BINS + 1;
  constexpr uint32_t DUMMY = BINS;
  constexpr size_t VAL_BYTES = PAIRS ? sizeof(Val) : 0;
  constexpr size_t STAGE_ELEM = sizeof(Bits) > VAL_BYTES ? sizeof(Bits) : VAL_BYTES;
  static_assert(THREADS >= BINS, "one thread per digit is required");
  static_assert(uint64_t(GROUP) * TILE <= GAGG_MASK, "group counts must fit the packed word");
  static_assert(LOOKBACK >= 1 && GWIN >= 1, "look-back windows");
  using DI = DescInfo<Desc>;
  using ValReg = typename std::conditional<PAIRS, Val, char>::type;

  // Ranking words (one per sub-wave and digit: the sub-wave's running digit
  // count in the high half, the match mask of the current item in the low
  // half) and the staged tile (scatter) are never live at the same time, so
  // they share one LDS buffer.
  constexpr size_t STAGE_BYTES = (TILE + 1) * STAGE_ELEM;
  constexpr size_t RANK_BYTES = size_t(SUBS) * NB * sizeof(uint64_t);
  __shared__ __attribute__((aligned(16)))
  unsigned char stage_raw[STAGE_BYTES > RANK_BYTES ? STAGE_BYTES : RANK_BYTES];
  uint64_t(*rankw)[NB] = reinterpret_cast<uint64_t(*)[NB]>(stage_raw);
  // Per sub-wave and digit: first tile position of that sub-wave's keys.
  // 16-bit: offsets are tile-relative (at most TILE), which halves the table.
  static_assert(TILE < 65536, "tile offsets are 16-bit");
  __shared__ uint16_t hist[SUBS][NB];
  __shared__ uint32_t digit_off[BINS];
  __shared__ uint32_t wave_sum[BINS / 64];
  __shared__ uint32_t s_tile;

  const uint32_t tid0 = threadIdx.x;
  Bits *stage_keys = reinterpret_cast<Bits *>(stage_raw);

  if (tid0 == 0) s_tile = add_agent(tile_counter, 1u);
  // Global start of each digit's bucket (exclusive offsets computed by the
  // histogram kernel).
  const uint32_t bin_start = tid0 < BINS ? pass_bins[tid0] : 0u;
  __syncthreads();
  uint32_t tile = s_tile;
  if (tile >= num_tiles) return;
  // Sub-wave-contiguous, lane-striped load: item j of sub-wave lane l is key
  // sub_base + 32 j + l, so (sub-wave, item, lane) order is source order.
  // Loads are clamped instead of predicated: items past the end rank as
  // dummies whatever they hold, and unpredicated loads keep the compiler's
  // memory-counter waits exact.
  Bits key[ITEMS];
  const size_t last_item = n - 1;
  size_t sub_base = size_t(tile) * TILE + size_t(tid0 >> 5) * SUB_ITEMS;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j)
    key[j] = keys_in[min(sub_base + size_t(j) * 32 + (tid0 & 31u), last_item)];
  // The next tile is claimed one tile ahead by a thread of a wave that has no
  // other global memory traffic before the claim is consumed, so waiting for
  // the claim never waits for look-back or prefetch loads. Claims only ever
  // grow, so a block's next tile is above its current one and the lowest
  // tile in progress never waits on an unstarted tile.
  constexpr uint32_t CLAIM = BINS;
  static_assert(!RCCL_RADIX_PERSISTENT || THREADS > BINS,
                "the claiming thread must not be a look-back thread");
  uint32_t claimed = 0;


  while (true) {
#if RCCL_RADIX_PERSISTENT && RCCL_RADIX_CLAIM_POINT == 0
    if (threadIdx.x == CLAIM) claimed = add_agent(tile_counter, 1u);
#endif
    // Values derived from the thread index are recomputed every tile: an
    // opaque copy keeps the compiler from hoisting dozens of per-item
    // addresses out of the tile loop into registers.
    uint32_t tid = tid0;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t sw = tid >> 5;       // sub-wave
    const uint32_t sl = tid & 31u;      // lane within the sub-wave
    // The staging buffer of the previous tile becomes this tile's ranking
    // words: clear them (the end-of-tile barrier has passed).
    for (uint32_t i = tid; i < SUBS * NB; i += THREADS) (&rankw[0][0])[i] = 0;
    __syncthreads();
    uint64_t *srank = rankw[sw];
    const uint32_t lane_bit = 1u << sl;
    const size_t tile_base = size_t(tile) * TILE;
    // Items of this sub-wave's chunk that exist (the last tile may be partial).
    const uint32_t sub_valid =
        n > sub_base ? static_cast<uint32_t>(min<size_t>(n - sub_base, SUB_ITEMS)) : 0u;

    ValReg val[ITEMS];
    if constexpr (PAIRS) {
      // Issued now, consumed after the key scatter.
#pragma unroll
      for (int j = 0; j < ITEMS; ++j)
        val[j] = vals_in[min(sub_base + size_t(j) * 32 + sl, last_item)];
    }

    // Stable rank within the sub-wave. For each item the lanes OR their lane
    // bit into the low half of their digit's ranking word; reading the word
    // back gives the peer set and the sub-wave's running count for that digit
    // in one load, and rank = count + peers below this lane. The lowest peer
    // then writes count + peers with an empty mask, which both advances the
    // count and clears the mask for the next item. LDS operations of one wave
    // execute in order, so no barrier is needed between the steps.
    uint32_t rank[ITEMS];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const uint32_t d =
          uint32_t(j) * 32 + sl < sub_valid ? Ops::digit(key[j], bit, mask) : DUMMY;
      atomicOr(reinterpret_cast<uint32_t *>(&srank[d]), lane_bit);
      __builtin_amdgcn_wave_barrier();
      const uint64_t word = srank[d];
      const uint32_t peers = static_cast<uint32_t>(word);
      const uint32_t base = static_cast<uint32_t>(word >> 32);
      const uint32_t below = static_cast<uint32_t>(__popc(peers & (lane_bit - 1u)));
      rank[j] = base + below;
      // Keep one register per item (not base and below separately).
      asm volatile("" : "+v"(rank[j]));
      __builtin_amdgcn_wave_barrier();
      if (below == 0)
        srank[d] = static_cast<uint64_t>(base + static_cast<uint32_t>(__popc(peers))) << 32;
      __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
#if RCCL_RADIX_PERSISTENT && RCCL_RADIX_CLAIM_POINT == 1
    if (tid == CLAIM) claimed = add_agent(tile_counter, 1u);
#endif

    // Per digit: exclusive prefix over waves and tile total; publish the
    // aggregate and start the look-back loads at once.
    uint32_t count = 0;
    uint32_t tile_inc = 0;
    const uint32_t group = tile / GROUP;
    const int gfirst = static_cast<int>(group) * GROUP;
    Desc lb[LOOKBACK];
    Desc gi[GWIN];
    uint32_t ga[GWIN];
    if (tid < BINS) {
#pragma unroll
      for (int w = 0; w < SUBS; ++w) {
        const uint32_t c = static_cast<uint32_t>(rankw[w][tid] >> 32);
        hist[w][tid] = static_cast<uint16_t>(count);
        count += c;
      }
      store_agent(&lbuf.tile[size_t(tile) * BINS + tid],
                  static_cast<Desc>((tile == 0 ? DI::INCL : DI::AGG) | Desc(count)));
      add_agent(&lbuf.gagg[size_t(group) * BINS + tid], (1u << GAGG_SHIFT) | count);
      // Issue both first windows now: in-group predecessors (newest first)
      // and the groups before this one.
      // Window loads are clamped to valid slots; slots outside the window
      // are masked when the window is consumed, so the loads stay in flight
      // until then.
#pragma unroll
      for (int w = 0; w < LOOKBACK; ++w)
        lb[w] = load_agent(&lbuf.tile[size_t(max(static_cast<int>(tile) - 1 - w, 0)) * BINS + tid]);
#pragma unroll
      for (int w = 0; w < GWIN; ++w) {
        const size_t g = size_t(max(static_cast<int>(group) - 1 - w, 0));
        gi[w] = load_agent(&lbuf.ginc[g * BINS + tid]);
        ga[w] = load_agent(&lbuf.gagg[g * BINS + tid]);
      }
      tile_inc = wave_inclusive_sum(count, lane);
      if (lane == 63) wave_sum[wave] = tile_inc;
    }
    __syncthreads();
    uint32_t tile_start = 0;
    if (tid < BINS) {
      tile_start = tile_inc - count;
      for (uint32_t w = 0; w < wave; ++w) tile_start += wave_sum[w];
#pragma unroll
      for (int w = 0; w < SUBS; ++w) hist[w][tid] = static_cast<uint16_t>(hist[w][tid] + tile_start);
    }
    if (tid < SUBS) hist[tid][DUMMY] = TILE;  // dummy items stage into the spare slot
#if RCCL_RADIX_PERSISTENT && RCCL_RADIX_CLAIM_POINT < 2
    if (tid == CLAIM) s_tile = claimed;
#endif
    __syncthreads();
#if !RCCL_RADIX_PERSISTENT
    const uint32_t next = num_tiles;
#elif RCCL_RADIX_CLAIM_POINT < 2
    const uint32_t next = s_tile;
#else
    if (tid == CLAIM) claimed = add_agent(tile_counter, 1u);
#endif

    // Stage keys in digit order. The empty asm statements stop the compiler
    // from keeping per-item digit addresses alive from the ranking loop
    // (recomputing them is cheaper than the registers).
    uint32_t slane = sl;
    asm volatile("" : "+v"(slane));
    const uint16_t *shist = hist[sw];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) asm volatile("" : "+v"(key[j]));
    // In batches: the batch's offset reads are in flight together before its
    // staging writes.
#pragma unroll
    for (int j0 = 0; j0 < ITEMS; j0 += BATCH) {
      uint32_t base[BATCH];
#pragma unroll
      for (int b = 0; b < BATCH && j0 + b < ITEMS; ++b) {
        const int j = j0 + b;
        const uint32_t d =
            uint32_t(j) * 32 + slane < sub_valid ? Ops::digit(key[j], bit, mask) : DUMMY;
        base[b] = shist[d];
      }
#pragma unroll
      for (int b = 0; b < BATCH && j0 + b < ITEMS; ++b) {
        const int j = j0 + b;
        rank[j] = min(rank[j] + base[b], uint32_t(TILE));
        stage_keys[rank[j]] = key[j];
      }
    }

    // Prefetch the next tile's keys into the key registers (the current keys
    // live in LDS now); they land while this tile's look-back and scatter
    // run. No branch around the loads: past the last tile every element is
    // masked off, and a fixed count of loads lets the look-back wait for its
    // own window loads only.
#if RCCL_RADIX_PERSISTENT && RCCL_RADIX_CLAIM_POINT < 2
    const size_t next_sub_base = size_t(next) * TILE + size_t(sw) * SUB_ITEMS;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j)
      key[j] = keys_in[min(next_sub_base + size_t(j) * 32 + sl, last_item)];
#endif

    // Two-level decoupled look-back, one thread per digit, consuming the
    // windows issued above newest first. In-group predecessors are summed
    // tile by tile until an inclusive prefix or the group start; earlier
    // groups are then summed whole (complete aggregates) until a group's
    // inclusive prefix. A slot that is not yet published is polled again.
    if (tid < BINS) {
      Desc excl = 0;
      bool done = tile == 0;
      // Window slot w holds tile t - w; slots before the group are boundaries.
      int t = static_cast<int>(tile) - 1;
      auto eat_tiles = [&]() {
        int consumed = 0;
        bool stop = false;
#pragma unroll
        for (int w = 0; w < LOOKBACK; ++w) {
          if (!done && !stop) {
            const Desc v = t - w >= gfirst ? lb[w] : DI::BOUNDARY;
            const Desc flag = v >> DI::SHIFT;
            if (flag == 0 || flag == (DI::BOUNDARY >> DI::SHIFT)) {
              stop = true;
            } else {
              excl += v & DI::MASK;
              ++consumed;
              done = flag == (DI::INCL >> DI::SHIFT);
            }
          }
        }
        t -= consumed;
        return consumed;
      };
      // Group slot w holds group g - w; slots before group 0 read as an
      // inclusive zero.
      int g = static_cast<int>(group) - 1;
      auto eat_groups = [&]() {
        int consumed = 0;
        bool blocked = false;
#pragma unroll
        for (int w = 0; w < GWIN; ++w) {
          if (!done && !blocked) {
            const bool real = g - w >= 0;
            const Desc vi = real ? gi[w] : DI::INCL;
            const uint32_t va = real ? ga[w] : 0u;
            if ((vi >> DI::SHIFT) == (DI::INCL >> DI::SHIFT)) {
              excl += vi & DI::MASK;
              done = true;
            } else if ((va >> GAGG_SHIFT) == uint32_t(GROUP)) {
              excl += va & GAGG_MASK;  // earlier groups are always full
              ++consumed;
            } else {
              blocked = true;
            }
          }
        }
        g -= consumed;
        return consumed;
      };
      // The first windows were issued before the staging; they are consumed
      // outside the polling loops so that waiting for them does not wait for
      // the prefetch issued after them.
      if (!done) {
        int c = eat_tiles();
        while (!done && t >= gfirst) {
          if (c == 0) __builtin_amdgcn_s_sleep(1);
#pragma unroll
          for (int w = 0; w < LOOKBACK; ++w)
            lb[w] = load_agent(&lbuf.tile[size_t(max(t - w, 0)) * BINS + tid]);
          c = eat_tiles();
        }
      }
      if (!done) {
        int c = eat_groups();
        while (!done) {
          if (c == 0) __builtin_amdgcn_s_sleep(1);
#pragma unroll
          for (int w = 0; w < GWIN; ++w) {
            const size_t gg = size_t(max(g - w, 0));
            gi[w] = load_agent(&lbuf.ginc[gg * BINS + tid]);
            ga[w] = load_agent(&lbuf.gagg[gg * BINS + tid]);
          }
          c = eat_groups();
        }
      }
      const Desc incl = static_cast<Desc>(DI::INCL | (excl + Desc(count)));
      if (tile > 0) store_agent(&lbuf.tile[size_t(tile) * BINS + tid], incl);
      const uint32_t glast = min(uint32_t(gfirst + GROUP), num_tiles) - 1u;
      if (tile == glast) store_agent(&lbuf.ginc[size_t(group) * BINS + tid], incl);
      digit_off[tid] = bin_start + static_cast<uint32_t>(excl) - tile_start;
    }
#if RCCL_RADIX_PERSISTENT && RCCL_RADIX_CLAIM_POINT == 2
    if (tid == CLAIM) s_tile = claimed;
#endif
    __syncthreads();
#if RCCL_RADIX_PERSISTENT && RCCL_RADIX_CLAIM_POINT == 2
    const uint32_t next = s_tile;
    const size_t next_sub_base = size_t(next) * TILE + size_t(sw) * SUB_ITEMS;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j)
      key[j] = keys_in[min(next_sub_base + size_t(j) * 32 + sl, last_item)];
#endif

    // Coalesced scatter: consecutive staged keys of one digit go to
    // consecutive output positions.
    const uint32_t valid_count = static_cast<uint32_t>(min<size_t>(TILE, n - tile_base));
    // Positions are exact when the bins match the keys; the clamp only keeps
    // a caller that changes the keys mid-sort from writing out of bounds.
    const uint32_t last = static_cast<uint32_t>(n - 1);
    // In batches: the batch's staged keys are read together, then their
    // digits' offsets together, then stored; only the stores are predicated.
    uint32_t dst[PAIRS ? ITEMS : 1];
#pragma unroll
    for (int k0 = 0; k0 < ITEMS; k0 += BATCH) {
      Bits kk[BATCH];
      uint32_t off[BATCH];
#pragma unroll
      for (int b = 0; b < BATCH && k0 + b < ITEMS; ++b)
        kk[b] = stage_keys[uint32_t(k0 + b) * THREADS + tid];
#pragma unroll
      for (int b = 0; b < BATCH && k0 + b < ITEMS; ++b)
        off[b] = digit_off[Ops::digit(kk[b], bit, mask)];
#pragma unroll
      for (int b = 0; b < BATCH && k0 + b < ITEMS; ++b) {
        const uint32_t i = uint32_t(k0 + b) * THREADS + tid;
        const uint32_t p = min(off[b] + i, last);
        if (i < valid_count) keys_out[p] = kk[b];
        if constexpr (PAIRS) dst[k0 + b] = p;
      }
    }
    if constexpr (PAIRS) {
      __syncthreads();
      Val *stage_vals = reinterpret_cast<Val *>(stage_raw);
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) stage_vals[rank[j]] = val[j];
      __syncthreads();
#pragma unroll
      for (int k = 0; k < ITEMS; ++k) {
        const uint32_t i = uint32_t(k) * THREADS + tid;
        if (i < valid_count) vals_out[dst[k]] = stage_vals[i];
      }
    }
    if (tid < BINS && lbuf_next.tile) {
      lbuf_next.tile[size_t(tile) * BINS + tid] = 0;
      if (static_cast<int>(tile) == gfirst) {
        lbuf_next.ginc[size_t(group) * BINS + tid] = 0;
        lbuf_next.gagg[size_t(group) * BINS + tid] = 0;
      }
    }
    __syncthreads();

    if (next >= num_tiles) break;
#if RCCL_RADIX_PERSISTENT
    tile = next;
    sub_base = next_sub_base;
#endif
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

// Largest item count the control words support: 30-bit look-back counts
// switch to 62-bit descriptors at 2^30; positions are 32-bit.
constexpr uint64_t MAX_ITEMS = 0xffffffffull;

struct Layout {
  size_t tiles = 0;
  size_t groups = 0;
  size_t desc_bytes = 4;
  size_t bins = 0, counters = 0;
  size_t lb[2] = {0, 0};  // look-back buffers: tile descriptors, group prefixes, aggregates
  size_t lb_ginc = 0, lb_gagg = 0, lb_bytes = 0;  // offsets/size within one buffer
  size_t total = 0;
};

Layout layout(size_t key_bytes, size_t value_bytes, size_t n);

struct SortArgs {
  void *keys[2];
  void *vals[2];
  size_t n;
  int cur;  // index of the buffer holding the input
  uint32_t begin_bit, end_bit;
  unsigned char *ws;
  hipStream_t stream;
};

template <class Bits, class Val, class Ops, class Desc>
rccl_hip_status run_passes(SortArgs &a, const Layout &l, uint32_t passes) {
  constexpr size_t VBYTES = std::is_same<Val, NoValue>::value ? 0 : sizeof(Val);
  constexpr int ITEMS = items_for(sizeof(Bits), VBYTES);
  constexpr int THREADS = threads_for(VBYTES);
  uint32_t *bins = reinterpret_cast<uint32_t *>(a.ws + l.bins);
  uint32_t *counters = reinterpret_cast<uint32_t *>(a.ws + l.counters);
  LookbackBuf<Desc> lb[2];
  for (int b = 0; b < 2; ++b) {
    unsigned char *base = a.ws + l.lb[b];
    lb[b].tile = reinterpret_cast<Desc *>(base);
    lb[b].ginc = reinterpret_cast<Desc *>(base + l.lb_ginc);
    lb[b].gagg = reinterpret_cast<uint32_t *>(base + l.lb_gagg);
  }

  {
    KernelTimer t("radix_init", a.stream, 0);
    init_kernel<<<1, 256, 0, a.stream>>>(bins, counters, passes);
  }
  RCCL_HIP_TRY(check_launch("radix init"));

  const size_t chunk = size_t(HIST_THREADS) * HIST_ITEMS;
  const size_t hist_blocks = std::max<size_t>(1, std::min<size_t>((a.n + chunk - 1) / chunk, 2048));
  const size_t zero_words = l.lb_bytes / sizeof(uint32_t);
  {
    KernelTimer t("radix_histogram", a.stream, a.n);
    histogram_kernel<Bits, Ops><<<dim3(static_cast<uint32_t>(hist_blocks)), HIST_THREADS, 0,
                                  a.stream>>>(
        static_cast<const Bits *>(a.keys[a.cur]), a.n, bins, a.begin_bit, a.end_bit, passes,
        reinterpret_cast<uint32_t *>(a.ws + l.lb[0]), zero_words);
  }
  RCCL_HIP_TRY(check_launch("radix histogram"));
  {
    KernelTimer t("radix_bins_scan", a.stream, passes * BINS);
    bins_scan_kernel<<<1, BINS, 0, a.stream>>>(bins, passes);
  }
  RCCL_HIP_TRY(check_launch("radix bins scan"));

  // Persistent grid: as many blocks as fit on the device at once, but never
  // more than there are tiles.
  static int blocks_per_cu = 0;
  static int cus = 0;
  if (blocks_per_cu == 0) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess)
      err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err == hipSuccess)
      err = hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &blocks_per_cu, onesweep_kernel<Bits, Val, Ops, ITEMS, Desc, THREADS>, THREADS, 0);
    if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_DRIVER, "radix occupancy", err);
    if (blocks_per_cu < 1 || cus < 1)
      return set_error(RCCL_HIP_ERROR_LAUNCH, "radix onesweep does not fit on the device");
  }
  const uint32_t grid = static_cast<uint32_t>(
      RCCL_RADIX_PERSISTENT ? std::min<size_t>(l.tiles, size_t(blocks_per_cu) * size_t(cus))
                            : l.tiles);

  for (uint32_t p = 0; p < passes; ++p) {
    const uint32_t bit = a.begin_bit + 8u * p;
    const uint32_t width = std::min(8u, a.end_bit - bit);
    const uint32_t mask = (1u << width) - 1u;
    const int in = a.cur, out = 1 - a.cur;
    KernelTimer t("radix_onesweep", a.stream, a.n);
    onesweep_kernel<Bits, Val, Ops, ITEMS, Desc, THREADS><<<dim3(grid), THREADS, 0, a.stream>>>(
        static_cast<const Bits *>(a.keys[in]), static_cast<Bits *>(a.keys[out]),
        static_cast<const Val *>(a.vals[in]), static_cast<Val *>(a.vals[out]), a.n,
        static_cast<uint32_t>(l.tiles), bins + size_t(p) * BINS, lb[p & 1],
        p + 1 < passes ? lb[(p + 1) & 1] : LookbackBuf<Desc>{nullptr, nullptr, nullptr},
        counters + p, bit, mask);
    RCCL_HIP_TRY(check_launch("radix onesweep"));
    a.cur = out;
  }
  return ok();
}

template <class Bits, class Ops>
rccl_hip_status run_values(SortArgs &a, size_t value_bytes, const Layout &l, uint32_t passes) {
  const bool wide = l.desc_bytes == 8;
  switch (value_bytes) {
  case 0:
    return wide ? run_passes<Bits, NoValue, Ops, uint64_t>(a, l, passes)
                : run_passes<Bits, NoValue, Ops, uint32_t>(a, l, passes);
  case 1:
    return wide ? run_passes<Bits, uint8_t, Ops, uint64_t>(a, l, passes)
                : run_passes<Bits, uint8_t, Ops, uint32_t>(a, l, passes);
  case 2:
    return wide ? run_passes<Bits, uint16_t, Ops, uint64_t>(a, l, passes)
                : run_passes<Bits, uint16_t, Ops, uint32_t>(a, l, passes);
  case 4:
    return wide ? run_passes<Bits, uint32_t, Ops, uint64_t>(a, l, passes)
                : run_passes<Bits, uint32_t, Ops, uint32_t>(a, l, passes);
  case 8:
    return wide ? run_passes<Bits, uint64_t, Ops, uint64_t>(a, l, passes)
                : run_passes<Bits, uint64_t, Ops, uint32_t>(a, l, passes);
  case 16:
    return wide ? run_passes<Bits, Value16, Ops, uint64_t>(a, l, passes)
                : run_passes<Bits, Value16, Ops, uint32_t>(a, l, passes);
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix value bytes");
}

// One entry per key kind, each compiled in its own translation unit.
#define RCCL_RADIX_DECLARE_KIND(NAME)                                                   \
  rccl_hip_status run_##NAME(SortArgs &a, size_t value_bytes, const Layout &l,         \
                             uint32_t passes, bool descending);
RCCL_RADIX_DECLARE_KIND(u32)
RCCL_RADIX_DECLARE_KIND(i32)
RCCL_RADIX_DECLARE_KIND(f32)
RCCL_RADIX_DECLARE_KIND(u64)
RCCL_RADIX_DECLARE_KIND(i64)
RCCL_RADIX_DECLARE_KIND(f64)
#undef RCCL_RADIX_DECLARE_KIND

#define RCCL_RADIX_DEFINE_KIND(NAME, BITS, CLASS)                                       \
  rccl_hip_status run_##NAME(SortArgs &a, size_t value_bytes, const Layout &l,         \
                             uint32_t passes, bool descending) {                       \
    return descending                                                                  \
               ? run_values<BITS, KeyOps<BITS, KeyClass::CLASS, true>>(a, value_bytes, l, \
                                                                       passes)         \
               : run_values<BITS, KeyOps<BITS, KeyClass::CLASS, false>>(a, value_bytes, \
                                                                        l, passes);    \
  }

} // namespace radix
} // namespace rccl_hip
