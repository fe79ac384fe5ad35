// DeviceRadixSort kernels for gfx950: onesweep LSD radix sort, 8-bit digits.
//
// Reference behaviour: rccl-cub/src/radix.rs:364-876 (validation and pass
// control) and rccl-cub/src/ordering_backend/radix.rs (device agents). The
// kernels are an independent wave64 design:
//   init        zero the per-pass bins (one tiny block)
//   histogram   one read of all keys builds every pass's 256-bin histogram in
//               LDS (per-lane counter columns) and adds them to the bins;
//               it also zeroes look-back buffer 0
//   onesweep    one launch per pass, one tile per block (XCD-aware tile
//               order); per-wave LDS digit counts, ranking by lane-ordered
//               returning LDS atomics, a windowed two-level decoupled
//               look-back on agent-scope atomics, and a scatter through LDS
//               so HBM writes coalesce
#pragma once

#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "radix_plan.hpp"

namespace rccl_hip {
namespace radix {

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

  // The order-preserving bijection, before the collapse. Onesweep passes keep
  // keys in this form between passes: the first converts its raw input
  // (image), the last its output back (raw), and every digit in between
  // needs only the collapse (image_digit): about half the ALU work per digit
  // for float keys.
  __device__ static __forceinline__ Bits image(Bits raw) {
    Bits x = raw;
    if constexpr (KC == KeyClass::Signed) x ^= SIGN;
    if constexpr (KC == KeyClass::Float)
      x ^= static_cast<Bits>(static_cast<SBits>(raw) >> (NBITS - 1)) | SIGN;
    if constexpr (DESC) x = ~x;
    return x;
  }
  __device__ static __forceinline__ Bits raw(Bits x) {
    if constexpr (DESC) x = ~x;
    if constexpr (KC == KeyClass::Signed) x ^= SIGN;
    // A set top bit marks a non-negative float (sign flipped), a clear one a
    // negative float (all bits inverted).
    if constexpr (KC == KeyClass::Float)
      x ^= static_cast<Bits>(~(static_cast<SBits>(x) >> (NBITS - 1))) | SIGN;
    return x;
  }
  __device__ static __forceinline__ Bits collapse(Bits x) {
    if constexpr (KC == KeyClass::Float) return x == SIGN - 1 ? SIGN : x;
    else return x;
  }

  __device__ static __forceinline__ Bits digit_source(Bits raw) { return collapse(image(raw)); }

  __device__ static __forceinline__ uint32_t digit(Bits raw, uint32_t bit, uint32_t mask) {
    return static_cast<uint32_t>(digit_source(raw) >> bit) & mask;
  }
  __device__ static __forceinline__ uint32_t image_digit(Bits y, uint32_t bit, uint32_t mask) {
    return static_cast<uint32_t>(collapse(y) >> bit) & mask;
  }
};

// Key loads of a keys-only onesweep are non-temporal: they are read once, and
// leaving L2 to the scattered writes (whose partial lines merge there) and the
// look-back measured faster. Pair sorts and stores keep the default policy:
// non-temporal value loads and stores measured slower.
template <bool NT, class T>
__device__ __forceinline__ T stream_load(const T *p) {
  if constexpr (NT && std::is_arithmetic<T>::value)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}

// The histogram's key loads are non-temporal too (measured faster).
#ifndef RCCL_RADIX_NT_PAIR_KEYS
#define RCCL_RADIX_NT_PAIR_KEYS 0
#endif
#ifndef RCCL_RADIX_HIST_NT
#define RCCL_RADIX_HIST_NT 1
#endif

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
// its own descriptor (its count; tile 0's is inclusive), every tile adds
// (1 << GAGG_SHIFT) | count to its group's per-digit aggregate word, which is
// therefore complete exactly when its top byte equals the group size. Only
// the group's last tile publishes an inclusive prefix, through the group
// (an inclusive descriptor per tile measured no faster: look-backs rarely
// found one, and its stores added 1 KB of writes per tile). A look-back sums
// in-group predecessors tile by tile and earlier groups whole, so the prefix
// chain advances a group per step instead of a tile.
constexpr int GAGG_SHIFT = 24;
constexpr uint32_t GAGG_MASK = (1u << GAGG_SHIFT) - 1;
template <class Desc> struct LookbackBuf {
  Desc *tile;        // tiles x BINS descriptors
  Desc *ginc;        // groups x BINS inclusive prefixes through each group
  uint32_t *gagg;    // groups x BINS packed (tiles counted, count)
  uint32_t *ticket;  // XCDS tile-ticket counters of the pass
};

// ---------------------------------------------------------------------------
// init: zero the bins. (Internal linkage: every translation unit that
// launches it carries its own copy.)
// ---------------------------------------------------------------------------
namespace {
__global__ void __launch_bounds__(256) init_kernel(uint32_t *bins, uint32_t passes) {
  for (uint32_t i = threadIdx.x; i < passes * BINS; i += 256) bins[i] = 0;
}
} // namespace

// ---------------------------------------------------------------------------
// histogram: every pass's digit counts from one read of the keys.
// ---------------------------------------------------------------------------
// Per-lane counter columns: lane l of every wave counts into column
// l % cols of its digit's row, so the lanes of one LDS atomic hit at most a
// few banks' worth of conflicts instead of random ones (random digits into one
// shared row per wave cost about twice as many LDS cycles per atomic; for
// 8-byte keys the LDS was busy 69% of the time, half of it in conflicts).
// All passes' rows take 64 KB (16 columns for 4-byte keys, 8 for 8-byte
// keys): two blocks per CU, grid-striding over chunks.
#ifndef RCCL_RADIX_HIST_THREADS
#define RCCL_RADIX_HIST_THREADS 512
#endif
#ifndef RCCL_RADIX_HIST_ITEMS
#define RCCL_RADIX_HIST_ITEMS 16
#endif
#ifndef RCCL_RADIX_HIST_COLS
#define RCCL_RADIX_HIST_COLS 16
#endif
constexpr int HIST_THREADS = RCCL_RADIX_HIST_THREADS;
constexpr int HIST_ITEMS = RCCL_RADIX_HIST_ITEMS;
constexpr int HIST_COLS_4B = RCCL_RADIX_HIST_COLS;

template <class Bits>
constexpr int hist_cols() {
  return HIST_COLS_4B * 4 / int(sizeof(Bits));
}

// 8-byte keys are loaded 16 bytes (two keys) per lane and instruction (the
// histogram counts keys in any order): C2's u64 histogram 130 -> 120 us at
// 2^26. 4-byte keys keep one key per lane: four per load measured 3-5 us
// slower at 2^28 u32. (16-bit counters packed two per word, twice the
// columns in the same LDS, measured slower for every key width: 2^28 u32
// 212 -> 272 us.)
#ifndef RCCL_RADIX_HIST_VLOAD_8B
#define RCCL_RADIX_HIST_VLOAD_8B 1
#endif
typedef unsigned int hist_v4u __attribute__((ext_vector_type(4)));

template <class Bits, class Ops>
__global__ void __launch_bounds__(HIST_THREADS)
histogram_kernel(const Bits *__restrict__ keys, size_t n, uint32_t *__restrict__ bins,
                 uint32_t begin_bit, uint32_t end_bit, uint32_t passes,
                 uint32_t *__restrict__ zero_words, size_t zero_count) {
  constexpr int PMAX = int(sizeof(Bits));  // 8-bit passes
  constexpr bool VLOAD = sizeof(Bits) == 8 && RCCL_RADIX_HIST_VLOAD_8B;
  constexpr int COLS = hist_cols<Bits>();
  constexpr int WORDS = PMAX * BINS * COLS;
  constexpr int VEC = VLOAD ? 16 / int(sizeof(Bits)) : 1;  // keys per load
  constexpr int LOADS = HIST_ITEMS / VEC;
  __shared__ uint32_t hist[WORDS];  // [pass][digit][column]
  const uint32_t tid = threadIdx.x;
  for (uint32_t i = tid; i < WORDS; i += HIST_THREADS) hist[i] = 0;
  for (size_t i = size_t(blockIdx.x) * HIST_THREADS + tid; i < zero_count;
       i += size_t(gridDim.x) * HIST_THREADS)
    zero_words[i] = 0;
  __syncthreads();

  const uint32_t col = tid % COLS;
  uint32_t shift[PMAX], dmask[PMAX];
#pragma unroll
  for (int p = 0; p < PMAX; ++p) {
    const uint32_t bit = begin_bit + 8u * p;
    shift[p] = bit;
    dmask[p] = uint32_t(p) < passes ? (1u << min(8u, end_bit - bit)) - 1u : 0u;
  }
  auto count = [&](Bits key) {
    const Bits s = Ops::digit_source(key);
#pragma unroll
    for (int p = 0; p < PMAX; ++p) {
      if (uint32_t(p) >= passes) break;
      const uint32_t d = static_cast<uint32_t>(s >> shift[p]) & dmask[p];
      __hip_atomic_fetch_add(&hist[(uint32_t(p) * BINS + d) * COLS + col], 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  // All 8-bit digits of the key (the usual full bit range).
  const bool all_digits = begin_bit == 0 && passes == uint32_t(PMAX) && end_bit == 8u * PMAX;
  auto count_all = [&](Bits key) {
    const Bits s = Ops::digit_source(key);
#pragma unroll
    for (int p = 0; p < PMAX; ++p) {
      const uint32_t d = static_cast<uint32_t>(s >> (8 * p)) & 0xFFu;
      __hip_atomic_fetch_add(&hist[(uint32_t(p) * BINS + d) * COLS + col], 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  // With vector loads, the keys before the first 16-byte boundary and after
  // the last whole vector are counted by block 0, one per thread.
  const size_t head = VLOAD ? min<size_t>(
      ((16u - (reinterpret_cast<uintptr_t>(keys) & 15u)) & 15u) / sizeof(Bits), n) : 0;
  const size_t nvec = (n - head) / VEC;
  const size_t tail = head + nvec * VEC;
  if (VLOAD && blockIdx.x == 0) {
    if (tid < head) count(keys[tid]);
    else if (tid - head < n - tail) count(keys[tail + (tid - head)]);
  }
  using LoadT = typename std::conditional<VLOAD, hist_v4u, Bits>::type;
  const LoadT *src = reinterpret_cast<const LoadT *>(keys + head);
  // The next chunk's keys are loaded before the current chunk is counted, so
  // the load latency hides behind the counting.
  constexpr size_t CHUNK = size_t(HIST_THREADS) * LOADS;  // loads per chunk
  const size_t stride = size_t(gridDim.x) * CHUNK;
  LoadT next[LOADS];
  auto load_chunk = [&](size_t base) {
    const uint32_t avail = static_cast<uint32_t>(min<size_t>(nvec - base, CHUNK));
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const LoadT *ptr = &src[base + min(uint32_t(j) * HIST_THREADS + tid, avail - 1u)];
      if constexpr (VLOAD) next[j] = __builtin_nontemporal_load(ptr);
      else next[j] = stream_load<RCCL_RADIX_HIST_NT>(ptr);
    }
  };
  if (size_t(blockIdx.x) * CHUNK < nvec) load_chunk(size_t(blockIdx.x) * CHUNK);
  for (size_t base = size_t(blockIdx.x) * CHUNK; base < nvec; base += stride) {
    const uint32_t avail = static_cast<uint32_t>(min<size_t>(nvec - base, CHUNK));
    LoadT k[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) k[j] = next[j];
    if (base + stride < nvec) load_chunk(base + stride);
    if (all_digits && avail == uint32_t(CHUNK)) {
      // Every pass of the key and a whole chunk (all but a block's last):
      // constant digit positions, no per-key or per-pass tests.
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        Bits kv[VEC];
        __builtin_memcpy(kv, &k[j], sizeof(LoadT));
#pragma unroll
        for (int e = 0; e < VEC; ++e) count_all(kv[e]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        if (uint32_t(j) * HIST_THREADS + tid >= avail) continue;
        Bits kv[VEC];
        __builtin_memcpy(kv, &k[j], sizeof(LoadT));
#pragma unroll
        for (int e = 0; e < VEC; ++e) count(kv[e]);
      }
    }
  }
  __syncthreads();
  // Row sums. Thread e reads its row's columns in rotated order, so the
  // threads of a wave read distinct banks.
  for (uint32_t e = tid; e < passes * BINS; e += HIST_THREADS) {
    const uint32_t *row = &hist[e * COLS];
    uint32_t sum = 0;
#pragma unroll
    for (uint32_t c = 0; c < uint32_t(COLS); ++c) sum += row[(c + e) % COLS];
    if (sum) add_agent(&bins[e], sum);
  }
}


// Skew word of a pass (bins_scan_kernel): 1 when the pass's most frequent
// digit holds at least 1 / RCCL_RADIX_HOT_DIV of the keys, else 0.
#ifndef RCCL_RADIX_HOT_DIV
#define RCCL_RADIX_HOT_DIV 16
#endif

// Turn every pass's digit counts into exclusive offsets (the first output
// position of each digit), once, so the onesweep blocks read them instead of
// each scanning the bins. One block of BINS threads; MAXP bounds the passes
// (the key's bytes). Every pass's counts are loaded at once and scanned with
// one barrier. It also writes each pass's skew word and, with a plan, marks
// the trivial passes (a digit counting all n keys) and writes the pass plan.
// A separate launch: folding it into the histogram's last block (a
// device-scope completion counter) measured slower at 2^28 (229 against 216
// us), as the agent-scope release writes back every block's dirty L2 lines.
// (Internal linkage, like init_kernel.)
namespace {
template <int MAXP>
__global__ void __launch_bounds__(BINS)
bins_scan_kernel(uint32_t *bins, uint32_t passes, uint32_t n, PassPlan *plan,
                 uint32_t plan_flags, uint32_t *skew) {
  constexpr int WAVES = BINS / 64;
  __shared__ uint32_t s_wave[MAXP][WAVES];  // per wave: its digits' total
  __shared__ uint32_t s_top[MAXP][WAVES];   // per wave: its largest digit count
  __shared__ uint32_t s_full[WAVES];        // per wave: passes with a digit of n keys
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  uint32_t c[MAXP], inc[MAXP];
#pragma unroll
  for (int p = 0; p < MAXP; ++p) c[p] = uint32_t(p) < passes ? bins[p * BINS + tid] : 0u;
  uint32_t full = 0;
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    inc[p] = wave_inclusive_sum(c[p], lane);
    uint32_t top = c[p];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
      top = max(top, static_cast<uint32_t>(__shfl_xor(static_cast<int>(top), o, 64)));
    if (__ballot(c[p] == n) != 0) full |= 1u << p;
    if (lane == 63) s_wave[p][wave] = inc[p];
    if (lane == 0) s_top[p][wave] = top;
  }
  if (lane == 0) s_full[wave] = full;
  __syncthreads();
#pragma unroll
  for (int p = 0; p < MAXP; ++p) {
    if (uint32_t(p) >= passes) break;
    uint32_t excl = inc[p] - c[p];
#pragma unroll
    for (int w = 0; w < WAVES; ++w)
      if (uint32_t(w) < wave) excl += s_wave[p][w];
    bins[p * BINS + tid] = excl;
  }
  if (skew && tid < passes) {
    uint32_t top = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) top = max(top, s_top[tid][w]);
    skew[tid] = uint64_t(top) * RCCL_RADIX_HOT_DIV >= uint64_t(n) ? 1u : 0u;
  }
  if (plan && tid == 0) {
    uint32_t trivial = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) trivial |= s_full[w];
    assign_plan(static_cast<int>(passes), trivial, plan_flags, plan);
  }
}
} // namespace

// ---------------------------------------------------------------------------
// onesweep: one stable counting-sort pass, one tile per block.
//
// Per tile: load the keys (wave-contiguous, lane-striped), count digits into
// per-wave LDS counters, publish the tile's digit counts for the look-back,
// turn the counters into tile positions, rank every key, stage the tile in
// digit order, finish the look-back and scatter so that each digit's keys
// leave in contiguous runs.
//
// Ranking, two modes (both stable: equal digits get positions in (wave,
// item, lane) order, which is source order):
//  - lane-ordered atomics: one returning LDS atomic per key on its wave's
//    digit counter. This relies on a property of the gfx950 LDS, checked
//    once per device at load time: lanes of one atomic that hit the same
//    address are served in ascending lane order;
//  - match-any: per item, the lanes holding the same digit are found with
//    one ballot per digit bit; the lowest of them adds the group's size with
//    one atomic, and each lane's position is the returned base (broadcast by
//    ds_bpermute) plus its count of peers in lower lanes (mbcnt). It makes no
//    assumption about the LDS, costs more ALU work, and is used where the
//    lane-order check fails (or when selected at run time).
// The digit counting before the ranking is order-free: plain LDS atomics in
// both modes.
// ---------------------------------------------------------------------------

enum class Rank : int { LaneAtomic = 0, MatchAny = 1 };

// Items per batch of match-any ranking.
#ifndef RCCL_RADIX_MATCH_BATCH
#define RCCL_RADIX_MATCH_BATCH 8
#endif
// Skewed passes (lane-ordered ranking only): 1 takes each key's rank from
// the counting atomic (see onesweep_tile), 0 ranks them like uniform passes.
#ifndef RCCL_RADIX_SKEW_RANKING
#define RCCL_RADIX_SKEW_RANKING 1
#endif
// Lanes of one item sharing lane 0's digit that make a wave take the skewed
// ranking in a pass that is not skewed as a whole.
#ifndef RCCL_RADIX_SKEW_LANES
#define RCCL_RADIX_SKEW_LANES 8
#endif
// Items per batch of counter reads in the skewed ranking.
#ifndef RCCL_RADIX_RANK_BATCH
#define RCCL_RADIX_RANK_BATCH 8
#endif

// Tile shapes with the skewed ranking: not those whose keys and values alone
// take more than 48 registers per thread (u32 keys + 4-byte values at 28
// items, 8-byte keys + 8-byte values). Their onesweep already fills the
// register budget, and the skewed branch would make it spill.
template <class Bits, class Val, int ITEMS>
constexpr bool skew_ranking() {
  constexpr size_t VREGS = std::is_same<Val, NoValue>::value ? 0 : (sizeof(Val) + 3) / 4;
  return RCCL_RADIX_SKEW_RANKING &&
         size_t(ITEMS) * ((sizeof(Bits) + 3) / 4 + VREGS) <= 48;
}

// s_waitcnt vmcnt(N): wait until at most N vector memory operations of this
// wave are outstanding (gfx9 encoding: vmcnt bits [3:0] and [15:14]; expcnt
// and lgkmcnt left at their no-wait maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Tile processed by a block, in XCD order (xcd_order_tile): the cache lines
// that neighbouring tiles both write at digit-run boundaries are merged in
// their shared L2 instead of reaching HBM as two partial writes. This is used
// where the load-time probe saw the blocks of a launch land on the XCDs
// round-robin (nx == XCDS); elsewhere a block claims its tile from an atomic
// ticket (tiles in claim order: a tile is only claimed by a started block, so
// the lowest unfinished tile's look-back never waits on an unstarted one).
__device__ __forceinline__ uint32_t xcd_tile(uint32_t block) {
  return xcd_order_tile<XCD_RUN>(block);
}
inline size_t onesweep_grid(size_t tiles, uint32_t nx) {
  return nx == XCDS ? xcd_order_grid(tiles, XCD_RUN) : tiles;
}

// Two-level decoupled look-back for one digit (one thread per digit): in-group
// predecessors tile by tile until an inclusive prefix or the group start, then
// earlier groups whole (complete aggregates) until a group's inclusive prefix.
// lb, gi and ga hold the first windows, issued when the tile's own counts were
// published; a slot not yet published is polled again. Returns the exclusive
// prefix of the tile's count for this digit.
template <class Desc>
__device__ __forceinline__ Desc lookback_consume(const LookbackBuf<Desc> &lbuf, uint32_t tile,
                                                 uint32_t group, uint32_t digit,
                                                 Desc (&lb)[lookback_window<Desc>()],
                                                 Desc (&gi)[GWIN], uint32_t (&ga)[GWIN]) {
  using DI = DescInfo<Desc>;
  constexpr int WIN = lookback_window<Desc>();
  const int gfirst = static_cast<int>(group) * GROUP;
  Desc excl = 0;
  bool done = tile == 0;
  // Window slot w holds tile t - w; slots before the group are boundaries.
  int t = static_cast<int>(tile) - 1;
  auto eat_tiles = [&]() {
    int consumed = 0;
    bool stop = false;
#pragma unroll
    for (int w = 0; w < WIN; ++w) {
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
  // Group slot w holds group g - w; slots before group 0 read as an inclusive
  // zero.
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
  if (!done) {
    int c = eat_tiles();
    while (!done && t >= gfirst) {
      if (c == 0) __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int w = 0; w < WIN; ++w)
        lb[w] = load_agent(&lbuf.tile[size_t(max(t - w, 0)) * BINS + digit]);
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
        gi[w] = load_agent(&lbuf.ginc[gg * BINS + digit]);
        ga[w] = load_agent(&lbuf.gagg[gg * BINS + digit]);
      }
      c = eat_groups();
    }
  }
  return excl;
}

// Opaque copy: the compiler must assume the value changed here, so it cannot
// carry values derived from it across this point. Aggregate keys (record
// rows) overload it in their own namespace, found by argument-dependent
// lookup.
template <class T>
__device__ __forceinline__ void launder(T &x) {
  asm volatile("" : "+v"(x));
}

// True when every lane of the (fully active) wave holds the same value.
__device__ __forceinline__ bool wave_uniform(uint32_t v) {
  return __ballot(v == __builtin_amdgcn_readfirstlane(v)) == ~uint64_t(0);
}

// Lanes of the fully active wave whose value of `d` equals this lane's, over
// the bits set in `bits` (one ballot per bit; the digits differ in no other
// bit).
__device__ __forceinline__ uint64_t peer_lanes(uint32_t d, uint32_t bits) {
  uint64_t m = ~uint64_t(0);
#pragma unroll
  for (int b = 0; b < 9; ++b) {
    if (bits & (1u << b)) {
      const bool set = ((d >> b) & 1u) != 0;
      const uint64_t bal = __ballot(set);
      m &= set ? bal : ~bal;
    }
  }
  return m;
}

// Lowest set lane of a non-zero mask.
__device__ __forceinline__ uint32_t lowest_lane(uint64_t m) {
  return static_cast<uint32_t>(__builtin_ctzll(m));
}

// One tile of a onesweep pass. Keys are any trivially copyable type whose
// digits Ops::digit extracts (scalar keys, or record rows); the kernels below
// wrap it. nx == XCDS: the block's tile is xcd_tile(block); otherwise the
// block claims its tile from the pass's ticket counter.
template <class Bits, class Val, class Ops, int ITEMS, class Desc, int THREADS, Rank RANK>
__device__ __forceinline__ void
onesweep_tile(const Bits *__restrict__ keys_in, Bits *__restrict__ keys_out,
              const Val *__restrict__ vals_in, Val *__restrict__ vals_out, size_t n,
              uint32_t num_tiles, const uint32_t *__restrict__ pass_bins,
              const uint32_t *__restrict__ pass_skew, LookbackBuf<Desc> lbuf,
              LookbackBuf<Desc> lbuf_next, uint32_t nx, uint32_t bit, uint32_t mask,
              uint32_t conv) {
  constexpr bool PAIRS = !std::is_same<Val, NoValue>::value;
  constexpr int WAVES = THREADS / 64;
  constexpr int TILE = THREADS * ITEMS;
  constexpr int WAVE_ITEMS = 64 * ITEMS;
  // Items past the end of the input (last tile only) count in an extra dummy
  // bin and stage into one spare slot, so the loops need no branches.
  constexpr int NB = BINS + 1;
  constexpr uint32_t DUMMY = BINS;
  constexpr size_t VAL_BYTES = PAIRS ? sizeof(Val) : 0;
  constexpr size_t STAGE_ELEM = sizeof(Bits) > VAL_BYTES ? sizeof(Bits) : VAL_BYTES;
  constexpr int BATCH = RCCL_RADIX_LDS_BATCH;
  static_assert(THREADS >= BINS, "one thread per digit is required");
  static_assert(uint64_t(GROUP) * TILE <= GAGG_MASK, "group counts must fit the packed word");
  static_assert(LOOKBACK >= 1 && GWIN >= 1, "look-back windows");
  using DI = DescInfo<Desc>;
  using ValReg = typename std::conditional<PAIRS, Val, char>::type;

  __shared__ __attribute__((aligned(16))) unsigned char stage_raw[(TILE + 1) * STAGE_ELEM];
  __shared__ uint32_t cnt[WAVES][NB];  // per-wave digit counters, then positions
  __shared__ uint32_t digit_off[BINS];
  __shared__ uint32_t wave_sum[BINS / 64];
  __shared__ uint32_t s_tile;
  __shared__ uint32_t s_skew_waves;  // set when some wave takes the skewed ranking
  Bits *stage_keys = reinterpret_cast<Bits *>(stage_raw);

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  uint32_t tile;
  if (nx == XCDS) {
    tile = xcd_tile(blockIdx.x);
  } else {
    // Tile tickets: claimed in order by started blocks only.
    if (tid == 0) s_tile = add_agent(&lbuf.ticket[0], 1u);
    __syncthreads();
    tile = s_tile;
  }
  if (tile >= num_tiles) return;
  for (uint32_t i = tid; i < WAVES * NB; i += THREADS) (&cnt[0][0])[i] = 0;
  if (tid == 0) s_skew_waves = 0;
  // Global start of each digit's bucket (exclusive offsets from bins_scan).
  const uint32_t bin_start = tid < BINS ? pass_bins[tid] : 0u;
  // The pass's skew word, read before the keys so its latency hides behind
  // theirs (the skewed ranking below).
  constexpr bool SKEW_PATH = RANK == Rank::LaneAtomic && skew_ranking<Bits, Val, ITEMS>();
  const bool pass_skewed = SKEW_PATH && pass_skew && *pass_skew != 0;

  // Wave-contiguous, lane-striped load: item j of lane l is key
  // wave_base + 64 j + l, so (wave, item, lane) order is source order. Loads
  // are clamped to the wave's last valid item instead of predicated (a wave
  // past the end reads the input's last key); items past the end rank as
  // dummies whatever they hold. Addresses are a wave-uniform base plus a
  // 32-bit item index.
  const size_t wave_base =
      size_t(tile) * TILE + size_t(__builtin_amdgcn_readfirstlane(wave)) * WAVE_ITEMS;
  const uint32_t wave_valid =
      n > wave_base ? static_cast<uint32_t>(n - wave_base < WAVE_ITEMS ? n - wave_base
                                                                       : size_t(WAVE_ITEMS))
                    : 0u;
  const size_t load_base = wave_valid ? wave_base : n - 1;
  const uint32_t last_in_wave = wave_valid ? wave_valid - 1 : 0u;
  const Bits *kp = keys_in + load_base;
  // An opaque copy of the lane: the load indices then share nothing with the
  // validity tests below, so they are not kept alive until those run.
  uint32_t load_lane = lane;
  asm("" : "+v"(load_lane));
  Bits key[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j)
    key[j] = stream_load<!PAIRS || RCCL_RADIX_NT_PAIR_KEYS>(
        &kp[min(uint32_t(j * 64) + load_lane, last_in_wave)]);
  ValReg val[ITEMS];
  if constexpr (PAIRS) {
    // Issued now, consumed after the key scatter.
    const Val *vp = vals_in + load_base;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) val[j] = vp[min(uint32_t(j * 64) + load_lane, last_in_wave)];
  }
  lds_barrier();
  // Wait for all the keys (not the values) before counting: one wait here is
  // measurably faster than the per-item waits the compiler would interleave
  // with the counting atomics.
  wait_vmcnt<PAIRS ? ITEMS : 0>();
  // Raw input (the sort's first pass): to the order-preserving image, which
  // the tile keeps (a no-op for unsigned ascending keys).
  if (conv & CONV_IN) {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) key[j] = Ops::image(key[j]);
  }

  // Per-wave digit counts. Lanes of one LDS atomic that hit the same counter
  // are served one after another, so an item whose digit is the same in all
  // 64 lanes (skewed or presorted keys, a constant byte) is counted by one
  // lane adding 64.
  //
  // Skewed passes (bins_scan_kernel flags a pass whose most frequent digit
  // holds at least 1 / RCCL_RADIX_HOT_DIV of the keys), and skewed waves of
  // other passes (below; lane-ordered ranking only), count with returning
  // atomics, whose results are the keys' ranks
  // within their wave and digit. Each thread parks its ranks in its own slots
  // of the staging area (free until the keys are staged) and reads them back
  // after the count, so the ranking below reads each wave's digit start
  // instead of adding to it: a read that many lanes share is served once,
  // where an atomic on a hot digit's counter is served lane by lane.
  uint32_t *wcnt = cnt[wave];
  bool skewed = pass_skewed;
  if (SKEW_PATH && !skewed) {
    // A wave of a pass that is not skewed as a whole can still hold a skewed
    // stretch of the input (the previous pass gathers equal digits into
    // neighbouring tiles). The wave takes the skewed path when, in its first
    // or middle item, at least RCCL_RADIX_SKEW_LANES lanes share lane 0's
    // digit; that includes waves of presorted keys, whose items are
    // wave-uniform (the skewed path counts such an item with one atomic), so
    // the other path spends no test on wave-uniform items.
    auto shared_with_lane0 = [&](int j) {
      const uint32_t d =
          uint32_t(j) * 64 + lane < wave_valid ? Ops::image_digit(key[j], bit, mask) : DUMMY;
      return static_cast<uint32_t>(
          __builtin_popcountll(__ballot(d == __builtin_amdgcn_readfirstlane(d))));
    };
    const uint32_t m0 = shared_with_lane0(0), m1 = shared_with_lane0(ITEMS / 2);
    skewed = m0 >= RCCL_RADIX_SKEW_LANES || m1 >= RCCL_RADIX_SKEW_LANES;
  }
  if (skewed && lane == 0) s_skew_waves = 1;
  uint32_t *rank_slot = reinterpret_cast<uint32_t *>(stage_raw) + wave * WAVE_ITEMS + lane;
  uint32_t pos[ITEMS];
  if (skewed) {
    // The lanes sharing lane 0's digit (a whole wave-uniform item, or a hot
    // digit's group) take one atomic: lane 0 adds the group's size, and each
    // of the others is lane 0's base plus its group lanes below (marked with
    // PEER until the bases return). Every other lane takes its own atomic.
    constexpr uint32_t PEER = 1u << 31;
    uint32_t ret[ITEMS];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const uint32_t d =
          uint32_t(j) * 64 + lane < wave_valid ? Ops::image_digit(key[j], bit, mask) : DUMMY;
      const bool in_group = d == __builtin_amdgcn_readfirstlane(d);
      const uint64_t group = __ballot(in_group);
      if (in_group) {
        ret[j] = lane == 0 ? __hip_atomic_fetch_add(
                                 &wcnt[d], static_cast<uint32_t>(__builtin_popcountll(group)),
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                           : PEER | popc_below(group);
      } else {
        ret[j] =
            __hip_atomic_fetch_add(&wcnt[d], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const uint32_t base = __builtin_amdgcn_readfirstlane(ret[j]);
      rank_slot[j * 64] = (ret[j] & PEER) ? base + (ret[j] & ~PEER) : ret[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const uint32_t d =
          uint32_t(j) * 64 + lane < wave_valid ? Ops::image_digit(key[j], bit, mask) : DUMMY;
      // (With the skewed path, waves with wave-uniform items take it.)
      if (!SKEW_PATH && wave_uniform(d)) {
        if (lane == 0)
          __hip_atomic_fetch_add(&wcnt[d], 64u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      } else {
        __hip_atomic_fetch_add(&wcnt[d], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
  }
  lds_barrier();
  // Whether some wave of the block parked its ranks in the staging area.
  const bool block_skew = SKEW_PATH && s_skew_waves != 0;

  // Per digit: the tile's count, published at once together with the first
  // look-back windows (consumed after the ranking, so their latency hides
  // behind it); then the block-wide exclusive scan over digits.
  const uint32_t group = tile / GROUP;
  const int gfirst = static_cast<int>(group) * GROUP;
  uint32_t count = 0, tile_inc = 0;
  Desc lb[lookback_window<Desc>()];
  Desc gi[GWIN];
  uint32_t ga[GWIN];
  if (tid < BINS) {
#pragma unroll
    for (int w = 0; w < WAVES; ++w) count += cnt[w][tid];
    store_agent(&lbuf.tile[size_t(tile) * BINS + tid],
                static_cast<Desc>((tile == 0 ? DI::INCL : DI::AGG) | Desc(count)));
    add_agent(&lbuf.gagg[size_t(group) * BINS + tid], (1u << GAGG_SHIFT) | count);
    // Window loads are clamped to valid slots; slots outside the window are
    // masked when the window is consumed.
#pragma unroll
    for (int w = 0; w < lookback_window<Desc>(); ++w)
      lb[w] = load_agent(
          &lbuf.tile[size_t(max(static_cast<int>(tile) - 1 - w, 0)) * BINS + tid]);
#pragma unroll
    for (int w = 0; w < GWIN; ++w) {
      const size_t g = size_t(max(static_cast<int>(group) - 1 - w, 0));
      gi[w] = load_agent(&lbuf.ginc[g * BINS + tid]);
      ga[w] = load_agent(&lbuf.gagg[g * BINS + tid]);
    }
    tile_inc = wave_inclusive_sum(count, lane);
    if (lane == 63) wave_sum[wave] = tile_inc;
  }
  lds_barrier();
  uint32_t tile_start = 0;
  if (tid < BINS) {
    tile_start = tile_inc - count;
    for (uint32_t w = 0; w < wave; ++w) tile_start += wave_sum[w];
    // Each wave's counter becomes the tile position of its first key of this
    // digit (the counts are read again rather than held in registers).
    uint32_t run = tile_start;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const uint32_t c = cnt[w][tid];
      cnt[w][tid] = run;
      run += c;
    }
  }
  if (tid < WAVES) cnt[tid][DUMMY] = TILE;
  lds_barrier();

  // Rank and stage. The digits are recomputed: an opaque copy of the keys
  // stops the compiler from keeping all of them (or their counter addresses)
  // alive from the counting loop. Equal digits get positions in (wave, item,
  // lane) order, which is source order; dummies all land in the spare slot.
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) launder(key[j]);
  if constexpr (RANK == Rank::MatchAny) {
    // Match-any, in batches of MB items (each item's peer data is held until
    // its base returns); a batch's atomics are issued together. Digits can
    // differ only in the bits of `mask`, and the dummy bin in the last tile.
    constexpr int MB = RCCL_RADIX_MATCH_BATCH;
    const uint32_t dbits = mask | (tile + 1 == num_tiles ? DUMMY : 0u);
#pragma unroll
    for (int j0 = 0; j0 < ITEMS; j0 += MB) {
      uint32_t peer[MB];  // lowest peer lane | peers below << 8
#pragma unroll
      for (int b = 0; b < MB && j0 + b < ITEMS; ++b) {
        const int j = j0 + b;
        const uint32_t d =
            uint32_t(j) * 64 + lane < wave_valid ? Ops::image_digit(key[j], bit, mask) : DUMMY;
        const uint64_t m = peer_lanes(d, dbits);
        const uint32_t below = popc_below(m);
        peer[b] = lowest_lane(m) | (below << 8);
        pos[j] = below == 0 ? __hip_atomic_fetch_add(
                                  &wcnt[d], static_cast<uint32_t>(__builtin_popcountll(m)),
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                            : 0u;
      }
#pragma unroll
      for (int b = 0; b < MB && j0 + b < ITEMS; ++b) asm volatile("" : "+v"(pos[j0 + b]));
#pragma unroll
      for (int b = 0; b < MB && j0 + b < ITEMS; ++b) {
        const int j = j0 + b;
        const uint32_t base = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(
            static_cast<int>((peer[b] & 63u) << 2), static_cast<int>(pos[j])));
        pos[j] = min(base + (peer[b] >> 8), uint32_t(TILE));
        stage_keys[pos[j]] = key[j];
      }
    }
  } else {
    // Where some wave of the block parked its ranks, every parked rank is read
    // before any key is staged over it: each wave passes one barrier (the
    // skewed flag is the same in all lanes of a wave).
    if (skewed) {
      // Position = the wave's start for the digit + the rank from the count.
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) pos[j] = rank_slot[j * 64];
      lds_barrier();
      // In batches: a batch's counter reads are issued together, then its keys
      // staged (all at once would hold a second register per key).
      constexpr int RB = RCCL_RADIX_RANK_BATCH;
#pragma unroll
      for (int j0 = 0; j0 < ITEMS; j0 += RB) {
        uint32_t start[RB];
#pragma unroll
        for (int j = j0; j < j0 + RB && j < ITEMS; ++j) {
          const uint32_t d =
              uint32_t(j) * 64 + lane < wave_valid ? Ops::image_digit(key[j], bit, mask) : DUMMY;
          start[j - j0] = wcnt[d];
        }
#pragma unroll
        for (int j = j0; j < j0 + RB && j < ITEMS; ++j) asm volatile("" : "+v"(start[j - j0]));
#pragma unroll
        for (int j = j0; j < j0 + RB && j < ITEMS; ++j) {
          pos[j] = min(pos[j] + start[j - j0], uint32_t(TILE));
          stage_keys[pos[j]] = key[j];
        }
      }
    } else {
      if (block_skew) lds_barrier();
      // The returning atomic hands equal digits consecutive positions in lane
      // order. All atomics are issued before the first staging write, so the
      // round trips overlap; the opaque copy of the positions keeps the
      // compiler from pairing each write with its atomic (which serialises
      // them). A wave-uniform digit takes 64 consecutive positions with one
      // atomic: lane l's is the returned base + l, as the lane-ordered atomic
      // would give.
      uint64_t uniform = 0;
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        const uint32_t d =
            uint32_t(j) * 64 + lane < wave_valid ? Ops::image_digit(key[j], bit, mask) : DUMMY;
        if (!SKEW_PATH && wave_uniform(d)) {
          uniform |= uint64_t(1) << j;
          pos[j] = lane == 0 ? __hip_atomic_fetch_add(&wcnt[d], 64u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_WORKGROUP)
                             : 0u;
        } else {
          pos[j] =
              __hip_atomic_fetch_add(&wcnt[d], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
      }
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) asm volatile("" : "+v"(pos[j]));
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        if (uniform & (uint64_t(1) << j)) pos[j] = __builtin_amdgcn_readfirstlane(pos[j]) + lane;
        pos[j] = min(pos[j], uint32_t(TILE));
        stage_keys[pos[j]] = key[j];
      }
    }
  }

  // All loads (the look-back windows included) are complete on both sides of
  // this branch before the prefix stores. Without that the compiler cannot
  // tell at the join which loads may still be in flight, and makes the
  // scatter wait for every outstanding operation, the prefix stores' round
  // trip included.
  if (tid < BINS) {
    const Desc excl = lookback_consume<Desc>(lbuf, tile, group, tid, lb, gi, ga);
    wait_vmcnt<0>();
    const Desc incl = static_cast<Desc>(DI::INCL | (excl + Desc(count)));
    const uint32_t glast = min(uint32_t(gfirst + GROUP), num_tiles) - 1u;
    if (tile == glast) store_agent(&lbuf.ginc[size_t(group) * BINS + tid], incl);
    digit_off[tid] = bin_start + static_cast<uint32_t>(excl) - tile_start;
  } else {
    wait_vmcnt<0>();
  }
  lds_barrier();

  // Coalesced scatter: consecutive staged keys of one digit go to consecutive
  // output positions. Positions are exact when the bins match the keys; the
  // clamp only keeps a caller that changes the keys mid-sort from writing out
  // of bounds. In batches: the staged keys are read together, then their
  // digits' offsets, then stored.
  const size_t tile_base = size_t(tile) * TILE;
  uint32_t valid_count = static_cast<uint32_t>(min<size_t>(TILE, n - tile_base));
  // Materialized here, in a scalar register: otherwise this compiler sinks
  // the min into the partial-tile branch below and selects on a stale scalar
  // condition code there (valid_count came out as TILE for the last tile).
  asm volatile("" : "+s"(valid_count));
  const uint32_t last = static_cast<uint32_t>(n - 1);
  uint32_t dst[PAIRS ? ITEMS : 1];
  // One batch of keys: staged keys read together, then their digits'
  // offsets, then stored (all items, or those before valid_count).
  auto scatter_batch = [&](int k0, auto full) {
    constexpr bool FULL = decltype(full)::value;
    Bits kk[BATCH];
    uint32_t off[BATCH];
#pragma unroll
    for (int b = 0; b < BATCH && k0 + b < ITEMS; ++b)
      kk[b] = stage_keys[uint32_t(k0 + b) * THREADS + tid];
#pragma unroll
    for (int b = 0; b < BATCH && k0 + b < ITEMS; ++b)
      off[b] = digit_off[Ops::image_digit(kk[b], bit, mask)];
    // The sort's last pass stores raw keys (a wave-uniform branch: the other
    // passes store the images as they are).
    if (conv & CONV_OUT) {
#pragma unroll
      for (int b = 0; b < BATCH && k0 + b < ITEMS; ++b) kk[b] = Ops::raw(kk[b]);
    }
#pragma unroll
    for (int b = 0; b < BATCH && k0 + b < ITEMS; ++b) {
      const uint32_t i = uint32_t(k0 + b) * THREADS + tid;
      const uint32_t p = min(off[b] + i, last);
      if (FULL || i < valid_count) keys_out[p] = kk[b];
      if constexpr (PAIRS) dst[k0 + b] = p;
    }
  };
  if constexpr (PAIRS) {
#pragma unroll
    for (int k0 = 0; k0 < ITEMS; k0 += BATCH) scatter_batch(k0, std::false_type{});
  } else if (valid_count == uint32_t(TILE)) {
    // Every tile but the last is full: for keys only, a copy of the loop
    // without the per-item test (and its exec-mask branch per store). (With
    // values, the copy and the positions kept for the value stores make the
    // 28-item shapes spill.)
#pragma unroll
    for (int k0 = 0; k0 < ITEMS; k0 += BATCH) scatter_batch(k0, std::true_type{});
  } else {
#pragma unroll
    for (int k0 = 0; k0 < ITEMS; k0 += BATCH) scatter_batch(k0, std::false_type{});
  }
  if constexpr (PAIRS) {
    lds_barrier();
    Val *stage_vals = reinterpret_cast<Val *>(stage_raw);
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) stage_vals[pos[j]] = val[j];
    lds_barrier();
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t i = uint32_t(k) * THREADS + tid;
      if (i < valid_count) vals_out[dst[k]] = stage_vals[i];
    }
  }
  // Clear this tile's slots of the next pass's look-back buffer (it is not
  // read before the next launch).
  if (tid < BINS && lbuf_next.tile) {
    lbuf_next.tile[size_t(tile) * BINS + tid] = 0;
    if (static_cast<int>(tile) == gfirst) {
      lbuf_next.ginc[size_t(group) * BINS + tid] = 0;
      lbuf_next.gagg[size_t(group) * BINS + tid] = 0;
    }
    if (tile == 0 && tid < XCDS) lbuf_next.ticket[tid] = 0;
  }
}

template <class Bits, class Val, class Ops, int ITEMS, class Desc, int THREADS, Rank RANK>
__global__ void __launch_bounds__(THREADS, RCCL_RADIX_WAVES_PER_SIMD)
onesweep_kernel(const Bits *__restrict__ keys_in, Bits *__restrict__ keys_out,
                const Val *__restrict__ vals_in, Val *__restrict__ vals_out, size_t n,
                uint32_t num_tiles, const uint32_t *__restrict__ pass_bins,
                const uint32_t *__restrict__ pass_skew, LookbackBuf<Desc> lbuf,
                LookbackBuf<Desc> lbuf_next, uint32_t nx, uint32_t bit, uint32_t mask,
                uint32_t conv) {
  // Never null here (only the record sort passes none): no branch around its
  // load before the keys'.
  __builtin_assume(pass_skew != nullptr);
  onesweep_tile<Bits, Val, Ops, ITEMS, Desc, THREADS, RANK>(keys_in, keys_out, vals_in, vals_out,
                                                            n, num_tiles, pass_bins, pass_skew,
                                                            lbuf, lbuf_next, nx, bit, mask, conv);
}

// Input, output and scratch buffers of a planned sort (PassPlan numbering).
template <class Bits, class Val>
struct PlanBuffers {
  const Bits *in;
  Bits *out, *scratch;
  const Val *vin;
  Val *vout, *vscratch;
};

// One pass of a planned sort: inactive passes return at once; active ones
// read and write the buffers and look-back buffer the plan names.
template <class Bits, class Val, class Ops, int ITEMS, class Desc, int THREADS, Rank RANK>
__global__ void __launch_bounds__(THREADS, RCCL_RADIX_WAVES_PER_SIMD)
planned_onesweep_kernel(PlanBuffers<Bits, Val> b, size_t n, uint32_t num_tiles,
                        const uint32_t *__restrict__ pass_bins,
                        const uint32_t *__restrict__ pass_skew, const PassPlan *__restrict__ plan,
                        LookbackBuf<Desc> lb0, LookbackBuf<Desc> lb1, uint32_t nx, uint32_t bit,
                        uint32_t mask) {
  __builtin_assume(pass_skew != nullptr);
  const PassPlan pl = *plan;
  if (!pl.active) return;
  const Bits *kin = pl.src == 0 ? b.in : (pl.src == 1 ? b.out : b.scratch);
  Bits *kout = pl.dst == 1 ? b.out : b.scratch;
  const Val *vin = pl.src == 0 ? b.vin : (pl.src == 1 ? b.vout : b.vscratch);
  Val *vout = pl.dst == 1 ? b.vout : b.vscratch;
  onesweep_tile<Bits, Val, Ops, ITEMS, Desc, THREADS, RANK>(kin, kout, vin, vout, n, num_tiles,
                                                            pass_bins, pass_skew, pl.lb ? lb1 : lb0,
                                                            pl.lb ? lb0 : lb1, nx, bit, mask,
                                                            pl.conv);
}

// ---------------------------------------------------------------------------
// single tile: inputs of at most single_tile_items() items are sorted by one
// block in one launch (the reference's single-tile route,
// rccl-cub/src/radix.rs:470-492, ordering_backend/radix.rs:366-715). Keys
// and values are loaded into LDS once; every 8-bit pass counts, scans and
// ranks them as a onesweep tile does (per-wave counters, either ranking
// mode) and scatters them into the other LDS buffer; the result is stored
// once. No workspace is touched.
// ---------------------------------------------------------------------------
constexpr int ST_THREADS = 256;

// The reference's single-tile capacity: 256 threads x 19 * 4 / max(item
// bytes, 4) items (rccl-cub/src/workspace.rs:22-66).
constexpr size_t single_tile_items(size_t key_bytes, size_t value_bytes) {
  const size_t item = std::max<size_t>(std::max(key_bytes, value_bytes), 4);
  return size_t(ST_THREADS) * std::max<size_t>(1, 19 * 4 / item);
}

template <class Bits, class Val, class Ops, int ITEMS, Rank RANK>
__global__ void __launch_bounds__(ST_THREADS)
single_tile_kernel(const Bits *keys_in, Bits *keys_out, const Val *vals_in, Val *vals_out,
                   uint32_t n, uint32_t begin_bit, uint32_t end_bit) {
  // keys_out may be keys_in (in place): every input is read before the first
  // barrier and every output written after the last.
  constexpr bool PAIRS = !std::is_same<Val, NoValue>::value;
  constexpr int WAVES = ST_THREADS / 64;
  constexpr int TILE = ST_THREADS * ITEMS;
  constexpr int WAVE_ITEMS = 64 * ITEMS;
  constexpr int NB = BINS + 1;
  constexpr uint32_t DUMMY = BINS;
  static_assert(ST_THREADS == BINS, "one thread per digit");
  using VStore = typename std::conditional<PAIRS, Val, char>::type;
  __shared__ Bits kbuf[2][TILE];
  __shared__ VStore vbuf[PAIRS ? 2 : 1][PAIRS ? TILE : 1];
  __shared__ uint32_t cnt[WAVES][NB];
  __shared__ uint32_t wave_sum[WAVES];

  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  for (uint32_t i = tid; i < n; i += ST_THREADS) {
    kbuf[0][i] = keys_in[i];
    if constexpr (PAIRS) vbuf[0][i] = vals_in[i];
  }
  int cur = 0;
  for (uint32_t bit = begin_bit; bit < end_bit; bit += 8) {
    const uint32_t mask = (1u << min(8u, end_bit - bit)) - 1u;
    for (uint32_t i = tid; i < WAVES * NB; i += ST_THREADS) (&cnt[0][0])[i] = 0;
    __syncthreads();
    // (wave, item, lane) order is source order; items at or past n are
    // dummies, placed after every key.
    Bits key[ITEMS];
    uint32_t dg[ITEMS];
    uint32_t *wcnt = cnt[wave];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const uint32_t i = wave * WAVE_ITEMS + uint32_t(j) * 64 + lane;
      key[j] = kbuf[cur][min(i, uint32_t(TILE - 1))];
      dg[j] = i < n ? Ops::digit(key[j], bit, mask) : DUMMY;
      __hip_atomic_fetch_add(&wcnt[dg[j]], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();
    // Digit starts (exclusive scan over digits), then each wave's start.
    uint32_t wc[WAVES], count = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      wc[w] = cnt[w][tid];
      count += wc[w];
    }
    const uint32_t inc = wave_inclusive_sum(count, lane);
    if (lane == 63) wave_sum[wave] = inc;
    __syncthreads();
    uint32_t run = inc - count;
    for (uint32_t w = 0; w < wave; ++w) run += wave_sum[w];
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      cnt[w][tid] = run;
      run += wc[w];
    }
    if (tid < WAVES) cnt[tid][DUMMY] = max(n, tid * uint32_t(WAVE_ITEMS));
    __syncthreads();
    const uint32_t dbits = mask | DUMMY;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const uint32_t d = dg[j];
      uint32_t pos;
      if constexpr (RANK == Rank::MatchAny) {
        const uint64_t m = peer_lanes(d, dbits);
        const uint32_t below = popc_below(m);
        const uint32_t base =
            below == 0 ? __hip_atomic_fetch_add(&wcnt[d],
                                                static_cast<uint32_t>(__builtin_popcountll(m)),
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                       : 0u;
        pos = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(
                  static_cast<int>(lowest_lane(m) << 2), static_cast<int>(base))) +
              below;
      } else {
        pos = __hip_atomic_fetch_add(&wcnt[d], 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      pos = min(pos, uint32_t(TILE - 1));
      kbuf[cur ^ 1][pos] = key[j];
      if constexpr (PAIRS) {
        const uint32_t i = wave * WAVE_ITEMS + uint32_t(j) * 64 + lane;
        vbuf[cur ^ 1][pos] = vbuf[cur][min(i, uint32_t(TILE - 1))];
      }
    }
    __syncthreads();
    cur ^= 1;
  }
  for (uint32_t i = tid; i < n; i += ST_THREADS) {
    keys_out[i] = kbuf[cur][i];
    if constexpr (PAIRS) vals_out[i] = vbuf[cur][i];
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

// Per-device facts a onesweep launch needs, found once per device
// (radix.hip): whether the LDS serves same-address atomic lanes in lane
// order, whether blocks land on the XCDs round-robin (nx = XCDS ticket
// counters, else 1), and the ranking mode to use (lane-ordered atomics where
// they hold, unless match-any is requested with rccl_hip_radix_set_ranking).
struct DeviceCaps {
  bool lane_order = false;
  uint32_t nx = 1;
  Rank rank = Rank::MatchAny;
  uint32_t cus = 0;  // compute units (sizes the histogram grid)
};
// Fails, before any launch, on a stream under graph capture when the device
// was not probed yet (rccl_hip_program_load probes it).
rccl_hip_status device_caps(DeviceCaps *caps, hipStream_t stream);

struct SortArgs {
  void *keys[2];
  void *vals[2];
  size_t n;
  int cur;  // index of the buffer holding the input
  uint32_t begin_bit, end_bit;
  unsigned char *ws;
  hipStream_t stream;
  // When set, the histogram and the first pass read the input from here
  // instead of keys[cur] / vals[cur], which then only receive output: sorts
  // that must leave their input untouched start without a copy.
  const void *src_keys = nullptr;
  const void *src_vals = nullptr;
  // Planned sorts skip trivial passes: keys[0] / vals[0] are the output,
  // keys[1] / vals[1] the scratch, src_keys / src_vals the input (either may
  // equal its output: in place). plan_flags says whether some stream is in
  // place and whether some is not (PLAN_IN_PLACE, PLAN_COPIES). The result
  // always ends in the output. The plan needs plan_bytes() of workspace after
  // the layout's.
  bool planned = false;
  uint32_t plan_flags = 0;
  // A single-tile sort (n <= single_tile_items) writes its result into the
  // other buffer of the pair (the DoubleBuffer form: one selector flip, as
  // the reference's single-tile route) or back into the current one.
  bool single_to_other = false;
};


template <class Desc>
void lookback_buffers(const SortArgs &a, const Layout &l, LookbackBuf<Desc> (&lb)[2]) {
  for (int b = 0; b < 2; ++b) {
    unsigned char *base = a.ws + l.lb[b];
    lb[b].tile = reinterpret_cast<Desc *>(base);
    lb[b].ginc = reinterpret_cast<Desc *>(base + l.lb_ginc);
    lb[b].gagg = reinterpret_cast<uint32_t *>(base + l.lb_gagg);
    lb[b].ticket = reinterpret_cast<uint32_t *>(base + l.lb_ticket);
  }
}

// The onesweep launches of a sort, in one ranking mode and tile shape, with
// or without a pass plan.
template <class Bits, class Val, class Ops, class Desc, Rank RANK, int THREADS, int ITEMS,
          bool PLANNED>
rccl_hip_status launch_onesweeps(SortArgs &a, const Layout &l, uint32_t passes,
                                 const uint32_t *bins, const uint32_t *skew, const PassPlan *plan,
                                 uint32_t nx) {
  LookbackBuf<Desc> lb[2];
  lookback_buffers(a, l, lb);
  size_t resident = 0;
  const void *kernel;
  if constexpr (PLANNED)
    kernel = reinterpret_cast<const void *>(
        &planned_onesweep_kernel<Bits, Val, Ops, ITEMS, Desc, THREADS, RANK>);
  else
    kernel = reinterpret_cast<const void *>(
        &onesweep_kernel<Bits, Val, Ops, ITEMS, Desc, THREADS, RANK>);
  RCCL_HIP_TRY(resident_blocks(kernel, THREADS, &resident));
  // The XCD order needs two rows of runs resident at once; with fewer, blocks
  // claim ticketed tiles instead.
  if (nx == XCDS && resident < 2 * size_t(XCDS) * XCD_RUN) nx = 1;
  const uint32_t grid = static_cast<uint32_t>(onesweep_grid(l.tiles, nx));

  if constexpr (PLANNED) {
    const PlanBuffers<Bits, Val> b{
        static_cast<const Bits *>(a.src_keys ? a.src_keys : a.keys[0]),
        static_cast<Bits *>(a.keys[0]), static_cast<Bits *>(a.keys[1]),
        static_cast<const Val *>(a.src_keys ? a.src_vals : a.vals[0]),
        static_cast<Val *>(a.vals[0]), static_cast<Val *>(a.vals[1])};
    for (uint32_t p = 0; p < passes; ++p) {
      const uint32_t bit = a.begin_bit + 8u * p;
      const uint32_t mask = (1u << std::min(8u, a.end_bit - bit)) - 1u;
      KernelTimer t("radix_onesweep", a.stream, a.n);
      planned_onesweep_kernel<Bits, Val, Ops, ITEMS, Desc, THREADS, RANK>
          <<<dim3(grid), THREADS, 0, a.stream>>>(b, a.n, static_cast<uint32_t>(l.tiles),
                                                 bins + size_t(p) * BINS, skew + p,
                                                 plan + p, lb[0], lb[1], nx, bit, mask);
      RCCL_HIP_TRY(check_launch("radix onesweep"));
    }
    a.cur = 0;
    return ok();
  }
  for (uint32_t p = 0; p < passes; ++p) {
    const uint32_t bit = a.begin_bit + 8u * p;
    const uint32_t width = std::min(8u, a.end_bit - bit);
    const uint32_t mask = (1u << width) - 1u;
    const int in = a.cur, out = 1 - a.cur;
    const bool from_src = p == 0 && a.src_keys;
    const void *kin = from_src ? a.src_keys : a.keys[in];
    const void *vin = from_src ? a.src_vals : a.vals[in];
    KernelTimer t("radix_onesweep", a.stream, a.n);
    onesweep_kernel<Bits, Val, Ops, ITEMS, Desc, THREADS, RANK>
        <<<dim3(grid), THREADS, 0, a.stream>>>(
            static_cast<const Bits *>(kin), static_cast<Bits *>(a.keys[out]),
            static_cast<const Val *>(vin), static_cast<Val *>(a.vals[out]), a.n,
            static_cast<uint32_t>(l.tiles), bins + size_t(p) * BINS, skew + p,
            lb[p & 1],
            p + 1 < passes ? lb[(p + 1) & 1]
                           : LookbackBuf<Desc>{nullptr, nullptr, nullptr, nullptr},
            nx, bit, mask, (p == 0 ? CONV_IN : 0u) | (p + 1 == passes ? CONV_OUT : 0u));
    RCCL_HIP_TRY(check_launch("radix onesweep"));
    a.cur = out;
  }
  return ok();
}

template <class Bits, class Val, class Ops, Rank RANK>
rccl_hip_status launch_single_tile(SortArgs &a) {
  constexpr size_t VBYTES = std::is_same<Val, NoValue>::value ? 0 : sizeof(Val);
  constexpr int ITEMS = static_cast<int>(single_tile_items(sizeof(Bits), VBYTES) / ST_THREADS);
  const int dst = a.single_to_other ? 1 - a.cur : a.cur;
  {
    KernelTimer t("radix_single_tile", a.stream, a.n);
    single_tile_kernel<Bits, Val, Ops, ITEMS, RANK><<<1, ST_THREADS, 0, a.stream>>>(
        static_cast<const Bits *>(a.keys[a.cur]), static_cast<Bits *>(a.keys[dst]),
        static_cast<const Val *>(a.vals[a.cur]), static_cast<Val *>(a.vals[dst]),
        static_cast<uint32_t>(a.n), a.begin_bit, a.end_bit);
  }
  RCCL_HIP_TRY(check_launch("radix single tile"));
  a.cur = dst;
  return ok();
}

template <class Bits, class Val, class Ops, class Desc>
rccl_hip_status run_passes(SortArgs &a, const Layout &l, uint32_t passes) {
  DeviceCaps caps;
  RCCL_HIP_TRY(device_caps(&caps, a.stream));
  constexpr size_t VBYTES = std::is_same<Val, NoValue>::value ? 0 : sizeof(Val);
  if (!a.planned && !a.src_keys && a.n <= single_tile_items(sizeof(Bits), VBYTES))
    return caps.rank == Rank::LaneAtomic ? launch_single_tile<Bits, Val, Ops, Rank::LaneAtomic>(a)
                                         : launch_single_tile<Bits, Val, Ops, Rank::MatchAny>(a);
  uint32_t *bins = reinterpret_cast<uint32_t *>(a.ws + l.bins);
  uint32_t *skew = reinterpret_cast<uint32_t *>(a.ws + l.skew);
  {
    KernelTimer t("radix_init", a.stream, 0);
    init_kernel<<<1, 256, 0, a.stream>>>(bins, passes);
  }
  RCCL_HIP_TRY(check_launch("radix init"));

  const size_t zero_words = l.lb_bytes / sizeof(uint32_t);
  PassPlan *plan = a.planned ? reinterpret_cast<PassPlan *>(a.ws + l.total) : nullptr;
  {
    KernelTimer t("radix_histogram", a.stream, a.n);
    const size_t chunk = size_t(HIST_THREADS) * HIST_ITEMS;
    const size_t per_cu =
        (160 * 1024) / (sizeof(Bits) * BINS * hist_cols<Bits>() * sizeof(uint32_t));
    const size_t blocks = std::max<size_t>(
        1, std::min<size_t>((a.n + chunk - 1) / chunk, size_t(caps.cus) * per_cu));
    histogram_kernel<Bits, Ops><<<dim3(static_cast<uint32_t>(blocks)), HIST_THREADS, 0,
                                  a.stream>>>(
        static_cast<const Bits *>(a.src_keys ? a.src_keys : a.keys[a.cur]), a.n, bins,
        a.begin_bit, a.end_bit, passes, reinterpret_cast<uint32_t *>(a.ws + l.lb[0]),
        zero_words);
  }
  RCCL_HIP_TRY(check_launch("radix histogram"));
  {
    KernelTimer t("radix_bins_scan", a.stream, passes * BINS);
    static_assert(sizeof(Bits) <= 8, "one pass per key byte");
    if (passes > sizeof(Bits))
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix passes", sizeof(Bits), passes);
    bins_scan_kernel<int(sizeof(Bits))><<<1, BINS, 0, a.stream>>>(
        bins, passes, static_cast<uint32_t>(a.n), plan, a.plan_flags, skew);
  }
  RCCL_HIP_TRY(check_launch("radix bins scan"));
  constexpr int ITEMS = items_for(sizeof(Bits), VBYTES);
  constexpr int THREADS = threads_for(VBYTES);
  constexpr int SITEMS = small_items_for(sizeof(Bits), VBYTES);
  constexpr Rank LA = Rank::LaneAtomic, MA = Rank::MatchAny;
  const bool la = caps.rank == LA;
  if (a.planned)
    return la ? launch_onesweeps<Bits, Val, Ops, Desc, LA, THREADS, ITEMS, true>(
                    a, l, passes, bins, skew, plan, caps.nx)
              : launch_onesweeps<Bits, Val, Ops, Desc, MA, THREADS, ITEMS, true>(
                    a, l, passes, bins, skew, plan, caps.nx);
  // Small tiles serve unplanned sorts only, all below 2^30 items (32-bit
  // descriptors); the layout chose them for this n.
  if constexpr (sizeof(Desc) == 4) {
    if (l.small)
      return la ? launch_onesweeps<Bits, Val, Ops, Desc, LA, SMALL_THREADS, SITEMS, false>(
                      a, l, passes, bins, skew, plan, caps.nx)
                : launch_onesweeps<Bits, Val, Ops, Desc, MA, SMALL_THREADS, SITEMS, false>(
                      a, l, passes, bins, skew, plan, caps.nx);
  }
  if (l.small) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix small-tile layout");
  return la ? launch_onesweeps<Bits, Val, Ops, Desc, LA, THREADS, ITEMS, false>(
                  a, l, passes, bins, skew, plan, caps.nx)
            : launch_onesweeps<Bits, Val, Ops, Desc, MA, THREADS, ITEMS, false>(
                  a, l, passes, bins, skew, plan, caps.nx);
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

// DeviceMergeSort over integer keys lowers to this stable radix sort (see
// radix.hip). Workspace: scratch keys and values, then the radix layout.
size_t merge_sort_lowering_bytes(size_t key_bytes, size_t value_bytes, size_t n);
rccl_hip_status merge_sort_lowering(rccl_hip_key_kind key, size_t value_bytes, bool descending,
                                    const void *in_keys, const void *in_vals, void *out_keys,
                                    void *out_vals, size_t n, void *workspace,
                                    size_t workspace_bytes, hipStream_t stream);


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
