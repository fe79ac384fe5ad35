// DeviceRadixSort for gfx950: onesweep LSD radix sort with 8-bit digits.
//
// Reference behaviour: rccl-cub/src/radix.rs:364-876 (validation and pass
// control) and rccl-cub/src/ordering_backend/radix.rs (device agents). The
// kernels below are an independent wave64 design:
//   init        zero the per-pass bins and tile counters (one tiny block)
//   histogram   one read of all keys builds every pass's 256-bin histogram in
//               LDS (per-wave private counters), then adds them to HBM bins;
//               it also zeroes look-back buffer 0
//   onesweep    one launch per pass: tile claim, wave64 match-any ranking via
//               LDS 64-bit OR masks, per-digit decoupled look-back on
//               agent-scope atomics, LDS-staged coalesced scatter
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace rccl_hip {
namespace radix {

constexpr int BINS = 256;

// Runtime key flags (uniform across the launch).
enum : uint32_t { KF_SIGNED = 1u, KF_FLOAT = 2u, KF_DESC = 4u };

struct NoValue {};

template <class Bits> struct BitsInfo;
template <> struct BitsInfo<uint32_t> {
  static constexpr uint32_t SIGN = 0x80000000u;
};
template <> struct BitsInfo<uint64_t> {
  static constexpr uint64_t SIGN = 0x8000000000000000ull;
};

// Ordered bit image of a raw key with the float ±0 collapse applied; digits
// are read from this value. Transforms: rccl-cub/src/ordering_backend/radix.rs:75-235;
// collapse: :257-337. Keys themselves are never rewritten.
template <class Bits>
__device__ __forceinline__ Bits digit_source(Bits raw, uint32_t flags) {
  constexpr Bits SIGN = BitsInfo<Bits>::SIGN;
  Bits x = raw;
  if (flags & (KF_SIGNED | KF_FLOAT)) {
    Bits m = ((flags & KF_FLOAT) && (raw & SIGN)) ? ~Bits(0) : SIGN;
    x ^= m;
  }
  if (flags & KF_DESC) x = ~x;
  if ((flags & KF_FLOAT) && x == SIGN - 1) x = SIGN;
  return x;
}

template <class Bits>
__device__ __forceinline__ uint32_t digit_of(Bits raw, uint32_t flags, uint32_t bit, uint32_t mask) {
  return static_cast<uint32_t>(digit_source(raw, flags) >> bit) & mask;
}

// Look-back descriptor: 2 flag bits over a count.
template <class Desc> struct DescInfo;
template <> struct DescInfo<uint32_t> {
  static constexpr int SHIFT = 30;
  static constexpr uint32_t AGG = 1u << 30, INCL = 2u << 30, MASK = (1u << 30) - 1;
};
template <> struct DescInfo<uint64_t> {
  static constexpr int SHIFT = 62;
  static constexpr uint64_t AGG = 1ull << 62, INCL = 2ull << 62, MASK = (1ull << 62) - 1;
};

// ---------------------------------------------------------------------------
// init: zero bins and tile counters.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) init_kernel(uint32_t *bins, uint32_t *counters,
                                                   uint32_t passes) {
  for (uint32_t i = threadIdx.x; i < passes * BINS; i += 256) bins[i] = 0;
  if (threadIdx.x < passes) counters[threadIdx.x] = 0;
}

// ---------------------------------------------------------------------------
// histogram: all passes' digit counts in one read of the keys.
// ---------------------------------------------------------------------------
constexpr int HIST_THREADS = 256;
constexpr int HIST_ITEMS = 16;

template <class Bits>
__global__ void __launch_bounds__(HIST_THREADS)
histogram_kernel(const Bits *__restrict__ keys, size_t n, uint32_t *__restrict__ bins,
                 uint32_t flags, uint32_t begin_bit, uint32_t end_bit, uint32_t passes,
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
    bool v[HIST_ITEMS];
#pragma unroll
    for (int j = 0; j < HIST_ITEMS; ++j) {
      size_t idx = base + size_t(j) * HIST_THREADS + tid;
      v[j] = idx < n;
      k[j] = v[j] ? keys[idx] : Bits(0);
    }
#pragma unroll
    for (int j = 0; j < HIST_ITEMS; ++j) {
      if (!v[j]) continue;
      Bits s = digit_source(k[j], flags);
      for (uint32_t p = 0; p < passes; ++p) {
        uint32_t bit = begin_bit + 8u * p;
        uint32_t width = min(8u, end_bit - bit);
        uint32_t d = static_cast<uint32_t>(s >> bit) & ((1u << width) - 1u);
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

// ---------------------------------------------------------------------------
// onesweep: one stable counting-sort pass over tiles of THREADS*ITEMS keys.
// ---------------------------------------------------------------------------
template <class Bits, class Val, int THREADS, int ITEMS, class Desc>
__global__ void __launch_bounds__(THREADS)
onesweep_kernel(const Bits *__restrict__ keys_in, Bits *__restrict__ keys_out,
                const Val *__restrict__ vals_in, Val *__restrict__ vals_out, size_t n,
                const uint32_t *__restrict__ pass_bins, Desc *lookback, Desc *lookback_next,
                uint32_t *tile_counter, uint32_t flags, uint32_t bit, uint32_t mask) {
  constexpr bool PAIRS = !std::is_same<Val, NoValue>::value;
  constexpr int WAVES = THREADS / 64;
  constexpr int TILE = THREADS * ITEMS;
  constexpr int WAVE_ITEMS = 64 * ITEMS;
  constexpr size_t VAL_BYTES = PAIRS ? sizeof(Val) : 0;
  constexpr size_t STAGE_ELEM = sizeof(Bits) > VAL_BYTES ? sizeof(Bits) : VAL_BYTES;
  static_assert(THREADS >= BINS, "one thread per digit is required");
  static_assert(size_t(TILE) * STAGE_ELEM >= size_t(WAVES) * BINS * 8,
                "match masks alias the staging buffer");
  using DI = DescInfo<Desc>;

  __shared__ __attribute__((aligned(16))) unsigned char stage_raw[TILE * STAGE_ELEM];
  __shared__ uint32_t hist[WAVES][BINS];
  __shared__ uint32_t digit_off[BINS];
  __shared__ uint64_t wave_sum[BINS / 64];
  __shared__ uint32_t s_tile;

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  uint64_t *match = reinterpret_cast<uint64_t *>(stage_raw);

  if (tid == 0) s_tile = add_agent(tile_counter, 1u);
  for (uint32_t i = tid; i < WAVES * BINS; i += THREADS) {
    match[i] = 0;
    (&hist[0][0])[i] = 0;
  }
  __syncthreads();
  const uint32_t tile = s_tile;
  const size_t tile_base = size_t(tile) * TILE;
  const size_t wave_base = tile_base + size_t(wave) * WAVE_ITEMS;

  // Wave-contiguous, lane-striped load: item j of lane l is key
  // wave_base + 64 j + l, so (item, lane) order is source order.
  Bits key[ITEMS];
  typename std::conditional<PAIRS, Val, char>::type val[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    size_t idx = wave_base + size_t(j) * 64 + lane;
    key[j] = idx < n ? keys_in[idx] : Bits(0);
  }
  if constexpr (PAIRS) {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      size_t idx = wave_base + size_t(j) * 64 + lane;
      if (idx < n) val[j] = vals_in[idx];
    }
  }

  // Stable rank within the wave. For each item the lanes OR their lane bit
  // into match[digit]; reading it back gives the peer set, whose popcount
  // below this lane plus the wave's running digit count is the rank. The
  // lowest peer advances the count and clears the mask. LDS operations of one
  // wave execute in order, so no barrier is needed between the steps.
  uint64_t *wmatch = match + wave * BINS;
  uint32_t *whist = hist[wave];
  const uint64_t lane_bit = 1ull << lane;
  uint32_t rank[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const bool valid = wave_base + size_t(j) * 64 + lane < n;
    const uint32_t d = digit_of(key[j], flags, bit, mask);
    if (valid) atomicOr(reinterpret_cast<unsigned long long *>(&wmatch[d]),
                        static_cast<unsigned long long>(lane_bit));
    __builtin_amdgcn_wave_barrier();
    uint64_t peers = 0;
    uint32_t base = 0;
    if (valid) {
      peers = wmatch[d];
      base = whist[d];
    }
    const uint32_t below = popc_below(peers);
    rank[j] = base + below;
    __builtin_amdgcn_wave_barrier();
    if (valid && below == 0) {
      whist[d] = base + __popcll(peers);
      wmatch[d] = 0;
    }
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();

  // Per digit: exclusive prefix over waves, tile total, aggregate publish.
  uint32_t count = 0;
  uint32_t tile_start = 0;
  uint32_t bin_start = 0;
  uint64_t packed = 0;
  uint64_t incl = 0;
  if (tid < BINS) {
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      uint32_t c = hist[w][tid];
      hist[w][tid] = count;
      count += c;
    }
    store_agent(&lookback[size_t(tile) * BINS + tid],
                static_cast<Desc>((tile == 0 ? DI::INCL : DI::AGG) | Desc(count)));
    // Exclusive scans over digits of (bin total, tile count), packed so one
    // 64-bit scan does both (tile counts never carry into the high word).
    packed = (uint64_t(pass_bins[tid]) << 32) | count;
    incl = wave_inclusive_sum(packed, lane);
    if (lane == 63) wave_sum[wave] = incl;
  }
  __syncthreads();
  if (tid < BINS) {
    uint64_t excl = incl - packed;
    for (uint32_t w = 0; w < wave; ++w) excl += wave_sum[w];
    tile_start = static_cast<uint32_t>(excl);
    bin_start = static_cast<uint32_t>(excl >> 32);
#pragma unroll
    for (int w = 0; w < WAVES; ++w) hist[w][tid] += tile_start;
  }
  __syncthreads();

  // Stage keys in digit order (the match masks are dead now).
  Bits *stage_keys = reinterpret_cast<Bits *>(stage_raw);
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const bool valid = wave_base + size_t(j) * 64 + lane < n;
    if (valid) {
      const uint32_t d = digit_of(key[j], flags, bit, mask);
      rank[j] += whist[d];
      stage_keys[rank[j]] = key[j];
    }
  }

  // Decoupled look-back, one thread per digit.
  if (tid < BINS) {
    Desc excl = 0;
    if (tile > 0) {
      uint32_t t = tile - 1;
      while (true) {
        Desc v = load_agent(&lookback[size_t(t) * BINS + tid]);
        Desc flag = v >> DI::SHIFT;
        if (flag == 0) {
          __builtin_amdgcn_s_sleep(1);
          continue;
        }
        excl += v & DI::MASK;
        if (flag == (DI::INCL >> DI::SHIFT)) break;
        --t;
      }
      store_agent(&lookback[size_t(tile) * BINS + tid],
                  static_cast<Desc>(DI::INCL | (excl + Desc(count))));
    }
    digit_off[tid] = bin_start + static_cast<uint32_t>(excl) - tile_start;
  }
  __syncthreads();

  // Coalesced scatter: consecutive staged keys of one digit go to
  // consecutive output positions.
  const uint32_t valid_count = static_cast<uint32_t>(min<size_t>(TILE, n - tile_base));
  uint32_t dst[PAIRS ? ITEMS : 1];
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const uint32_t i = uint32_t(k) * THREADS + tid;
    if (i < valid_count) {
      Bits kk = stage_keys[i];
      uint32_t p = digit_off[digit_of(kk, flags, bit, mask)] + i;
      keys_out[p] = kk;
      if constexpr (PAIRS) dst[k] = p;
    }
  }
  if constexpr (PAIRS) {
    __syncthreads();
    Val *stage_vals = reinterpret_cast<Val *>(stage_raw);
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const bool valid = wave_base + size_t(j) * 64 + lane < n;
      if (valid) stage_vals[rank[j]] = val[j];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t i = uint32_t(k) * THREADS + tid;
      if (i < valid_count) vals_out[dst[k]] = stage_vals[i];
    }
  }
  if (tid < BINS && lookback_next) lookback_next[size_t(tile) * BINS + tid] = 0;
}

} // namespace radix
} // namespace rccl_hip

// ===========================================================================
// Host pass control (rccl-cub/src/radix.rs:427-876 behaviour).
// ===========================================================================
namespace rccl_hip {
namespace radix {

constexpr int THREADS = 512;

constexpr int items_for(size_t elem_bytes) {
  return elem_bytes <= 4 ? 16 : (elem_bytes <= 8 ? 12 : 8);
}
constexpr size_t stage_elem(size_t key_bytes, size_t value_bytes) {
  return key_bytes > value_bytes ? key_bytes : value_bytes;
}
inline size_t tile_items(size_t key_bytes, size_t value_bytes) {
  return size_t(THREADS) * items_for(stage_elem(key_bytes, value_bytes));
}

// Largest item count the control words support: 30-bit look-back counts
// switch to 62-bit descriptors at 2^30; positions are 32-bit.
constexpr uint64_t MAX_ITEMS = 0xffffffffull;

struct Layout {
  size_t tiles = 0;
  size_t desc_bytes = 4;
  size_t bins = 0, counters = 0, lb0 = 0, lb1 = 0, total = 0;
};

inline Layout layout(size_t key_bytes, size_t value_bytes, size_t n) {
  Layout l;
  const size_t max_passes = key_bytes;  // 8-bit digits
  l.tiles = (n + tile_items(key_bytes, value_bytes) - 1) / tile_items(key_bytes, value_bytes);
  l.desc_bytes = n < (size_t(1) << 30) ? 4 : 8;
  size_t off = 0;
  l.bins = off;
  off += align_up(max_passes * BINS * sizeof(uint32_t), 256);
  l.counters = off;
  off += align_up(max_passes * sizeof(uint32_t), 256);
  l.lb0 = off;
  off += align_up(l.tiles * BINS * l.desc_bytes, 256);
  l.lb1 = off;
  off += align_up(l.tiles * BINS * l.desc_bytes, 256);
  l.total = n == 0 ? 0 : off;
  return l;
}

inline uint32_t key_flags(rccl_hip_key_kind k, rccl_hip_order order) {
  uint32_t f = 0;
  if (k == RCCL_HIP_KEY_I32 || k == RCCL_HIP_KEY_I64) f |= KF_SIGNED;
  if (k == RCCL_HIP_KEY_F32 || k == RCCL_HIP_KEY_F64) f |= KF_FLOAT;
  if (order == RCCL_HIP_ORDER_DESCENDING) f |= KF_DESC;
  return f;
}

struct SortArgs {
  void *keys[2];
  void *vals[2];
  size_t n;
  int cur;  // index of the buffer holding the input
  uint32_t begin_bit, end_bit, flags;
  unsigned char *ws;
  hipStream_t stream;
};

template <class Bits, class Val, class Desc>
rccl_hip_status run_passes(SortArgs &a, const Layout &l, uint32_t passes) {
  constexpr int ITEMS = items_for(stage_elem(sizeof(Bits), std::is_same<Val, NoValue>::value ? 0 : sizeof(Val)));
  uint32_t *bins = reinterpret_cast<uint32_t *>(a.ws + l.bins);
  uint32_t *counters = reinterpret_cast<uint32_t *>(a.ws + l.counters);
  Desc *lb[2] = {reinterpret_cast<Desc *>(a.ws + l.lb0), reinterpret_cast<Desc *>(a.ws + l.lb1)};

  init_kernel<<<1, 256, 0, a.stream>>>(bins, counters, passes);
  RCCL_HIP_TRY(check_launch("radix init"));

  const size_t chunk = size_t(HIST_THREADS) * HIST_ITEMS;
  size_t hist_blocks = std::min<size_t>((a.n + chunk - 1) / chunk, 2048);
  const size_t zero_words = l.tiles * BINS * sizeof(Desc) / sizeof(uint32_t);
  hist_blocks = std::max<size_t>(hist_blocks, 1);
  histogram_kernel<Bits><<<dim3(static_cast<uint32_t>(hist_blocks)), HIST_THREADS, 0, a.stream>>>(
      static_cast<const Bits *>(a.keys[a.cur]), a.n, bins, a.flags, a.begin_bit, a.end_bit, passes,
      reinterpret_cast<uint32_t *>(lb[0]), zero_words);
  RCCL_HIP_TRY(check_launch("radix histogram"));

  for (uint32_t p = 0; p < passes; ++p) {
    const uint32_t bit = a.begin_bit + 8u * p;
    const uint32_t width = std::min(8u, a.end_bit - bit);
    const uint32_t mask = (1u << width) - 1u;
    const int in = a.cur, out = 1 - a.cur;
    onesweep_kernel<Bits, Val, THREADS, ITEMS, Desc>
        <<<dim3(static_cast<uint32_t>(l.tiles)), THREADS, 0, a.stream>>>(
            static_cast<const Bits *>(a.keys[in]), static_cast<Bits *>(a.keys[out]),
            static_cast<const Val *>(a.vals[in]), static_cast<Val *>(a.vals[out]), a.n,
            bins + size_t(p) * BINS, lb[p & 1], p + 1 < passes ? lb[(p + 1) & 1] : nullptr,
            counters + p, a.flags, bit, mask);
    RCCL_HIP_TRY(check_launch("radix onesweep"));
    a.cur = out;
  }
  return ok();
}

template <class Bits, class Val>
rccl_hip_status run_typed(SortArgs &a, const Layout &l, uint32_t passes) {
  if (l.desc_bytes == 4) return run_passes<Bits, Val, uint32_t>(a, l, passes);
  return run_passes<Bits, Val, uint64_t>(a, l, passes);
}

template <class Bits>
rccl_hip_status run_values(SortArgs &a, size_t value_bytes, const Layout &l, uint32_t passes) {
  switch (value_bytes) {
  case 0: return run_typed<Bits, NoValue>(a, l, passes);
  case 1: return run_typed<Bits, uint8_t>(a, l, passes);
  case 2: return run_typed<Bits, uint16_t>(a, l, passes);
  case 4: return run_typed<Bits, uint32_t>(a, l, passes);
  case 8: return run_typed<Bits, uint64_t>(a, l, passes);
  case 16: return run_typed<Bits, Value16>(a, l, passes);
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix value bytes");
}

inline bool radix_kind(rccl_hip_key_kind k) {
  return k >= RCCL_HIP_KEY_U32 && k <= RCCL_HIP_KEY_F64;
}

// Shared validation + launch for both ABI entry points.
rccl_hip_status sort_buffer(rccl_hip_key_kind key, size_t value_bytes, rccl_hip_order order,
                            SortArgs &a, size_t workspace_bytes) {
  if (!radix_kind(key)) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix key kind");
  if (!valid_value_bytes(value_bytes))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix value bytes");
  if (order != RCCL_HIP_ORDER_ASCENDING && order != RCCL_HIP_ORDER_DESCENDING)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix order");
  const uint32_t key_bits = static_cast<uint32_t>(key_bytes(key) * 8);
  // rccl-cub/src/radix.rs:370-376
  if (a.begin_bit > a.end_bit || a.end_bit > key_bits)
    return set_bit_range_error(a.begin_bit, a.end_bit, key_bits);
  if (a.n > MAX_ITEMS) return set_error(RCCL_HIP_ERROR_LENGTH_MISMATCH, "radix item count", MAX_ITEMS, a.n);
  const uint32_t passes = (a.end_bit - a.begin_bit + 7u) / 8u;
  // rccl-cub/src/radix.rs:467-469: empty input or window is a no-op.
  if (a.n == 0 || passes == 0) return ok();
  if (!a.keys[0] || !a.keys[1]) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix keys");
  if (value_bytes && (!a.vals[0] || !a.vals[1]))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix values");
  const Layout l = layout(key_bytes(key), value_bytes, a.n);
  if (!a.ws || workspace_bytes < l.total)
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "radix workspace", l.total, workspace_bytes);
  a.flags = key_flags(key, order);
  if (key_bytes(key) == 4) return run_values<uint32_t>(a, value_bytes, l, passes);
  return run_values<uint64_t>(a, value_bytes, l, passes);
}

} // namespace radix
} // namespace rccl_hip

using namespace rccl_hip;

extern "C" {

rccl_hip_status rccl_hip_radix_sort_workspace_bytes(rccl_hip_key_kind key, size_t value_bytes,
                                                    size_t n, size_t *bytes) {
  if (!bytes) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "bytes");
  if (!radix::radix_kind(key)) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix key kind");
  if (!valid_value_bytes(value_bytes))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix value bytes");
  if (n > radix::MAX_ITEMS)
    return set_error(RCCL_HIP_ERROR_LENGTH_MISMATCH, "radix item count", radix::MAX_ITEMS, n);
  *bytes = radix::layout(key_bytes(key), value_bytes, n).total;
  return ok();
}

rccl_hip_status rccl_hip_radix_sort_buffer(rccl_hip_key_kind key, size_t value_bytes,
                                           rccl_hip_order order, void *keys_first,
                                           void *keys_second, void *values_first,
                                           void *values_second, size_t n,
                                           int *current_is_first, uint32_t begin_bit,
                                           uint32_t end_bit, void *workspace,
                                           size_t workspace_bytes, hipStream_t stream) {
  if (!current_is_first) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "current_is_first");
  radix::SortArgs a{};
  a.keys[0] = keys_first;
  a.keys[1] = keys_second;
  a.vals[0] = values_first;
  a.vals[1] = values_second;
  a.n = n;
  a.cur = *current_is_first ? 0 : 1;
  a.begin_bit = begin_bit;
  a.end_bit = end_bit;
  a.ws = static_cast<unsigned char *>(workspace);
  a.stream = stream;
  RCCL_HIP_TRY(radix::sort_buffer(key, value_bytes, order, a, workspace_bytes));
  *current_is_first = a.cur == 0 ? 1 : 0;
  return ok();
}

rccl_hip_status rccl_hip_radix_sort(rccl_hip_key_kind key, size_t value_bytes,
                                    rccl_hip_order order, void *keys, void *values,
                                    void *scratch_keys, void *scratch_values, size_t n,
                                    void *workspace, size_t workspace_bytes, hipStream_t stream) {
  radix::SortArgs a{};
  a.keys[0] = keys;
  a.keys[1] = scratch_keys;
  a.vals[0] = values;
  a.vals[1] = scratch_values;
  a.n = n;
  a.cur = 0;
  a.begin_bit = 0;
  a.end_bit = static_cast<uint32_t>(key_bytes(key) * 8);
  a.ws = static_cast<unsigned char *>(workspace);
  a.stream = stream;
  RCCL_HIP_TRY(radix::sort_buffer(key, value_bytes, order, a, workspace_bytes));
  // rccl-cub/src/radix.rs:617-621: copy back when the result is in scratch.
  if (a.cur == 1) {
    hipError_t err = hipMemcpyAsync(keys, scratch_keys, n * key_bytes(key),
                                    hipMemcpyDeviceToDevice, stream);
    if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_MEMORY, "radix copy back", err);
    if (value_bytes) {
      err = hipMemcpyAsync(values, scratch_values, n * value_bytes, hipMemcpyDeviceToDevice, stream);
      if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_MEMORY, "radix copy back", err);
    }
  }
  return ok();
}

} // extern "C"
