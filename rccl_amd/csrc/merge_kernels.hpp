// DeviceMerge for gfx950: merge-path partitioned stable merge.
//
// Reference behaviour: rccl-cub/src/merge.rs:194-368 (host control) and
// rccl-cub/src/ordering_backend/merge.rs:16-297,308-391 (tile agents). Design:
//   partition  one thread per tile boundary: a merge-path binary search in
//              HBM gives the A/B split of that output diagonal
//   merge      one block per output tile: the tile's A and B slices are
//              staged in LDS with striped (coalesced) loads; every thread
//              finds its own split by a merge-path search in LDS and merges
//              ITEMS outputs serially (B only when strictly before A); keys
//              and values leave through a padded LDS blocked->striped
//              transpose so the HBM stores coalesce.
// The merge tile routine is shared with the merge sort passes.
#pragma once

#include <algorithm>

#include "ordering_common.hpp"

namespace rccl_hip {
namespace merge {

using ordering::NoValue;

// Tile policy: 256 threads; items per thread by key + value bytes.
// Overridable at build time for tuning.
#ifndef RCCL_MERGE_THREADS
#define RCCL_MERGE_THREADS 256
#endif
#ifndef RCCL_MERGE_ITEMS_4B
#define RCCL_MERGE_ITEMS_4B 16
#endif
#ifndef RCCL_MERGE_ITEMS_8B
#define RCCL_MERGE_ITEMS_8B 12
#endif
constexpr int THREADS = RCCL_MERGE_THREADS;

template <class K, class V>
constexpr int items_for() {
  constexpr size_t bytes = sizeof(K) + (std::is_same<V, NoValue>::value ? 0 : sizeof(V));
  return bytes <= 4 ? RCCL_MERGE_ITEMS_4B
                    : (bytes <= 8 ? RCCL_MERGE_ITEMS_8B : (bytes <= 16 ? 8 : 6));
}

template <class K, class V>
constexpr size_t tile_items() {
  return size_t(THREADS) * items_for<K, V>();
}

// DeviceMerge's own tile (the merge sort keeps items_for, whose larger block
// tiles save it passes): with the sampled partition a tile boundary costs
// little, and shorter serial merges per thread keep more blocks per CU busy.
#ifndef RCCL_MERGE_CALL_ITEMS_4B
#define RCCL_MERGE_CALL_ITEMS_4B 16
#endif
#ifndef RCCL_MERGE_CALL_ITEMS_8B
#define RCCL_MERGE_CALL_ITEMS_8B 8
#endif
#ifndef RCCL_MERGE_CALL_ITEMS_16B
#define RCCL_MERGE_CALL_ITEMS_16B 6
#endif
template <class K, class V>
constexpr int call_items_for() {
  constexpr size_t bytes = sizeof(K) + (std::is_same<V, NoValue>::value ? 0 : sizeof(V));
  return bytes <= 4 ? RCCL_MERGE_CALL_ITEMS_4B
                    : (bytes <= 8 ? RCCL_MERGE_CALL_ITEMS_8B
                                  : (bytes <= 16 ? RCCL_MERGE_CALL_ITEMS_16B : 4));
}
template <class K, class V>
constexpr size_t call_tile_items() {
  return size_t(THREADS) * call_items_for<K, V>();
}
// Keys-only merges of 4-byte keys up to RCCL_MERGE_SHORT_TOTAL outputs use
// shorter tiles (more blocks in flight): 2 x 2^23 u32 keys 0.0541 -> 0.0483 ms
// at 12 items, while 2 x 2^27 keys are fastest at 16 (0.585 against 0.605 ms).
#ifndef RCCL_MERGE_SHORT_ITEMS_4B
#define RCCL_MERGE_SHORT_ITEMS_4B 12
#endif
#ifndef RCCL_MERGE_SHORT_TOTAL
#define RCCL_MERGE_SHORT_TOTAL (size_t(1) << 24)
#endif
template <class K, class V>
constexpr bool short_tiles_for() {
  return std::is_same<V, NoValue>::value && sizeof(K) == 4 &&
         RCCL_MERGE_SHORT_ITEMS_4B != RCCL_MERGE_CALL_ITEMS_4B;
}
template <class K, class V>
constexpr bool short_tiles(size_t total) {
  return short_tiles_for<K, V>() && total <= RCCL_MERGE_SHORT_TOTAL;
}
template <class K, class V>
constexpr size_t call_tile_items(size_t total) {
  return short_tiles<K, V>(total) ? size_t(THREADS) * RCCL_MERGE_SHORT_ITEMS_4B
                                  : call_tile_items<K, V>();
}

// Splits for tile boundaries 0..tiles: splits[t] = A items among the first
// min(t * tile, na + nb) merged outputs.
template <class K, class Cmp>
__global__ void __launch_bounds__(256)
partition_kernel(const K *__restrict__ a, size_t na, const K *__restrict__ b, size_t nb,
                 size_t tile, size_t count, uint64_t *__restrict__ splits) {
  const size_t t = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= count) return;
  const size_t diag = std::min(t * tile, na + nb);
  splits[t] = ordering::merge_path<K>([&](size_t i) { return a[i]; }, na,
                                      [&](size_t j) { return b[j]; }, nb, diag, Cmp{});
}

// Sampled partition (integer keys, from SAMPLED_MIN_TILES tiles):
// ordering::merge_sample_kernel, then each tile boundary's split from
// ordering::sampled_merge_path.
constexpr size_t SAMPLED_MIN_TILES = 512;

template <class K, class Cmp>
__global__ void __launch_bounds__(256)
sampled_partition_kernel(const K *__restrict__ a, size_t na, const K *__restrict__ b, size_t nb,
                         size_t tile, size_t count, const uint32_t *__restrict__ m,
                         uint64_t *__restrict__ splits) {
  const size_t t = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= count) return;
  const size_t d = std::min(t * tile, na + nb);
  splits[t] = ordering::sampled_merge_path<K>([&](size_t x) { return a[x]; }, na,
                                              [&](size_t x) { return b[x]; }, nb, d, m, Cmp{});
}

// LDS layout of one merge tile.
template <class K, class V, int ITEMS>
struct MergeSmem {
  static constexpr uint32_t TILE = THREADS * ITEMS;
  static constexpr bool PAIRS = !std::is_same<V, NoValue>::value;
  K keys[ordering::padded_size(TILE, ITEMS)];
  typename std::conditional<PAIRS, V, char>::type
      vals[PAIRS ? ordering::padded_size(TILE, ITEMS) : 1];
};

// Merge the tile whose A slice is a[i0, i1) and B slice is b[j0, j1) into
// out[o0, o0 + (i1 - i0) + (j1 - j0)). Values follow their keys.
template <class K, class V, class Cmp, int ITEMS>
__device__ __forceinline__ void merge_tile(MergeSmem<K, V, ITEMS> &sm, const K *__restrict__ a,
                                           const V *__restrict__ av, size_t i0, size_t i1,
                                           const K *__restrict__ b, const V *__restrict__ bv,
                                           size_t j0, size_t j1, K *__restrict__ out,
                                           V *__restrict__ outv, size_t o0) {
  constexpr bool PAIRS = MergeSmem<K, V, ITEMS>::PAIRS;
  const uint32_t tid = threadIdx.x;
  const uint32_t la = static_cast<uint32_t>(i1 - i0);
  const uint32_t lb = static_cast<uint32_t>(j1 - j0);
  const uint32_t len = la + lb;
  const Cmp less{};

  // Stage A then B keys (and values), striped for coalescing.
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const uint32_t i = uint32_t(k) * THREADS + tid;
    if (i < len) {
      sm.keys[i] = i < la ? a[i0 + i] : b[j0 + (i - la)];
      if constexpr (PAIRS) sm.vals[i] = i < la ? av[i0 + i] : bv[j0 + (i - la)];
    }
  }
  __syncthreads();

  // This thread's outputs [d, d + ITEMS) of the tile.
  const uint32_t d = min(tid * uint32_t(ITEMS), len);
  uint32_t ia = ordering::merge_path_lds<K>(sm.keys, la, sm.keys + la, lb, d, less);
  uint32_t ib = d - ia;
  K outk[ITEMS];
  uint32_t src[PAIRS ? ITEMS : 1];
  if constexpr (ordering::use_merge_network<K, V, ITEMS>()) {
    const K last = Cmp::last();
    ordering::network_merge<K, Cmp, ITEMS>(
        outk, [&](int i) { return ia + i < la ? sm.keys[ia + i] : last; },
        [&](int i) { return ib + i < lb ? sm.keys[la + ib + i] : last; }, less);
  } else {
    using ordering::pick;
    K ka = ia < la ? sm.keys[ia] : K{};
    K kb = ib < lb ? sm.keys[la + ib] : K{};
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const bool take_b = ib < lb && (ia >= la || less(kb, ka));
      outk[k] = pick(take_b, kb, ka);
      if constexpr (PAIRS) src[k] = take_b ? la + ib : ia;
      if (take_b) {
        ++ib;
        if (ib < lb) kb = sm.keys[la + ib];
      } else {
        ++ia;
        if (ia < la) ka = sm.keys[ia];
      }
    }
  }
  V outv_reg[PAIRS ? ITEMS : 1];
  if constexpr (PAIRS) {
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) outv_reg[k] = sm.vals[min(src[k], len ? len - 1 : 0u)];
  }
  __syncthreads();

  // Blocked -> striped through padded LDS, then coalesced stores.
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const uint32_t i = tid * uint32_t(ITEMS) + k;
    sm.keys[ordering::padded<ITEMS>(i)] = outk[k];
    if constexpr (PAIRS) sm.vals[ordering::padded<ITEMS>(i)] = outv_reg[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const uint32_t i = uint32_t(k) * THREADS + tid;
    if (i < len) {
      out[o0 + i] = sm.keys[ordering::padded<ITEMS>(i)];
      if constexpr (PAIRS) outv[o0 + i] = sm.vals[ordering::padded<ITEMS>(i)];
    }
  }
}

template <class K, class V, class Cmp, int ITEMS>
__global__ void __launch_bounds__(THREADS)
merge_kernel(const K *__restrict__ a, const V *__restrict__ av, size_t na, const K *__restrict__ b,
             const V *__restrict__ bv, size_t nb, K *__restrict__ out, V *__restrict__ outv,
             const uint64_t *__restrict__ splits) {
  __shared__ MergeSmem<K, V, ITEMS> sm;
  constexpr size_t TILE = size_t(THREADS) * ITEMS;
  const size_t t = blockIdx.x;
  const size_t o0 = t * TILE;
  const size_t o1 = std::min(o0 + TILE, na + nb);
  const size_t i0 = splits[t], i1 = splits[t + 1];
  merge_tile<K, V, Cmp, ITEMS>(sm, a, av, i0, i1, b, bv, o0 - i0, o1 - i1, out, outv, o0);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct MergeArgs {
  const void *a, *av, *b, *bv;
  size_t na, nb;
  void *out, *outv;
  void *ws;
  size_t ws_bytes;
  hipStream_t stream;
};

// The sampled partition serves merges of at least SAMPLED_MIN_TILES tiles.
template <class K, class V>
bool use_sampled(size_t na, size_t nb) {
  const size_t tile = call_tile_items<K, V>(na + nb);
  const size_t tiles = (na + nb + tile - 1) / tile;
  return ordering::sampled_partition_for<K>() && na > 0 && nb > 0 && tiles >= SAMPLED_MIN_TILES;
}

// Splits (one u64 per tile boundary), then the samples' m_k (one u32 per
// MERGE_SAMPLE items of A) when the sampled partition runs.
template <class K, class V>
size_t workspace_bytes(size_t na, size_t nb) {
  const size_t total = na + nb;
  if (total == 0) return 0;
  const size_t tile = call_tile_items<K, V>(total);
  const size_t tiles = (total + tile - 1) / tile;
  size_t bytes = align_up((tiles + 1) * sizeof(uint64_t), 256);
  if (use_sampled<K, V>(na, nb)) bytes += align_up(ordering::merge_samples(na) * 4, 256);
  return bytes;
}

template <class K, class V, class Cmp, int ITEMS>
rccl_hip_status run_merge_shape(const MergeArgs &m) {
  constexpr size_t TILE = size_t(THREADS) * ITEMS;
  const size_t total = m.na + m.nb;
  const size_t need = workspace_bytes<K, V>(m.na, m.nb);
  if (!m.ws || m.ws_bytes < need)
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "merge workspace", need, m.ws_bytes);
  const size_t tiles = (total + TILE - 1) / TILE;
  uint64_t *splits = static_cast<uint64_t *>(m.ws);
  const dim3 pgrid(static_cast<uint32_t>((tiles + 1 + 255) / 256));
  if (use_sampled<K, V>(m.na, m.nb)) {
    uint32_t *samples = reinterpret_cast<uint32_t *>(static_cast<unsigned char *>(m.ws) +
                                                     align_up((tiles + 1) * sizeof(uint64_t), 256));
    const size_t ka = ordering::merge_samples(m.na);
    {
      KernelTimer t("merge_sample", m.stream, ka);
      ordering::merge_sample_kernel<K, Cmp>
          <<<dim3(static_cast<uint32_t>(ordering::merge_sample_blocks(m.na))), 256, 0,
             m.stream>>>(static_cast<const K *>(m.a), m.na, static_cast<const K *>(m.b), m.nb,
                         samples);
    }
    RCCL_HIP_TRY(check_launch("merge sample"));
    KernelTimer t("merge_partition", m.stream, tiles + 1);
    sampled_partition_kernel<K, Cmp><<<pgrid, 256, 0, m.stream>>>(
        static_cast<const K *>(m.a), m.na, static_cast<const K *>(m.b), m.nb, TILE, tiles + 1,
        samples, splits);
  } else {
    KernelTimer t("merge_partition", m.stream, tiles + 1);
    partition_kernel<K, Cmp><<<pgrid, 256, 0, m.stream>>>(static_cast<const K *>(m.a), m.na,
                                                          static_cast<const K *>(m.b), m.nb, TILE,
                                                          tiles + 1, splits);
  }
  RCCL_HIP_TRY(check_launch("merge partition"));
  {
    KernelTimer t("merge", m.stream, total);
    merge_kernel<K, V, Cmp, ITEMS><<<dim3(static_cast<uint32_t>(tiles)), THREADS, 0, m.stream>>>(
        static_cast<const K *>(m.a), static_cast<const V *>(m.av), m.na,
        static_cast<const K *>(m.b), static_cast<const V *>(m.bv), m.nb, static_cast<K *>(m.out),
        static_cast<V *>(m.outv), splits);
  }
  return check_launch("merge");
}

template <class K, class V, class Cmp>
rccl_hip_status run_merge(const MergeArgs &m) {
  const size_t total = m.na + m.nb;
  if (total == 0) return ok();
  if constexpr (short_tiles_for<K, V>()) {
    if (short_tiles<K, V>(total)) return run_merge_shape<K, V, Cmp, RCCL_MERGE_SHORT_ITEMS_4B>(m);
  }
  return run_merge_shape<K, V, Cmp, call_items_for<K, V>()>(m);
}

// Per key kind entry points (one translation unit each).
#define RCCL_MERGE_DECLARE_KIND(NAME)                                                   \
  rccl_hip_status run_##NAME(const MergeArgs &m, size_t value_bytes, bool descending);  \
  size_t bytes_##NAME(size_t na, size_t nb, size_t value_bytes);
RCCL_MERGE_DECLARE_KIND(u8)
RCCL_MERGE_DECLARE_KIND(i8)
RCCL_MERGE_DECLARE_KIND(u16)
RCCL_MERGE_DECLARE_KIND(i16)
RCCL_MERGE_DECLARE_KIND(u32)
RCCL_MERGE_DECLARE_KIND(i32)
RCCL_MERGE_DECLARE_KIND(f32)
RCCL_MERGE_DECLARE_KIND(u64)
RCCL_MERGE_DECLARE_KIND(i64)
RCCL_MERGE_DECLARE_KIND(f64)
#undef RCCL_MERGE_DECLARE_KIND

template <class K, bool DESC>
struct KindRunner {
  template <class V>
  static rccl_hip_status run(const MergeArgs &m) {
    return run_merge<K, V, ordering::Less<K, DESC>>(m);
  }
};

template <class V, class K>
size_t bytes_v(size_t na, size_t nb) {
  return workspace_bytes<K, V>(na, nb);
}

#define RCCL_MERGE_DEFINE_KIND(NAME, KT)                                                  \
  rccl_hip_status run_##NAME(const MergeArgs &m, size_t value_bytes, bool descending) {   \
    using Desc = KindRunner<KT, true>;                                                    \
    using Asc = KindRunner<KT, false>;                                                    \
    if (descending) {                                                                     \
      RCCL_ORDERING_DISPATCH_VALUE(value_bytes, Desc, m)                                  \
    } else {                                                                              \
      RCCL_ORDERING_DISPATCH_VALUE(value_bytes, Asc, m)                                   \
    }                                                                                     \
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge value bytes");               \
  }                                                                                       \
  size_t bytes_##NAME(size_t na, size_t nb, size_t value_bytes) {                         \
    switch (value_bytes) {                                                                \
    case 0: return bytes_v<ordering::NoValue, KT>(na, nb);                                \
    case 1: return bytes_v<uint8_t, KT>(na, nb);                                          \
    case 2: return bytes_v<uint16_t, KT>(na, nb);                                         \
    case 4: return bytes_v<uint32_t, KT>(na, nb);                                         \
    case 8: return bytes_v<uint64_t, KT>(na, nb);                                         \
    default: return bytes_v<Value16, KT>(na, nb);                                         \
    }                                                                                     \
  }

} // namespace merge
} // namespace rccl_hip
