// DeviceMergeSort for gfx950: block sort + merge-path merge passes.
//
// Reference behaviour: rccl-cub/src/merge_sort.rs:140-690 (pass control) and
// rccl-cub/src/ordering_backend/merge.rs:399-1846 (block sort, partition,
// merge agents). Design:
//   block_sort   one block per tile of BT*ITEMS keys: each thread sorts
//                its items in registers (stable odd-even transposition),
//                then log2(BT) merge-path rounds in padded LDS double
//                the sorted runs; source indices travel with the keys so
//                values are gathered once at the end
//   partition    per output tile of a merge pass: the pair of runs it lies
//                in and its merge-path split (binary search in HBM)
//   merge        the DeviceMerge tile routine on (run 2p, run 2p + 1)
// Passes ping-pong between the output and a scratch buffer so that the last
// pass writes the output; everything is stable (left run first on ties).
#pragma once

#include "merge_kernels.hpp"

namespace rccl_hip {
namespace merge_sort {

using ordering::NoValue;
constexpr int THREADS = merge::THREADS;

template <class K, class V>
constexpr int items_for() {
  return merge::items_for<K, V>();
}
template <class K, class V>
constexpr size_t tile_items() {
  return merge::tile_items<K, V>();
}

// Block sort threads: keys-only sorts of keys up to 4 bytes sort bigger
// blocks (fewer merge passes); others use the merge tile. A multiple of
// THREADS, so that every merge pass's pairs of runs hold whole merge tiles.
#ifndef RCCL_MERGE_SORT_BLOCK_THREADS_4B
#define RCCL_MERGE_SORT_BLOCK_THREADS_4B 1024
#endif
template <class K, class V>
constexpr int block_threads() {
  return (std::is_same<V, NoValue>::value && sizeof(K) <= 4) ? RCCL_MERGE_SORT_BLOCK_THREADS_4B
                                                            : THREADS;
}
template <class K, class V>
constexpr size_t block_tile_items() {
  return size_t(block_threads<K, V>()) * items_for<K, V>();
}

template <class K, class V, int ITEMS, int BT>
struct BlockSortSmem {
  static constexpr uint32_t TILE = BT * ITEMS;
  static constexpr bool PAIRS = !std::is_same<V, NoValue>::value;
  K keys[ordering::padded_size(TILE, ITEMS)];
  uint16_t idx[PAIRS ? ordering::padded_size(TILE, ITEMS) : 1];
  typename std::conditional<PAIRS, V, char>::type vals[PAIRS ? TILE : 1];
};

template <class K, class V, class Cmp, int ITEMS, int BT>
__global__ void __launch_bounds__(BT)
block_sort_kernel(const K *__restrict__ in, const V *__restrict__ in_v, size_t n,
                  K *__restrict__ out, V *__restrict__ out_v) {
  constexpr int THREADS = BT;
  using Smem = BlockSortSmem<K, V, ITEMS, BT>;
  constexpr bool PAIRS = Smem::PAIRS;
  constexpr uint32_t TILE = Smem::TILE;
  static_assert(TILE <= 65536, "source indices are 16-bit");
  __shared__ Smem sm;
  const Cmp less{};
  const uint32_t tid = threadIdx.x;
  const size_t base = size_t(blockIdx.x) * TILE;
  const uint32_t len = static_cast<uint32_t>(min<size_t>(TILE, n - base));

#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const uint32_t i = uint32_t(k) * THREADS + tid;
    if (i < len) {
      sm.keys[ordering::padded<ITEMS>(i)] = in[base + i];
      if constexpr (PAIRS) sm.vals[i] = in_v[base + i];
    }
  }
  __syncthreads();

  // Stable sort of this thread's blocked items in registers.
  const uint32_t first = tid * uint32_t(ITEMS);
  const uint32_t cnt = first < len ? min(uint32_t(ITEMS), len - first) : 0u;
  K key[ITEMS];
  uint32_t idx[ITEMS];
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    key[k] = uint32_t(k) < cnt ? sm.keys[ordering::padded<ITEMS>(first + k)] : K{};
    idx[k] = first + k;
  }
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
#pragma unroll
    for (int j = r & 1; j + 1 < ITEMS; j += 2) {
      if (uint32_t(j + 1) < cnt && less(key[j + 1], key[j])) {
        const K tk = key[j];
        key[j] = key[j + 1];
        key[j + 1] = tk;
        const uint32_t ti = idx[j];
        idx[j] = idx[j + 1];
        idx[j + 1] = ti;
      }
    }
  }

  // Merge rounds: runs of `w` items become runs of 2w. Source indices are
  // tracked for pairs only; keys-only sorts of integer keys merge with a
  // network.
  constexpr bool NETWORK = ordering::use_merge_network<K, V, ITEMS>();
  for (uint32_t w = ITEMS; w < TILE; w *= 2) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      sm.keys[ordering::padded<ITEMS>(first + k)] = key[k];
      if constexpr (PAIRS)
        sm.idx[ordering::padded<ITEMS>(first + k)] = static_cast<uint16_t>(idx[k]);
    }
    __syncthreads();
    const uint32_t g = first / (2 * w) * (2 * w);
    const uint32_t a0 = min(g, len), a1 = min(g + w, len);
    const uint32_t b0 = a1, b1 = min(g + 2 * w, len);
    const uint32_t la = a1 - a0, lb = b1 - b0;
    const uint32_t d = min(first - g, la + lb);
    // Merge path over the padded LDS runs.
    uint32_t lo = d > lb ? d - lb : 0u, hi = min(d, la);
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      if (less(sm.keys[ordering::padded<ITEMS>(b0 + d - 1 - mid)],
               sm.keys[ordering::padded<ITEMS>(a0 + mid)]))
        hi = mid;
      else
        lo = mid + 1;
    }
    uint32_t ia = lo, ib = d - lo;
    if constexpr (NETWORK) {
      const K last = Cmp::last();
      ordering::network_merge<K, Cmp, ITEMS>(
          key,
          [&](int i) {
            return ia + i < la ? sm.keys[ordering::padded<ITEMS>(a0 + ia + i)] : last;
          },
          [&](int i) {
            return ib + i < lb ? sm.keys[ordering::padded<ITEMS>(b0 + ib + i)] : last;
          },
          less);
      continue;
    }
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const bool a_ok = ia < la, b_ok = ib < lb;
      const uint32_t pa = ordering::padded<ITEMS>(a0 + min(ia, la ? la - 1 : 0u));
      const uint32_t pb = ordering::padded<ITEMS>(b0 + min(ib, lb ? lb - 1 : 0u));
      const K ka = sm.keys[pa], kb = sm.keys[pb];
      const bool take_b = b_ok && (!a_ok || less(kb, ka));
      key[k] = take_b ? kb : ka;
      if constexpr (PAIRS) idx[k] = take_b ? sm.idx[pb] : sm.idx[pa];
      ib += take_b ? 1u : 0u;
      ia += take_b ? 0u : 1u;
    }
  }

  // Blocked -> striped and store (values gathered by source index).
  __syncthreads();
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    sm.keys[ordering::padded<ITEMS>(first + k)] = key[k];
    if constexpr (PAIRS) sm.idx[ordering::padded<ITEMS>(first + k)] = static_cast<uint16_t>(idx[k]);
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const uint32_t i = uint32_t(k) * THREADS + tid;
    if (i < len) {
      out[base + i] = sm.keys[ordering::padded<ITEMS>(i)];
      if constexpr (PAIRS) out_v[base + i] = sm.vals[sm.idx[ordering::padded<ITEMS>(i)]];
    }
  }
}

// Split of every output tile of one merge pass (runs of `run` items).
template <class K, class Cmp>
__global__ void __launch_bounds__(256)
pass_partition_kernel(const K *__restrict__ src, size_t n, size_t run, size_t tile, size_t tiles,
                      uint64_t *__restrict__ splits) {
  const size_t t = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= tiles) return;
  const size_t o = t * tile;
  const size_t pair_start = o / (2 * run) * (2 * run);
  const size_t na = min(run, n - pair_start);
  const size_t nb = n - pair_start > run ? min(run, n - pair_start - run) : 0;
  const K *a = src + pair_start;
  const K *b = a + na;
  splits[t] = ordering::merge_path<K>([&](size_t i) { return a[i]; }, na,
                                      [&](size_t j) { return b[j]; }, nb, o - pair_start, Cmp{});
}

template <class K, class V, class Cmp, int ITEMS>
__global__ void __launch_bounds__(THREADS)
pass_merge_kernel(const K *__restrict__ src, const V *__restrict__ src_v, size_t n, size_t run,
                  K *__restrict__ dst, V *__restrict__ dst_v, const uint64_t *__restrict__ splits) {
  __shared__ merge::MergeSmem<K, V, ITEMS> sm;
  constexpr size_t TILE = size_t(THREADS) * ITEMS;
  const size_t t = blockIdx.x;
  const size_t o0 = t * TILE;
  const size_t o1 = min(o0 + TILE, n);
  const size_t pair_start = o0 / (2 * run) * (2 * run);
  const size_t na = min(run, n - pair_start);
  const size_t nb = n - pair_start > run ? min(run, n - pair_start - run) : 0;
  const size_t i0 = splits[t];
  // The tile ends inside the same pair (the pair length is a multiple of
  // TILE); at the pair's end every A item has been consumed.
  const size_t i1 = (o1 - pair_start == na + nb) ? na : splits[t + 1];
  const size_t j0 = (o0 - pair_start) - i0, j1 = (o1 - pair_start) - i1;
  const K *a = src + pair_start;
  const K *b = a + na;
  const V *av = src_v;
  const V *bv = src_v;
  if constexpr (!std::is_same<V, NoValue>::value) {
    av = src_v + pair_start;
    bv = av + na;
  }
  merge::merge_tile<K, V, Cmp, ITEMS>(sm, a, av, i0, i1, b, bv, j0, j1, dst, dst_v, o0);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct SortArgs {
  const void *in, *in_v;
  void *out, *out_v;
  size_t n;
  void *ws;
  size_t ws_bytes;
  hipStream_t stream;
};

struct Layout {
  size_t tiles = 0, block_tiles = 0, passes = 0;
  size_t scratch_k = 0, scratch_v = 0, splits = 0, total = 0;
};

template <class K, class V>
Layout layout(size_t n) {
  Layout l;
  if (n == 0) return l;
  constexpr size_t TILE = tile_items<K, V>();
  constexpr size_t BTILE = block_tile_items<K, V>();
  constexpr size_t VB = std::is_same<V, NoValue>::value ? 0 : sizeof(V);
  l.tiles = (n + TILE - 1) / TILE;
  l.block_tiles = (n + BTILE - 1) / BTILE;
  while ((size_t(1) << l.passes) < l.block_tiles) ++l.passes;
  size_t off = 0;
  l.scratch_k = off;
  off += align_up(n * sizeof(K), 256);
  l.scratch_v = off;
  off += align_up(n * VB, 256);
  l.splits = off;
  off += align_up((l.tiles + 1) * sizeof(uint64_t), 256);
  l.total = off;
  return l;
}

template <class K, class V, class Cmp>
rccl_hip_status run_sort(const SortArgs &s) {
  constexpr int ITEMS = items_for<K, V>();
  constexpr size_t TILE = tile_items<K, V>();
  constexpr int BT = block_threads<K, V>();
  static_assert(BT % THREADS == 0, "block sort tiles hold whole merge tiles");
  if (s.n < 1) return ok();
  const Layout l = layout<K, V>(s.n);
  if (!s.ws || s.ws_bytes < l.total)
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "merge sort workspace", l.total,
                     s.ws_bytes);
  unsigned char *ws = static_cast<unsigned char *>(s.ws);
  K *bufk[2] = {static_cast<K *>(s.out), reinterpret_cast<K *>(ws + l.scratch_k)};
  V *bufv[2] = {static_cast<V *>(s.out_v), reinterpret_cast<V *>(ws + l.scratch_v)};
  uint64_t *splits = reinterpret_cast<uint64_t *>(ws + l.splits);
  const int first = static_cast<int>(l.passes & 1);
  {
    KernelTimer t("merge_sort_block", s.stream, s.n);
    block_sort_kernel<K, V, Cmp, ITEMS, BT><<<dim3(static_cast<uint32_t>(l.block_tiles)), BT, 0,
                                              s.stream>>>(
        static_cast<const K *>(s.in), static_cast<const V *>(s.in_v), s.n, bufk[first],
        bufv[first]);
  }
  RCCL_HIP_TRY(check_launch("merge sort block"));
  int cur = first;
  for (size_t p = 0; p < l.passes; ++p) {
    const size_t run = block_tile_items<K, V>() << p;
    {
      KernelTimer t("merge_sort_partition", s.stream, l.tiles);
      pass_partition_kernel<K, Cmp><<<dim3(static_cast<uint32_t>((l.tiles + 255) / 256)), 256, 0,
                                      s.stream>>>(bufk[cur], s.n, run, TILE, l.tiles, splits);
    }
    RCCL_HIP_TRY(check_launch("merge sort partition"));
    {
      KernelTimer t("merge_sort_pass", s.stream, s.n);
      pass_merge_kernel<K, V, Cmp, ITEMS><<<dim3(static_cast<uint32_t>(l.tiles)), THREADS, 0,
                                            s.stream>>>(bufk[cur], bufv[cur], s.n, run,
                                                        bufk[1 - cur], bufv[1 - cur], splits);
    }
    RCCL_HIP_TRY(check_launch("merge sort pass"));
    cur = 1 - cur;
  }
  return ok();
}

#define RCCL_MERGE_SORT_DECLARE_KIND(NAME)                                                  \
  rccl_hip_status run_##NAME(const SortArgs &s, size_t value_bytes, bool descending);       \
  size_t bytes_##NAME(size_t n, size_t value_bytes);
RCCL_MERGE_SORT_DECLARE_KIND(u8)
RCCL_MERGE_SORT_DECLARE_KIND(i8)
RCCL_MERGE_SORT_DECLARE_KIND(u16)
RCCL_MERGE_SORT_DECLARE_KIND(i16)
RCCL_MERGE_SORT_DECLARE_KIND(u32)
RCCL_MERGE_SORT_DECLARE_KIND(i32)
RCCL_MERGE_SORT_DECLARE_KIND(f32)
RCCL_MERGE_SORT_DECLARE_KIND(u64)
RCCL_MERGE_SORT_DECLARE_KIND(i64)
RCCL_MERGE_SORT_DECLARE_KIND(f64)
#undef RCCL_MERGE_SORT_DECLARE_KIND

template <class K, bool DESC>
struct KindRunner {
  template <class V>
  static rccl_hip_status run(const SortArgs &s) {
    return run_sort<K, V, ordering::Less<K, DESC>>(s);
  }
};

#define RCCL_MERGE_SORT_DEFINE_KIND(NAME, KT)                                               \
  rccl_hip_status run_##NAME(const SortArgs &s, size_t value_bytes, bool descending) {      \
    using Desc = KindRunner<KT, true>;                                                      \
    using Asc = KindRunner<KT, false>;                                                      \
    if (descending) {                                                                       \
      RCCL_ORDERING_DISPATCH_VALUE(value_bytes, Desc, s)                                    \
    } else {                                                                                \
      RCCL_ORDERING_DISPATCH_VALUE(value_bytes, Asc, s)                                     \
    }                                                                                       \
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge sort value bytes");            \
  }                                                                                         \
  size_t bytes_##NAME(size_t n, size_t value_bytes) {                                       \
    switch (value_bytes) {                                                                  \
    case 0: return layout<KT, ordering::NoValue>(n).total;                                  \
    case 1: return layout<KT, uint8_t>(n).total;                                            \
    case 2: return layout<KT, uint16_t>(n).total;                                           \
    case 4: return layout<KT, uint32_t>(n).total;                                           \
    case 8: return layout<KT, uint64_t>(n).total;                                           \
    default: return layout<KT, Value16>(n).total;                                           \
    }                                                                                       \
  }

} // namespace merge_sort
} // namespace rccl_hip
