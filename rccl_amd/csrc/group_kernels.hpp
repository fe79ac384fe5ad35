// Adjacent-run compaction for gfx950: unique (keep the first of every run of
// equal adjacent keys) and reduce-by-key (one output per run: the run's first
// key and the left fold of its values), the steps after a sort in datalog
// deduplication.
//
// Reference behaviour: rccl-thrust/src/compaction.rs:224-378 (unique_copy_by,
// unique_by) and rccl-thrust/src/grouped_reduction.rs:102-216 over
// rccl-cub/src/grouped_reduction.rs:83-143 and compaction_kernels.rs:64-236:
// an item starts a run when it is the first or differs from its predecessor;
// a run's aggregate is a left fold, ((v0 op v1) op v2) ..., in index order.
// The reference marks run heads, scans them and folds each run on one thread
// in three launches. Here one pass over the input does all of it:
//   tile    one block per tile (tiles in XCD order or from a ticket,
//           lookback::claim_tile): keys
//           (and values) staged in LDS, run heads per thread, a block scan
//           of the head counts, the tile's output offset from a two-level
//           decoupled look-back (tile_lookback.hpp); for a reduction the
//           thread holding a head folds its run in index order, from LDS and,
//           past the tile's end, from global memory; results compacted in
//           LDS and stored coalesced; the last tile writes the count
// Keys compare with ==: scalar keys (floats by IEEE ==, so NaN keys never
// join a run) or [u32; N] rows (all columns equal). A key may carry a payload
// that takes no part in the comparison (the reference's key/value ranges
// compared by key, compaction.rs examples): each output takes the payload of
// its run's first item.
#pragma once

#include <type_traits>

#include "ordering_common.hpp"
#include "record_rows.hpp"
#include "tile_lookback.hpp"

namespace rccl_hip {
namespace group {

using ordering::NoValue;

// Key equality: == for scalars, every column for rows.
template <class K>
struct KeyEq {
  __device__ __forceinline__ bool operator()(const K &a, const K &b) const { return a == b; }
};
template <int N>
struct KeyEq<record_sort::Row<N>> {
  __device__ __forceinline__ bool operator()(const record_sort::Row<N> &a,
                                             const record_sort::Row<N> &b) const {
    bool eq = true;
#pragma unroll
    for (int i = 0; i < N; ++i) eq = eq && a.w[i] == b.w[i];
    return eq;
  }
};

// Copies keys; rows are copied column by column, which keeps arrays of rows
// in registers where a whole-struct copy under a branch would put them in
// scratch memory.
template <class K>
__device__ __forceinline__ void assign(K &dst, const K &src) {
  dst = src;
}
template <int N>
__device__ __forceinline__ void assign(record_sort::Row<N> &dst, const record_sort::Row<N> &src) {
#pragma unroll
  for (int i = 0; i < N; ++i) dst.w[i] = src.w[i];
}

// The reference's sealed group operators (rccl-cub/src/grouped_reduction.rs:17-75).
struct Unique {  // no values
  using Value = NoValue;
};
struct NaturalBagAdd {  // u64, wrapping
  using Value = uint64_t;
  __device__ __forceinline__ uint64_t operator()(uint64_t l, uint64_t r) const { return l + r; }
};
struct BooleanOr {  // BooleanProvenance: one byte, nonzero is true
  using Value = uint8_t;
  __device__ __forceinline__ uint8_t operator()(uint8_t l, uint8_t r) const {
    return (l != 0 || r != 0) ? 1 : 0;
  }
};
struct IndependentProbabilityOr {  // f64: l + r - l * r, clamped to [0, 1]
  using Value = double;
  __device__ __forceinline__ double operator()(double l, double r) const {
    // Rounded as written, (l + r) - (l * r): contraction into a fused
    // multiply-add would round once fewer and change the last bit.
#pragma clang fp contract(off)
    const double s = l + r;
    const double c = s - l * r;
    if (c < 0.0) return 0.0;
    if (c > 1.0) return 1.0;
    return c;
  }
};

#ifndef RCCL_GROUP_ITEMS_8B
#define RCCL_GROUP_ITEMS_8B 16
#endif
constexpr int THREADS = 256;
constexpr uint32_t XCD_RUN = 8;  // tiles per XCD run (xcd_order_tile)
constexpr int WAVES = THREADS / 64;

template <class T>
constexpr size_t bytes_of() {
  return std::is_same<T, NoValue>::value ? 0 : sizeof(T);
}
template <class K, class P, class V>
constexpr int items_for() {
  constexpr size_t bytes = sizeof(K) + bytes_of<P>() + bytes_of<V>();
  return bytes <= 8 ? RCCL_GROUP_ITEMS_8B : (bytes <= 16 ? 12 : (bytes <= 32 ? 8 : 6));
}
template <class K, class P, class V>
constexpr size_t tile_items() {
  return size_t(THREADS) * items_for<K, P, V>();
}

template <class T>
using Reg = typename std::conditional<std::is_same<T, NoValue>::value, char, T>::type;

template <class K, class P, class V, int ITEMS>
struct TileSmem {
  static constexpr uint32_t TILE = THREADS * ITEMS;
  static constexpr bool HAS_P = !std::is_same<P, NoValue>::value;
  static constexpr bool HAS_V = !std::is_same<V, NoValue>::value;
  K keys[TILE + 1];  // keys[0] is the item before the tile (when there is one)
  Reg<P> pays[HAS_P ? TILE : 1];
  Reg<V> vals[HAS_V ? TILE : 1];
  uint32_t wave_total[WAVES];
  uint64_t tile_offset;
};

template <class K, class P, class Op, int ITEMS>
__global__ void __launch_bounds__(THREADS)
group_tile_kernel(const K *__restrict__ keys, const P *__restrict__ pays,
                  const typename Op::Value *__restrict__ vals, size_t n, size_t tiles,
                  K *__restrict__ out_keys, P *__restrict__ out_pays,
                  typename Op::Value *__restrict__ out_vals, uint64_t *__restrict__ out_count,
                  uint64_t *desc, uint64_t *gagg, uint64_t *ginc, uint64_t *ticket,
                  uint32_t nx) {
  using V = typename Op::Value;
  using Smem = TileSmem<K, P, V, ITEMS>;
  constexpr bool HAS_P = Smem::HAS_P;
  constexpr bool HAS_V = Smem::HAS_V;
  constexpr uint32_t TILE = Smem::TILE;
  __shared__ Smem sm;
  const KeyEq<K> eq{};
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  // XCD order or a ticket (claim_tile): every tile a look-back waits on has
  // been started.
  __shared__ uint64_t s_tile;
  const size_t t = lookback::claim_tile<XCD_RUN>(nx, ticket, s_tile);
  if (t >= tiles) return;
  const size_t base = t * TILE;
  const uint32_t len = static_cast<uint32_t>(std::min<size_t>(TILE, n - base));

  // Stage the tile (striped, coalesced; clamped loads) and the key before it.
  {
    K kr[ITEMS];
    Reg<P> pr[HAS_P ? ITEMS : 1];
    Reg<V> vr[HAS_V ? ITEMS : 1];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t i = min(uint32_t(k) * THREADS + tid, len - 1u);
      assign(kr[k], keys[base + i]);
      if constexpr (HAS_P) pr[k] = pays[base + i];
      if constexpr (HAS_V) vr[k] = vals[base + i];
    }
    if (tid == 0 && t > 0) assign(sm.keys[0], keys[base - 1]);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const uint32_t i = uint32_t(k) * THREADS + tid;
      if (i < len) {
        assign(sm.keys[1 + i], kr[k]);
        if constexpr (HAS_P) sm.pays[i] = pr[k];
        if constexpr (HAS_V) sm.vals[i] = vr[k];
      }
    }
  }
  __syncthreads();

  // Run heads among this thread's ITEMS consecutive items.
  const uint32_t first = tid * uint32_t(ITEMS);
  uint32_t mask = 0;
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const uint32_t i = first + uint32_t(k);
    const bool head = i < len && ((base + i == 0) || !eq(sm.keys[i], sm.keys[1 + i]));
    mask |= head ? (1u << k) : 0u;
  }
  const uint32_t mine = __popc(mask);

  // Each head's key and payload; for a reduction, the fold of its run in
  // index order. A run ends at the next head; past the tile it continues in
  // global memory.
  K outk[ITEMS];
  Reg<P> outp[HAS_P ? ITEMS : 1];
  Reg<V> outv[HAS_V ? ITEMS : 1];
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    if (!(mask & (1u << k))) continue;
    const uint32_t i = first + uint32_t(k);
    assign(outk[k], sm.keys[1 + i]);
    if constexpr (HAS_P) outp[k] = sm.pays[i];
    if constexpr (HAS_V) {
      const Op op{};
      V agg = sm.vals[i];
      uint32_t j = i + 1;
      while (j < len && eq(sm.keys[j], sm.keys[1 + j])) {
        agg = op(agg, sm.vals[j]);
        ++j;
      }
      if (j == len) {
        size_t g = base + len;
        K prev;
        assign(prev, sm.keys[len]);
        while (g < n) {
          K next;
          assign(next, keys[g]);
          if (!eq(prev, next)) break;
          agg = op(agg, vals[g]);
          assign(prev, next);
          ++g;
        }
      }
      outv[k] = agg;
    }
  }

  // Block-wide exclusive scan of the head counts.
  const uint32_t inc = wave_inclusive_sum(mine, lane);
  if (lane == 63) sm.wave_total[wave] = inc;
  __syncthreads();
  uint32_t excl = inc - mine;
  uint32_t tile_count = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    if (uint32_t(w) < wave) excl += sm.wave_total[w];
    tile_count += sm.wave_total[w];
  }
  if (wave == 0) {
    const uint64_t prefix = lookback::tile_prefix(t, tiles, tile_count, desc, gagg, ginc, lane);
    if (lane == 0) {
      if (t + 1 == tiles) *out_count = prefix + tile_count;
      sm.tile_offset = prefix;
    }
  }

  // Compact through LDS (the staged tile is no longer read), then coalesced
  // stores.
  __syncthreads();
  {
    uint32_t o = excl;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      if (mask & (1u << k)) {
        assign(sm.keys[o], outk[k]);
        if constexpr (HAS_P) sm.pays[o] = outp[k];
        if constexpr (HAS_V) sm.vals[o] = outv[k];
        ++o;
      }
    }
  }
  __syncthreads();
  const size_t obase = sm.tile_offset;
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const uint32_t i = uint32_t(k) * THREADS + tid;
    if (i < tile_count) {
      assign(out_keys[obase + i], sm.keys[i]);
      if constexpr (HAS_P) out_pays[obase + i] = sm.pays[i];
      if constexpr (HAS_V) out_vals[obase + i] = sm.vals[i];
    }
  }
}

namespace {
__global__ void __launch_bounds__(256) group_clear_kernel(uint64_t *p, size_t words) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < words; i += size_t(gridDim.x) * 256)
    p[i] = 0;
}
} // namespace

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct GroupArgs {
  const void *keys, *pays, *vals;
  void *out_keys, *out_pays, *out_vals;
  size_t n;
  uint64_t *out_count;
  void *ws;
  size_t ws_bytes;
  hipStream_t stream;
};

struct Layout {
  size_t tiles = 0, groups = 0;
  size_t desc = 0, gagg = 0, ginc = 0, ticket = 0, total = 0;
};

template <class K, class P, class V>
Layout layout(size_t n) {
  Layout l;
  if (n == 0) return l;
  constexpr size_t TILE = tile_items<K, P, V>();
  l.tiles = (n + TILE - 1) / TILE;
  l.groups = (l.tiles + lookback::GROUP - 1) / lookback::GROUP;
  // Descriptors, group words and the ticket: one span (lookback::state_layout).
  const lookback::State st = lookback::state_layout(l.tiles);
  l.desc = 0;
  l.gagg = st.gagg * sizeof(uint64_t);
  l.ginc = st.ginc * sizeof(uint64_t);
  l.ticket = st.ticket * sizeof(uint64_t);
  l.total = align_up(st.words * sizeof(uint64_t), 256);
  return l;
}

// Zeroes *out_count for an empty input (no tile runs).
rccl_hip_status write_zero_count(uint64_t *out_count, hipStream_t stream);

template <class K, class P, class Op>
rccl_hip_status run(const GroupArgs &a) {
  using V = typename Op::Value;
  constexpr int ITEMS = items_for<K, P, V>();
  if (a.n == 0) return write_zero_count(a.out_count, a.stream);
  const Layout l = layout<K, P, V>(a.n);
  if (!a.ws || a.ws_bytes < l.total)
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "group workspace", l.total, a.ws_bytes);
  unsigned char *ws = static_cast<unsigned char *>(a.ws);
  uint64_t *desc = reinterpret_cast<uint64_t *>(ws + l.desc);
  const size_t words = lookback::state_words(l.tiles);
  uint32_t nx = 1;
  RCCL_HIP_TRY(tile_order(&nx, a.stream));
  RCCL_HIP_TRY(fit_tile_order(reinterpret_cast<const void *>(&group_tile_kernel<K, P, Op, ITEMS>),
                              THREADS, XCD_RUN, &nx));
  {
    KernelTimer t("group_clear", a.stream, words);
    group_clear_kernel<<<dim3(static_cast<uint32_t>(std::min<size_t>((words + 255) / 256, 1024))),
                         256, 0, a.stream>>>(desc, words);
  }
  RCCL_HIP_TRY(check_launch("group clear"));
  {
    KernelTimer t("group_tile", a.stream, a.n);
    group_tile_kernel<K, P, Op, ITEMS>
        <<<dim3(static_cast<uint32_t>(nx == XCDS ? xcd_order_grid(l.tiles, XCD_RUN) : l.tiles)),
           THREADS, 0, a.stream>>>(
        static_cast<const K *>(a.keys), static_cast<const P *>(a.pays),
        static_cast<const V *>(a.vals), a.n, l.tiles, static_cast<K *>(a.out_keys),
        static_cast<P *>(a.out_pays), static_cast<V *>(a.out_vals), a.out_count, desc,
        reinterpret_cast<uint64_t *>(ws + l.gagg), reinterpret_cast<uint64_t *>(ws + l.ginc),
        reinterpret_cast<uint64_t *>(ws + l.ticket), nx);
  }
  return check_launch("group tile");
}

// Runtime (operator, payload width) -> run<K, P, Op>. Unique carries 0, 1, 2,
// 4 or 8 payload bytes; the reductions 0, 4 or 8.
template <class K, class Op>
rccl_hip_status run_payload(const GroupArgs &a, size_t pb) {
  switch (pb) {
  case 0: return run<K, NoValue, Op>(a);
  case 4: return run<K, uint32_t, Op>(a);
  case 8: return run<K, uint64_t, Op>(a);
  }
  if constexpr (std::is_same<Op, Unique>::value) {
    if (pb == 1) return run<K, uint8_t, Op>(a);
    if (pb == 2) return run<K, uint16_t, Op>(a);
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "group payload bytes");
}
template <class K, class V>
size_t bytes_payload(size_t n, size_t pb) {
  switch (pb) {
  case 0: return layout<K, NoValue, V>(n).total;
  case 1: return layout<K, uint8_t, V>(n).total;
  case 2: return layout<K, uint16_t, V>(n).total;
  case 4: return layout<K, uint32_t, V>(n).total;
  default: return layout<K, uint64_t, V>(n).total;
  }
}

template <class K>
rccl_hip_status run_key(const GroupArgs &a, rccl_hip_group_op op, size_t pb) {
  switch (op) {
  case RCCL_HIP_GROUP_UNIQUE: return run_payload<K, Unique>(a, pb);
  case RCCL_HIP_GROUP_NATURAL_BAG_ADD: return run_payload<K, NaturalBagAdd>(a, pb);
  case RCCL_HIP_GROUP_BOOLEAN_OR: return run_payload<K, BooleanOr>(a, pb);
  case RCCL_HIP_GROUP_INDEPENDENT_PROBABILITY_OR:
    return run_payload<K, IndependentProbabilityOr>(a, pb);
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "group operator");
}
template <class K>
size_t bytes_key(size_t n, rccl_hip_group_op op, size_t pb) {
  switch (op) {
  case RCCL_HIP_GROUP_UNIQUE: return bytes_payload<K, NoValue>(n, pb);
  case RCCL_HIP_GROUP_NATURAL_BAG_ADD: return bytes_payload<K, uint64_t>(n, pb);
  case RCCL_HIP_GROUP_BOOLEAN_OR: return bytes_payload<K, uint8_t>(n, pb);
  default: return bytes_payload<K, double>(n, pb);
  }
}

// One key type per translation unit (group_<key>.hip).
#define RCCL_GROUP_DECLARE_KEY(NAME)                                                      \
  rccl_hip_status run_##NAME(const GroupArgs &a, rccl_hip_group_op op, size_t pb);      \
  size_t bytes_##NAME(size_t n, rccl_hip_group_op op, size_t pb);
RCCL_GROUP_DECLARE_KEY(u8)
RCCL_GROUP_DECLARE_KEY(i8)
RCCL_GROUP_DECLARE_KEY(u16)
RCCL_GROUP_DECLARE_KEY(i16)
RCCL_GROUP_DECLARE_KEY(u32)
RCCL_GROUP_DECLARE_KEY(i32)
RCCL_GROUP_DECLARE_KEY(f32)
RCCL_GROUP_DECLARE_KEY(u64)
RCCL_GROUP_DECLARE_KEY(i64)
RCCL_GROUP_DECLARE_KEY(f64)
RCCL_GROUP_DECLARE_KEY(row2)
RCCL_GROUP_DECLARE_KEY(row3)
RCCL_GROUP_DECLARE_KEY(row4)
RCCL_GROUP_DECLARE_KEY(row5)
RCCL_GROUP_DECLARE_KEY(row6)
#undef RCCL_GROUP_DECLARE_KEY

#define RCCL_GROUP_DEFINE_KEY(NAME, KT)                                                   \
  rccl_hip_status run_##NAME(const GroupArgs &a, rccl_hip_group_op op, size_t pb) {     \
    return run_key<KT>(a, op, pb);                                                       \
  }                                                                                      \
  size_t bytes_##NAME(size_t n, rccl_hip_group_op op, size_t pb) {                       \
    return bytes_key<KT>(n, op, pb);                                                     \
  }

} // namespace group
} // namespace rccl_hip
