// Sorted multiset operations for gfx950: union, intersection, difference and
// symmetric difference (keys or key/value pairs, or a count only).
//
// Reference behaviour: rccl-cub/src/set_operation.rs:265-589 (host control)
// and rccl-cub/src/ordering_backend/set.rs (agents): balanced-path
// partitioning (:401-506), the four serial operations (:564-827), tile
// compaction with decoupled look-back and the final count (:830-1546).
// Design:
//   partition  one thread per tile boundary: balanced path in HBM
//   tile       one block per tile: A and B slices staged in LDS, a balanced
//              path per thread in LDS, ITEMS steps of the serial operation,
//              a block scan of the emitted counts, a two-level decoupled
//              look-back for the tile's global output offset (a whole wave
//              polls 64 predecessors at once, tile_lookback.hpp),
//              LDS-compacted coalesced stores; the last tile writes the
//              output count
#pragma once

#include <algorithm>
#include <cstring>

#include "ordering_common.hpp"
#include "tile_lookback.hpp"

namespace rccl_hip {
namespace set_ops {

using ordering::NoValue;

#ifndef RCCL_SET_THREADS
#define RCCL_SET_THREADS 512
#endif
#ifndef RCCL_SET_ITEMS_8B
#define RCCL_SET_ITEMS_8B 16
#endif
#ifndef RCCL_SET_XCD_RUN
#define RCCL_SET_XCD_RUN 8
#endif
// The tile kernel's in-LDS run-bound searches gallop from the split too: in
// C5, 41% of the threads' diagonals split a run of equal keys (A and B share
// keys), so every wave has a thread that searches them; galloping measured
// 0.5-1.5% faster per operation than binary searches over the sub-tile.
#ifndef RCCL_SET_TILE_GALLOP
#define RCCL_SET_TILE_GALLOP true
#endif
constexpr int THREADS = RCCL_SET_THREADS;
constexpr int WAVES = THREADS / 64;
constexpr size_t GROUP = lookback::GROUP;
constexpr uint32_t XCD_RUN = RCCL_SET_XCD_RUN;  // tiles per XCD run (xcd_order_tile)

enum Op : int { UNION = 0, INTERSECTION = 1, DIFFERENCE = 2, SYMMETRIC_DIFFERENCE = 3 };

// Union and symmetric difference of 8-byte keys emit from both inputs: their
// outputs, kept in registers for two partition tiles, fit the 128-register
// budget without spilling at one item fewer per thread.
#ifndef RCCL_SET_ITEMS_8B_BOTH
#define RCCL_SET_ITEMS_8B_BOTH 15
#endif
template <class K, class V, int OP>
constexpr int items_for() {
  constexpr bool keys_only = std::is_same<V, NoValue>::value;
  constexpr size_t bytes = sizeof(K) + (keys_only ? 0 : sizeof(V));
  if constexpr (keys_only && sizeof(K) == 8 && (OP == UNION || OP == SYMMETRIC_DIFFERENCE))
    return RCCL_SET_ITEMS_8B_BOTH;
  return bytes <= 8 ? RCCL_SET_ITEMS_8B : (bytes <= 16 ? 12 : 8);
}
// The fewest items per thread over the four operations: the most partition
// tiles, which sizes a workspace that serves every operation.
template <class K, class V>
constexpr int min_items_for() {
  return std::min(std::min(items_for<K, V, UNION>(), items_for<K, V, INTERSECTION>()),
                  std::min(items_for<K, V, DIFFERENCE>(), items_for<K, V, SYMMETRIC_DIFFERENCE>()));
}
// Partition tiles per block (and per look-back tile): two for keys only,
// whose two register sets of outputs fit; one where values double them.
#ifndef RCCL_SET_SUB_TILES
#define RCCL_SET_SUB_TILES 2
#endif
template <class K, class V>
constexpr int sub_tiles_for() {
  return std::is_same<V, NoValue>::value ? RCCL_SET_SUB_TILES : 1;
}

// Finite arithmetic input range: item i is start + step * i in the key's own
// wrapping integer arithmetic (rccl-cub/src/ordering_backend/set.rs:49-81,
// rccl-cub/src/range.rs:43-78); nothing is materialised. Indices are checked
// on the host to fit the key type.
template <class K>
struct Arith {
  K start, step;
};
template <class K>
__device__ __forceinline__ K arith_at(const Arith<K> &r, size_t i) {
  if constexpr (std::is_integral<K>::value) {
    using W = typename std::conditional<(sizeof(K) <= 4), uint32_t, uint64_t>::type;
    return static_cast<K>(static_cast<W>(static_cast<W>(r.start) +
                                         static_cast<W>(r.step) * static_cast<W>(i)));
  } else {
    return K{};  // arithmetic ranges are integral only
  }
}

// First index x in [lo, hi) whose item is not `before` (the items are
// `before` up to some index and not after it), found from hi downward with
// doubling steps: O(log(hi - x)) probes, so a short run of equal keys at the
// end of the range costs a few probes instead of a full binary search.
template <class I, class R, class Pred>
__device__ __forceinline__ I gallop_down(R r, I lo, I hi, Pred before) {
  I b = hi, step = 1;  // every x in [b, hi) is not `before`
  while (b > lo) {
    const I p = b - lo > step ? b - step : lo;
    if (before(r(p))) {  // the answer is in (p, b]
      I l = p + 1, h = b;
      while (l < h) {
        const I m = l + (h - l) / 2;
        if (before(r(m))) l = m + 1; else h = m;
      }
      return l;
    }
    b = p;
    step <<= 1;
  }
  return lo;
}

// First index x in [lo, hi) whose item is `after` (the items are not `after`
// up to some index and are after it), found from lo upward with doubling
// steps; hi if there is none.
template <class I, class R, class Pred>
__device__ __forceinline__ I gallop_up(R r, I lo, I hi, Pred after) {
  I a = lo, step = 1;  // no x in [lo, a) is `after`
  while (a < hi) {
    const I p = hi - a > step ? a + step - 1 : hi - 1;
    if (after(r(p))) {  // the answer is in [a, p]
      I l = a, h = p;
      while (l < h) {
        const I m = l + (h - l) / 2;
        if (after(r(m))) h = m; else l = m + 1;
      }
      return l;
    }
    a = p + 1;
    step <<= 1;
  }
  return hi;
}

// Balanced path at `diag` (rccl-cub/src/ordering_backend/set.rs:436-506): the
// merge-path split, moved inside a run of keys equal to B[j] so that the run's
// A and B items are divided evenly and each A item stays on the side of its
// B partner; `star` adds the partner of a trailing unmatched A item to this
// side. Returns (i, j) with i + j = diag + star.
// GALLOP: the run bounds are searched outward from the split, since runs of
// equal keys are usually short (the partition kernel over HBM, where each
// probe is a dependent round trip: 60 -> 36 us per C5 operation; the tile
// kernel in LDS, RCCL_SET_TILE_GALLOP); otherwise by binary search.
// balanced_path_at starts from the merge-path split i of the diagonal.
template <bool GALLOP, class K, class I = size_t, class Cmp, class RA, class RB>
__device__ __forceinline__ void balanced_path_at(RA a, I na, RB b, I nb, I diag, I i,
                                                 Cmp less, I &out_i, I &out_j) {
  const I j = diag - i;
  I star = 0;
  // No A item before the split and no B item before it is equal to B[j]:
  // the balanced path is the merge path (the searches below would find
  // i_start = i, j_start = j and move nothing).
  const bool run_straddles =
      j < nb && ((i > 0 && !less(a(i - 1), b(j))) || (j > 0 && !less(b(j - 1), b(j))));
  if (run_straddles) {
    const K key = b(j);
    const auto before_key = [&](const K &x) { return less(x, key); };
    const auto after_key = [&](const K &x) { return less(key, x); };
    auto lower = [&](auto r, I lo, I hi) {  // first in [lo, hi) not before key
      if constexpr (GALLOP) return gallop_down<I>(r, lo, hi, before_key);
      while (lo < hi) {
        const I mid = lo + (hi - lo) / 2;
        if (before_key(r(mid))) lo = mid + 1; else hi = mid;
      }
      return lo;
    };
    const I i_start = lower(a, 0, i);
    const I j_start = lower(b, 0, j);
    const I a_run = i - i_start;
    const I b_seen = j - j_start;
    const I total = a_run + b_seen;
    I b_adv = std::max(total >> 1, b_seen);
    const I b_end = std::min(nb, j_start + b_adv + 1);
    // End of the key's B run within [j, b_end).
    I run_end;
    if constexpr (GALLOP) {
      run_end = gallop_up<I>(b, j, b_end, after_key);
    } else {
      I lo = j, hi = b_end;
      while (lo < hi) {
        const I mid = lo + (hi - lo) / 2;
        if (!after_key(b(mid))) lo = mid + 1; else hi = mid;
      }
      run_end = lo;
    }
    const I b_run = run_end - j_start;
    b_adv = std::min(b_adv, b_run);
    const I a_adv = total - b_adv;
    star = (a_adv == b_adv + 1 && b_adv < b_run) ? 1 : 0;
    i = i_start + a_adv;
  }
  out_i = i;
  out_j = diag - i + star;
}

template <bool GALLOP, class K, class Cmp, class RA, class RB>
__device__ __forceinline__ void balanced_path(RA a, size_t na, RB b, size_t nb, size_t diag,
                                              Cmp less, size_t &out_i, size_t &out_j) {
  balanced_path_at<GALLOP, K>(a, na, b, nb, diag, ordering::merge_path<K>(a, na, b, nb, diag, less),
                              less, out_i, out_j);
}

// Also zeroes the tile kernel's look-back state (descriptors, group words and
// the ticket: `state_words` words at `state`), which no earlier launch of the
// call touches, so no separate clearing launch is needed.
// With SAMPLED, the merge-path split comes from the samples of
// ordering::merge_sample_kernel (m) before the balanced path adjusts it.
template <class K, class Cmp, bool ARITH, bool SAMPLED>
__global__ void __launch_bounds__(256)
partition_kernel(const K *__restrict__ a, size_t na, const K *__restrict__ b, size_t nb,
                 size_t tile, size_t count, uint64_t *__restrict__ splits, Arith<K> ar,
                 Arith<K> br, uint64_t *__restrict__ state, size_t state_words,
                 const uint32_t *__restrict__ m) {
  const size_t t = size_t(blockIdx.x) * 256 + threadIdx.x;
  for (size_t w = t; w < state_words; w += size_t(gridDim.x) * 256) state[w] = 0;
  if (t >= count) return;
  const size_t diag = std::min(t * tile, na + nb);
  size_t i, j;
  if constexpr (ARITH) {
    balanced_path<true, K>([&](size_t x) { return arith_at(ar, x); }, na,
                           [&](size_t x) { return arith_at(br, x); }, nb, diag, Cmp{}, i, j);
  } else {
    auto ra = [&](size_t x) { return a[x]; };
    auto rb = [&](size_t x) { return b[x]; };
    if constexpr (SAMPLED)
      balanced_path_at<true, K>(ra, na, rb, nb, diag,
                                ordering::sampled_merge_path<K>(ra, na, rb, nb, diag, m, Cmp{}),
                                Cmp{}, i, j);
    else
      balanced_path<true, K>(ra, na, rb, nb, diag, Cmp{}, i, j);
  }
  splits[2 * t] = i;
  splits[2 * t + 1] = j;
}


template <class K, class V, int ITEMS>
struct TileSmem {
  static constexpr uint32_t TILE = THREADS * ITEMS;
  static constexpr uint32_t CAP = TILE + 2;  // a star can make a tile one item longer
  static constexpr bool PAIRS = !std::is_same<V, NoValue>::value;
  K keys[CAP];
  typename std::conditional<PAIRS, V, char>::type vals[PAIRS ? CAP : 1];
  uint32_t split_a[THREADS + 1];
  uint32_t split_b[THREADS + 1];
  uint32_t wave_total[WAVES];
  uint64_t tile_offset;
};

// One serial step of operation OP on the current heads. Mirrors the four
// serial operations of rccl-cub/src/ordering_backend/set.rs:564-827:
//   union         emit B if B < A, else emit A (equal heads: A, both advance)
//   intersection  emit A when the heads are equal
//   difference    emit A when A < B (or B is exhausted)
//   symmetric     emit the strictly smaller head (or the remaining side)
// `emit_b` selects the source of the emitted item.
template <int OP, class K, class Cmp>
__device__ __forceinline__ void serial_step(const K &ka, const K &kb, bool a_ok, bool b_ok,
                                            Cmp less, bool &emit, bool &emit_b, bool &adv_a,
                                            bool &adv_b) {
  bool a_sel, b_sel;
  if (!a_ok) {
    b_sel = true;
    a_sel = false;
  } else if (!b_ok) {
    a_sel = true;
    b_sel = false;
  } else {
    a_sel = less(ka, kb);
    b_sel = !a_sel && less(kb, ka);
  }
  const bool live = a_ok || b_ok;
  if constexpr (OP == INTERSECTION) {
    emit = a_ok && b_ok && !a_sel && !b_sel;
    emit_b = false;
  } else if constexpr (OP == UNION) {
    emit = live;
    emit_b = b_sel;
  } else if constexpr (OP == DIFFERENCE) {
    emit = live && a_sel;
    emit_b = false;
  } else {
    emit = live && (a_sel != b_sel);
    emit_b = b_sel;
  }
  adv_a = live && !b_sel;
  adv_b = live && !a_sel;
}

// Outputs of one partition tile, held in registers until the block's output
// offset is known.
template <class K, class VS, int ITEMS, bool PAIRS>
struct SubTile {
  K outk[ITEMS];
  VS outv[PAIRS ? ITEMS : 1];
  uint32_t mask;   // emitted items of this thread
  uint32_t excl;   // this thread's first output within the sub-tile
  uint32_t count;  // the sub-tile's outputs
};

// One block handles SUB consecutive partition tiles (a look-back tile): each
// is staged, partitioned and run through the serial operation in turn, its
// outputs kept in registers; the block then publishes one count and looks
// back once for all of them, and stores them in turn. SUB = 2 halves the
// look-backs at the same LDS footprint (two blocks per CU).
// Two blocks per CU (4 waves per SIMD): a register budget of 128.
#ifndef RCCL_SET_WAVES_PER_SIMD
#define RCCL_SET_WAVES_PER_SIMD 4
#endif
template <class K, class V, class Cmp, int OP, int ITEMS, int SUB, bool ARITH>
__global__ void __launch_bounds__(THREADS, RCCL_SET_WAVES_PER_SIMD)
tile_kernel(const K *__restrict__ a, const V *__restrict__ av, const K *__restrict__ b,
            const V *__restrict__ bv, const uint64_t *__restrict__ splits, size_t tiles,
            size_t lb_tiles, K *__restrict__ out, V *__restrict__ outv, size_t out_cap,
            uint64_t *__restrict__ out_count, uint64_t *desc, uint64_t *gagg, uint64_t *ginc,
            uint64_t *ticket, uint32_t nx, Arith<K> ar, Arith<K> br) {
  using Smem = TileSmem<K, V, ITEMS>;
  constexpr bool PAIRS = Smem::PAIRS;
  constexpr bool VALS_B = PAIRS && (OP == UNION || OP == SYMMETRIC_DIFFERENCE);
  using VS = typename std::conditional<PAIRS, V, char>::type;
  __shared__ Smem sm;
  const Cmp less{};
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  // Tiles in XCD order (no atomic to take first; neighbouring tiles share an
  // L2) or, where the device's placement is not round-robin, from a ticket:
  // either way every tile a look-back waits on has been started.
  __shared__ uint64_t s_tile;
  const size_t t = lookback::claim_tile<XCD_RUN>(nx, ticket, s_tile);
  if (t >= lb_tiles) return;

  // A partition tile's inputs, loaded into registers: a fixed, unrolled
  // number of loads per thread, each from A or B through a per-lane address,
  // clamped to the tile's last item (striped, so the loads coalesce).
  constexpr int STAGE = (Smem::CAP + THREADS - 1) / THREADS;
  K kr[STAGE];
  VS vr[PAIRS ? STAGE : 1];
  auto load_tile = [&](size_t pt) {
    const size_t i0 = splits[2 * pt], j0 = splits[2 * pt + 1];
    const uint32_t la = static_cast<uint32_t>(splits[2 * pt + 2] - i0);
    const uint32_t len = la + static_cast<uint32_t>(splits[2 * pt + 3] - j0);
#pragma unroll
    for (int k = 0; k < STAGE; ++k) {
      const uint32_t i = min(uint32_t(k) * THREADS + tid, len ? len - 1u : 0u);
      const bool from_a = i < la;
      if constexpr (ARITH)
        kr[k] = len ? (from_a ? arith_at(ar, i0 + i) : arith_at(br, j0 + (i - la))) : K{};
      else
        kr[k] = len ? *(from_a ? a + i0 + i : b + j0 + (i - la)) : K{};
      if constexpr (PAIRS) {
        if constexpr (VALS_B) vr[k] = len ? *(from_a ? av + i0 + i : bv + j0 + (i - la)) : V{};
        else vr[k] = from_a ? av[i0 + i] : V{};
      }
    }
  };
  if (t * SUB < tiles) load_tile(t * SUB);

  // Barriers order LDS only (lds_barrier): the next sub-tile's loads, issued
  // right after the current one is staged, stay in flight through its merge.
  SubTile<K, VS, ITEMS, PAIRS> sub[SUB];
#pragma unroll
  for (int s = 0; s < SUB; ++s) {
    SubTile<K, VS, ITEMS, PAIRS> &r = sub[s];
    const size_t pt = t * SUB + s;
    if (pt >= tiles) {  // uniform: the last look-back tile may be short
      r.mask = 0;
      r.excl = 0;
      r.count = 0;
      continue;
    }
    const size_t i0 = splits[2 * pt], j0 = splits[2 * pt + 1];
    const size_t i1 = splits[2 * pt + 2], j1 = splits[2 * pt + 3];
    const uint32_t la = static_cast<uint32_t>(i1 - i0);
    const uint32_t lb = static_cast<uint32_t>(j1 - j0);
    const uint32_t len = la + lb;

    // Stage the registers into LDS (the previous sub-tile's readers are past
    // its scan barrier), then load the next sub-tile.
#pragma unroll
    for (int k = 0; k < STAGE; ++k) {
      const uint32_t i = uint32_t(k) * THREADS + tid;
      if (i < len) {
        sm.keys[i] = kr[k];
        if constexpr (PAIRS) sm.vals[i] = vr[k];
      }
    }
    lds_barrier();
    if (s + 1 < SUB && pt + 1 < tiles) load_tile(pt + 1);

    // Per-thread balanced-path splits (diagonal tid * ITEMS of this tile).
    {
      const K *ka = sm.keys;
      const K *kb = sm.keys + la;
      // 32-bit indices: the tile is in LDS.
      uint32_t si, sj;
      const uint32_t diag = min(tid * uint32_t(ITEMS), len);
      const uint32_t ip = ordering::merge_path_lds<K>(ka, la, kb, lb, diag, less);
      balanced_path_at<RCCL_SET_TILE_GALLOP, K, uint32_t>(
          [&](uint32_t x) { return ka[x]; }, la, [&](uint32_t x) { return kb[x]; }, lb, diag,
          ip, less, si, sj);
      // Every split lies inside the tile; the star of a diagonal past the end
      // is clamped.
      sm.split_a[tid] = min(si, la);
      sm.split_b[tid] = min(sj, lb);
      if (tid == 0) {
        sm.split_a[THREADS] = la;
        sm.split_b[THREADS] = lb;
      }
    }
    lds_barrier();

    // Serial operation over this thread's A and B ranges.
    uint32_t ia = sm.split_a[tid], ib = sm.split_b[tid];
    const uint32_t ea = max(ia, sm.split_a[tid + 1]), eb = max(ib, sm.split_b[tid + 1]);
    uint32_t src[PAIRS ? ITEMS : 1];
    uint32_t mask = 0;
    // The heads live in registers; a step reloads only the side it advanced.
    const uint32_t last = len ? len - 1u : 0u;
    K ka = sm.keys[min(ia, last)];
    K kb = sm.keys[min(la + ib, last)];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const bool a_ok = ia < ea, b_ok = ib < eb;
      bool emit, emit_b, adv_a, adv_b;
      serial_step<OP, K>(ka, kb, a_ok, b_ok, less, emit, emit_b, adv_a, adv_b);
      r.outk[k] = emit_b ? kb : ka;
      if constexpr (PAIRS) src[k] = emit_b ? la + ib : ia;
      mask |= emit ? (1u << k) : 0u;
      ia += adv_a ? 1u : 0u;
      ib += adv_b ? 1u : 0u;
      if (k + 1 < ITEMS) {
        if (adv_a) ka = sm.keys[min(ia, last)];
        if (adv_b) kb = sm.keys[min(la + ib, last)];
      }
    }
    const uint32_t mine = __popc(mask);
    r.mask = mask;
    if constexpr (PAIRS) {
#pragma unroll
      for (int k = 0; k < ITEMS; ++k) r.outv[k] = sm.vals[min(src[k], last)];
    }

    // Block-wide exclusive scan of the emitted counts.
    const uint32_t inc = wave_inclusive_sum(mine, lane);
    if (lane == 63) sm.wave_total[wave] = inc;
    lds_barrier();
    r.excl = inc - mine;
    r.count = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      if (uint32_t(w) < wave) r.excl += sm.wave_total[w];
      r.count += sm.wave_total[w];
    }
    // The next sub-tile's scan writes wave_total only after two more
    // barriers, which every reader above has passed.
  }
  uint32_t total = 0;
#pragma unroll
  for (int s = 0; s < SUB; ++s) total += sub[s].count;

  auto compact = [&](const SubTile<K, VS, ITEMS, PAIRS> &r) {
    uint32_t o = r.excl;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      if (r.mask & (1u << k)) {
        sm.keys[o] = r.outk[k];
        if constexpr (PAIRS) sm.vals[o] = r.outv[k];
        ++o;
      }
    }
  };
  // Two-level decoupled look-back for the block's output offset (wave 0),
  // while the other waves compact the first sub-tile into LDS (every read of
  // the staged inputs lies before the last scan barrier).
  if (wave == 0) {
    const uint64_t prefix = lookback::tile_prefix(t, lb_tiles, total, desc, gagg, ginc, lane);
    if (lane == 0) {
      if (t + 1 == lb_tiles && out_count) *out_count = prefix + total;
      sm.tile_offset = prefix;
    }
  }
  if (out != nullptr) compact(sub[0]);
  lds_barrier();
  if (out == nullptr) return;  // count only

  // Coalesced stores from the LDS-compacted outputs, one sub-tile at a time
  // (each later sub-tile compacted once the previous stores have read the
  // buffer); positions at or past the destination's capacity are counted but
  // not written.
  size_t base = sm.tile_offset;
#pragma unroll
  for (int s = 0; s < SUB; ++s) {
    const SubTile<K, VS, ITEMS, PAIRS> &r = sub[s];
    if (base >= out_cap) return;  // uniform: the rest lies past the end
    const uint32_t keep = static_cast<uint32_t>(std::min<size_t>(r.count, out_cap - base));
    if (s > 0) {
      lds_barrier();  // the previous sub-tile's stores have read the buffer
      compact(r);
      lds_barrier();
    }
    constexpr int STORE = (Smem::CAP + THREADS - 1) / THREADS;
#pragma unroll
    for (int k = 0; k < STORE; ++k) {
      const uint32_t i = uint32_t(k) * THREADS + tid;
      if (i < keep) {
        out[base + i] = sm.keys[i];
        if constexpr (PAIRS) outv[base + i] = sm.vals[i];
      }
    }
    base += r.count;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct SetArgs {
  int op;
  const void *a, *av, *b, *bv;
  size_t na, nb;
  void *out, *outv;
  size_t out_cap;
  uint64_t *out_count;
  void *ws;
  size_t ws_bytes;
  hipStream_t stream;
  // Arithmetic inputs (keys only): a and b are unused; start and step hold
  // the key's bytes in their low bytes.
  bool arith;
  uint64_t a_start, a_step, b_start, b_step;
};

struct Layout {
  size_t tiles = 0, lb_tiles = 0, groups = 0;  // partition tiles, look-back tiles
  size_t splits = 0, desc = 0, gagg = 0, ginc = 0, ticket = 0, samples = 0, total = 0;
  bool sampled = false;  // integer keys from SAMPLED_MIN_TILES partition tiles
};

// The sampled merge-path partition serves inputs of at least this many
// partition tiles (integer keys; arithmetic ranges compute their items and
// keep the plain search).
constexpr size_t SAMPLED_MIN_TILES = 512;

// Workspace layout for partition tiles of ITEMS items per thread. Fewer items
// give more tiles and no smaller a section, so the layout at min_items_for
// bounds every operation's.
template <class K, class V, int ITEMS>
Layout layout(size_t na, size_t nb) {
  Layout l;
  const size_t total = na + nb;
  constexpr size_t TILE = size_t(THREADS) * ITEMS;
  l.tiles = total ? (total + TILE - 1) / TILE : 1;  // an empty input still reports its count
  constexpr size_t SUB = sub_tiles_for<K, V>();
  l.lb_tiles = (l.tiles + SUB - 1) / SUB;
  l.groups = (l.lb_tiles + GROUP - 1) / GROUP;
  size_t off = 0;
  l.splits = off;
  off += align_up((l.tiles + 1) * 2 * sizeof(uint64_t), 256);
  // Descriptors, group words and the ticket: one span (lookback::state_layout).
  const lookback::State st = lookback::state_layout(l.lb_tiles);
  l.desc = off;
  l.gagg = off + st.gagg * sizeof(uint64_t);
  l.ginc = off + st.ginc * sizeof(uint64_t);
  l.ticket = off + st.ticket * sizeof(uint64_t);
  off += st.words * sizeof(uint64_t);
  l.sampled = ordering::sampled_partition_for<K>() && na > 0 && nb > 0 &&
              l.tiles >= SAMPLED_MIN_TILES;
  if (l.sampled) {
    off = align_up(off, 256);
    l.samples = off;
    off += ordering::merge_samples(na) * sizeof(uint32_t);
  }
  l.total = align_up(off, 256);
  return l;
}

template <class K, class V, class Cmp, int OP>
rccl_hip_status run_op(const SetArgs &s) {
  constexpr int ITEMS = items_for<K, V, OP>();
  constexpr int SUB = sub_tiles_for<K, V>();
  constexpr size_t TILE = size_t(THREADS) * ITEMS;
  const Layout l = layout<K, V, ITEMS>(s.na, s.nb);
  if (!s.ws || s.ws_bytes < l.total)
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "set operation workspace", l.total,
                     s.ws_bytes);
  unsigned char *ws = static_cast<unsigned char *>(s.ws);
  uint64_t *splits = reinterpret_cast<uint64_t *>(ws + l.splits);
  uint64_t *desc = reinterpret_cast<uint64_t *>(ws + l.desc);
  uint64_t *gagg = reinterpret_cast<uint64_t *>(ws + l.gagg);
  uint64_t *ginc = reinterpret_cast<uint64_t *>(ws + l.ginc);
  uint64_t *ticket = reinterpret_cast<uint64_t *>(ws + l.ticket);
  // Descriptors, group words and the ticket are contiguous.
  const size_t state_words = lookback::state_words(l.lb_tiles);
  uint32_t nx = 1;
  RCCL_HIP_TRY(tile_order(&nx, s.stream));
  RCCL_HIP_TRY(fit_tile_order(
      s.arith ? reinterpret_cast<const void *>(&tile_kernel<K, V, Cmp, OP, ITEMS, SUB, true>)
              : reinterpret_cast<const void *>(&tile_kernel<K, V, Cmp, OP, ITEMS, SUB, false>),
      THREADS, XCD_RUN, &nx));
  const dim3 pgrid(static_cast<uint32_t>((l.tiles + 1 + 255) / 256));
  const dim3 tgrid(
      static_cast<uint32_t>(nx == XCDS ? xcd_order_grid(l.lb_tiles, XCD_RUN) : l.lb_tiles));
  const K *a = static_cast<const K *>(s.a);
  const K *b = static_cast<const K *>(s.b);
  const V *av = static_cast<const V *>(s.av);
  const V *bv = static_cast<const V *>(s.bv);
  K *out = static_cast<K *>(s.out);
  V *outv = static_cast<V *>(s.outv);
  if (s.arith) {
    if constexpr (std::is_integral<K>::value && std::is_same<V, NoValue>::value) {
      Arith<K> ar, br;
      std::memcpy(&ar.start, &s.a_start, sizeof(K));
      std::memcpy(&ar.step, &s.a_step, sizeof(K));
      std::memcpy(&br.start, &s.b_start, sizeof(K));
      std::memcpy(&br.step, &s.b_step, sizeof(K));
      {
        KernelTimer t("set_partition", s.stream, l.tiles + 1);
        partition_kernel<K, Cmp, true, false><<<pgrid, 256, 0, s.stream>>>(
            a, s.na, b, s.nb, TILE, l.tiles + 1, splits, ar, br, desc, state_words, nullptr);
      }
      RCCL_HIP_TRY(check_launch("set partition"));
      {
        KernelTimer t("set_tile", s.stream, s.na + s.nb);
        tile_kernel<K, V, Cmp, OP, ITEMS, SUB, true><<<tgrid, THREADS, 0, s.stream>>>(
            a, av, b, bv, splits, l.tiles, l.lb_tiles, out, outv, s.out_cap, s.out_count, desc, gagg, ginc,
            ticket, nx, ar, br);
      }
      return check_launch("set tile");
    } else {
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "arithmetic range key kind");
    }
  }
  uint32_t *m = l.sampled ? reinterpret_cast<uint32_t *>(ws + l.samples) : nullptr;
  if (l.sampled) {
    const size_t ka = ordering::merge_samples(s.na);
    {
      KernelTimer t("set_sample", s.stream, ka);
      ordering::merge_sample_kernel<K, Cmp>
          <<<dim3(static_cast<uint32_t>(ordering::merge_sample_blocks(s.na))), 256, 0,
             s.stream>>>(a, s.na, b, s.nb, m);
    }
    RCCL_HIP_TRY(check_launch("set sample"));
  }
  {
    KernelTimer t("set_partition", s.stream, l.tiles + 1);
    if (l.sampled) {
      partition_kernel<K, Cmp, false, true><<<pgrid, 256, 0, s.stream>>>(
          a, s.na, b, s.nb, TILE, l.tiles + 1, splits, Arith<K>{}, Arith<K>{}, desc, state_words,
          m);
    } else {
      partition_kernel<K, Cmp, false, false><<<pgrid, 256, 0, s.stream>>>(
          a, s.na, b, s.nb, TILE, l.tiles + 1, splits, Arith<K>{}, Arith<K>{}, desc, state_words,
          nullptr);
    }
  }
  RCCL_HIP_TRY(check_launch("set partition"));
  {
    KernelTimer t("set_tile", s.stream, s.na + s.nb);
    tile_kernel<K, V, Cmp, OP, ITEMS, SUB, false><<<tgrid, THREADS, 0, s.stream>>>(
        a, av, b, bv, splits, l.tiles, l.lb_tiles, out, outv, s.out_cap, s.out_count, desc, gagg, ginc,
        ticket, nx, Arith<K>{}, Arith<K>{});
  }
  return check_launch("set tile");
}

template <class K, bool DESC>
struct KindRunner {
  template <class V>
  static rccl_hip_status run(const SetArgs &s) {
    using Cmp = ordering::Less<K, DESC>;
    switch (s.op) {
    case UNION: return run_op<K, V, Cmp, UNION>(s);
    case INTERSECTION: return run_op<K, V, Cmp, INTERSECTION>(s);
    case DIFFERENCE: return run_op<K, V, Cmp, DIFFERENCE>(s);
    default: return run_op<K, V, Cmp, SYMMETRIC_DIFFERENCE>(s);
    }
  }
};

// Workspace bytes for keys K and values V, whatever the operation.
template <class K, class V>
size_t bytes_v(size_t na, size_t nb) {
  return layout<K, V, min_items_for<K, V>()>(na, nb).total;
}

#define RCCL_SET_DECLARE_KIND(NAME)                                                       \
  rccl_hip_status run_##NAME(const SetArgs &s, size_t value_bytes, bool descending);      \
  size_t bytes_##NAME(size_t na, size_t nb, size_t value_bytes);
RCCL_SET_DECLARE_KIND(u8)
RCCL_SET_DECLARE_KIND(i8)
RCCL_SET_DECLARE_KIND(u16)
RCCL_SET_DECLARE_KIND(i16)
RCCL_SET_DECLARE_KIND(u32)
RCCL_SET_DECLARE_KIND(i32)
RCCL_SET_DECLARE_KIND(f32)
RCCL_SET_DECLARE_KIND(u64)
RCCL_SET_DECLARE_KIND(i64)
RCCL_SET_DECLARE_KIND(f64)
#undef RCCL_SET_DECLARE_KIND

#define RCCL_SET_DEFINE_KIND(NAME, KT)                                                      \
  rccl_hip_status run_##NAME(const SetArgs &s, size_t value_bytes, bool descending) {       \
    using Desc = KindRunner<KT, true>;                                                      \
    using Asc = KindRunner<KT, false>;                                                      \
    if (descending) {                                                                       \
      RCCL_ORDERING_DISPATCH_VALUE(value_bytes, Desc, s)                                    \
    } else {                                                                                \
      RCCL_ORDERING_DISPATCH_VALUE(value_bytes, Asc, s)                                     \
    }                                                                                       \
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "set operation value bytes");         \
  }                                                                                         \
  size_t bytes_##NAME(size_t na, size_t nb, size_t value_bytes) {                           \
    switch (value_bytes) {                                                                  \
    case 0: return bytes_v<KT, ordering::NoValue>(na, nb);                                  \
    case 1: return bytes_v<KT, uint8_t>(na, nb);                                            \
    case 2: return bytes_v<KT, uint16_t>(na, nb);                                           \
    case 4: return bytes_v<KT, uint32_t>(na, nb);                                           \
    case 8: return bytes_v<KT, uint64_t>(na, nb);                                           \
    default: return bytes_v<KT, Value16>(na, nb);                                           \
    }                                                                                       \
  }

} // namespace set_ops
} // namespace rccl_hip
