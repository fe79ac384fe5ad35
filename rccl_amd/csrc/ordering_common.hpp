// Shared pieces of the comparison-based ordering kernels (merge, merge sort,
// set operations): key comparators, value payload types, and the dispatch of
// a runtime (key kind, order, value width) onto compile-time instantiations.
#pragma once

#include <algorithm>
#include <limits>
#include <type_traits>

#include "common.hpp"

namespace rccl_hip {
namespace ordering {

struct NoValue {};

// Natural order of the key type, or its reverse. Floats compare with IEEE
// `<`, so -0.0 and +0.0 are equivalent. This is the closure-free natural
// order of rccl-thrust/src/merge.rs:169-178 (Less iff a < b, Greater iff
// b < a, else Equal) and its reversal `|a, b| b.cmp(a)`.
template <class K, bool DESC>
struct Less {
  __device__ __forceinline__ bool operator()(const K &a, const K &b) const {
    if constexpr (DESC) return b < a;
    else return a < b;
  }
  // A key no other key comes after (padding for merge networks).
  __device__ static __forceinline__ K last() {
    return DESC ? std::numeric_limits<K>::lowest() : std::numeric_limits<K>::max();
  }
};

// Keys-only merges of integer keys can use a merge network: equal integer
// keys are identical bit patterns, so which copy of an equal key lands where
// cannot be observed and stability holds trivially. (Float keys are left out:
// -0.0 and +0.0 compare equal but differ in their bits.)
template <class K, class V, int ITEMS>
constexpr bool use_merge_network() {
  return std::is_integral<K>::value && std::is_same<V, NoValue>::value &&
         (ITEMS & (ITEMS - 1)) == 0;
}

// The ITEMS first keys, in order, of the merge of two sorted windows: a(i)
// and b(i) return the windows' i-th keys (Cmp::last() past their ends). The
// elementwise minimum of a and reversed b is bitonic and holds exactly the
// ITEMS first keys; a bitonic merge network sorts it. The loads are
// independent of each other, unlike a serial merge's.
template <class K, class Cmp, int ITEMS, class LoadA, class LoadB>
__device__ __forceinline__ void network_merge(K (&out)[ITEMS], LoadA a, LoadB b, Cmp less) {
  K x[ITEMS], y[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    x[i] = a(i);
    y[i] = b(ITEMS - 1 - i);
  }
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) out[i] = less(y[i], x[i]) ? y[i] : x[i];
#pragma unroll
  for (int s = ITEMS / 2; s > 0; s >>= 1) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if ((i & s) == 0) {
        const K lo = out[i], hi = out[i + s];
        const bool swap = less(hi, lo);
        out[i] = swap ? hi : lo;
        out[i + s] = swap ? lo : hi;
      }
    }
  }
}

// Choice between two keys. Aggregate keys (record rows) overload it in their
// own namespace with a per-word choice, found by argument-dependent lookup, so
// the choice stays in registers instead of selecting between stack addresses.
template <class K>
__device__ __forceinline__ K pick(bool c, const K &x, const K &y) {
  return c ? x : y;
}

template <class T>
__device__ __forceinline__ T load_or(const T *p, size_t i, size_t n, T fallback) {
  return i < n ? p[i] : fallback;
}

// Merge-path split of diagonal `diag` between sorted A[0, na) and
// B[0, nb): the number of A items among the first `diag` merged outputs.
// B moves ahead only when strictly before A, so equal keys take A first
// (rccl-memory/src/device.rs:25-71, rccl-cub/src/ordering_backend/merge.rs:16-24).
template <class K, class Cmp, class ReadA, class ReadB>
__device__ __forceinline__ size_t merge_path(ReadA a, size_t na, ReadB b, size_t nb, size_t diag,
                                             Cmp less) {
  size_t lo = diag > nb ? diag - nb : 0;
  size_t hi = diag < na ? diag : na;
  while (lo < hi) {
    const size_t mid = lo + (hi - lo) / 2;
    if (less(b(diag - 1 - mid), a(mid)))
      hi = mid;
    else
      lo = mid + 1;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// Sampled merge path (integer keys). Every probe of a plain merge-path search
// over HBM fetches its own random line, and neighbouring searches share none.
// Here the top levels go to a shared sample instead:
//   merge_sample_kernel  for every MERGE_SAMPLE-th item a_k = A[k*S], m_k =
//                        the number of sampled B items B[m*S] strictly before
//                        it (a search over the sampled positions, which stay
//                        in L2)
//   sampled_merge_path   a_k's merged position is posA(k*S) = k*S + #{B < a_k},
//                        and #{B < a_k} lies in [(m_k - 1)*S + 1, m_k*S] (or
//                        is 0 when m_k = 0): bounds L_k <= posA <= U_k. The A
//                        split of diagonal d is i* = #{i : posA(i) < d}, so
//                        U_k < d gives i* > k*S and L_k >= d gives i* <= k*S.
//                        With kk the first sample whose U reaches d,
//                        i* > (kk - 1)*S; and since L_{k+1} > U_k whenever
//                        m_k > 0, sample kk or kk + 1 has L >= d, which caps
//                        i* at most 2*S above the lower bound. The merge-path
//                        search then runs in that window only.
// Floats keep the plain search: NaN makes the order partial.
// ---------------------------------------------------------------------------
#ifndef RCCL_MERGE_SAMPLE
#define RCCL_MERGE_SAMPLE 2048
#endif
constexpr size_t MERGE_SAMPLE = RCCL_MERGE_SAMPLE;

template <class K>
constexpr bool sampled_partition_for() {
  return std::is_integral<K>::value;
}

// Samples of an A of `na` items (entries of the m array).
__host__ __device__ inline size_t merge_samples(size_t na) { return (na + MERGE_SAMPLE - 1) / MERGE_SAMPLE; }

// ---------------------------------------------------------------------------
// Group searches. A search over HBM whose every probe is a dependent round
// trip is latency-bound. The searches below run on the 8 lanes of an aligned
// lane group, which all hold the same search: each round the lanes probe 8
// evenly spaced points and a ballot counts those still before the answer, a
// 9-ary search: about log9 of the range in dependent rounds instead of log2.
// ---------------------------------------------------------------------------
constexpr uint32_t SEARCH_GROUP = 8;

// First x in [lo, hi) with !before(x), or hi, where `before` holds on a
// prefix of the range (on any other predicate the result stays in [lo, hi]).
// Every lane of the group calls it with the same arguments.
template <class Before>
__device__ __forceinline__ size_t group_first_not(size_t lo, size_t hi, Before before) {
  const uint32_t lane = lane_id();
  const uint32_t sub = lane & (SEARCH_GROUP - 1u), base = lane & ~(SEARCH_GROUP - 1u);
  while (lo < hi) {
    const size_t span = hi - lo;
    if (span <= SEARCH_GROUP) {
      const bool bf = sub < span && before(lo + sub);
      return lo + __builtin_popcount(static_cast<uint32_t>(__ballot(bf) >> base) & 0xFFu);
    }
    const bool bf = before(lo + (size_t(sub) + 1) * span / 9);
    const size_t cnt = __builtin_popcount(static_cast<uint32_t>(__ballot(bf) >> base) & 0xFFu);
    // Probe j sits at lo + (j + 1) * span / 9: the answer lies after probe
    // cnt - 1 and at or before probe cnt.
    const size_t l0 = lo;
    if (cnt > 0) lo = l0 + cnt * span / 9 + 1;
    if (cnt < SEARCH_GROUP) hi = l0 + (cnt + 1) * span / 9;
  }
  return lo;
}

// Eight lanes per sample (group_first_not): with one sample per 2,048 items
// the searches are few and latency-bound (C4: 0.016 -> 0.014 ms, C5 0.013-0.015
// -> 0.010-0.011 ms against one thread per sample).
template <class K, class Cmp>
__global__ void __launch_bounds__(256)
merge_sample_kernel(const K *__restrict__ a, size_t na, const K *__restrict__ b, size_t nb,
                    uint32_t *__restrict__ m_out) {
  const size_t k = (size_t(blockIdx.x) * 256 + threadIdx.x) / SEARCH_GROUP;
  const size_t ka = merge_samples(na), kb = merge_samples(nb);
  if (k >= ka) return;  // whole groups
  const K x = a[k * MERGE_SAMPLE];
  const Cmp less{};
  // First sampled B position not before x.
  const size_t lo =
      group_first_not(0, kb, [&](size_t j) { return less(b[j * MERGE_SAMPLE], x); });
  if (threadIdx.x % SEARCH_GROUP == 0) m_out[k] = static_cast<uint32_t>(lo);
}
inline size_t merge_sample_blocks(size_t na) {
  return (merge_samples(na) * SEARCH_GROUP + 255) / 256;
}

// merge_path of diagonal d, searched in the window the samples allow. One
// thread per diagonal: with a boundary per merge tile (131,073 for C4) the
// searches are bound by their random line reads, which a group search would
// multiply (8 lanes per boundary: 0.069 -> 0.099 ms for C4).
template <class K, class Cmp, class ReadA, class ReadB>
__device__ __forceinline__ size_t sampled_merge_path(ReadA a, size_t na, ReadB b, size_t nb,
                                                     size_t d, const uint32_t *__restrict__ m,
                                                     Cmp less) {
  constexpr size_t S = MERGE_SAMPLE;
  const size_t ka = merge_samples(na);
  auto upper = [&](size_t k) { return k * S + std::min(nb, size_t(m[k]) * S); };
  auto lower = [&](size_t k) { return k * S + (m[k] ? (size_t(m[k]) - 1) * S + 1 : size_t(0)); };
  size_t lo = 0, hi = ka;  // kk: first sample with upper(k) >= d
  while (lo < hi) {
    const size_t mid = lo + (hi - lo) / 2;
    if (upper(mid) < d) lo = mid + 1; else hi = mid;
  }
  const size_t kk = lo;
  size_t ilo = d > nb ? d - nb : 0;
  size_t ihi = d < na ? d : na;
  if (kk > 0) ilo = std::max(ilo, (kk - 1) * S + 1);
  if (kk < ka) {
    if (lower(kk) >= d) ihi = std::min(ihi, kk * S);
    else if (kk + 1 < ka) ihi = std::min(ihi, (kk + 1) * S);
  }
  // merge_path restricted to [ilo, ihi].
  while (ilo < ihi) {
    const size_t mid = ilo + (ihi - ilo) / 2;
    if (less(b(d - 1 - mid), a(mid))) ihi = mid; else ilo = mid + 1;
  }
  return ilo;
}

// 32-bit variant for LDS-resident slices.
template <class K, class Cmp>
__device__ __forceinline__ uint32_t merge_path_lds(const K *a, uint32_t na, const K *b, uint32_t nb,
                                                   uint32_t diag, Cmp less) {
  uint32_t lo = diag > nb ? diag - nb : 0u;
  uint32_t hi = diag < na ? diag : na;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (less(b[diag - 1 - mid], a[mid]))
      hi = mid;
    else
      lo = mid + 1;
  }
  return lo;
}

// Padded LDS index for blocked <-> striped transposes: one pad slot after
// every ITEMS items makes a thread's blocked run start ITEMS + 1 slots after
// its neighbour's, so both access patterns spread over the banks.
template <int ITEMS>
__device__ __forceinline__ uint32_t padded(uint32_t i) {
  return i + i / ITEMS;
}
constexpr uint32_t padded_size(uint32_t n, uint32_t items) { return n + n / items + 1; }

} // namespace ordering

// Runtime value width -> RUNNER::run<V>(args...) (RUNNER is a type name).
#define RCCL_ORDERING_DISPATCH_VALUE(VB, RUNNER, ...)                                    \
  switch (VB) {                                                                          \
  case 0: return RUNNER::run<ordering::NoValue>(__VA_ARGS__);                            \
  case 1: return RUNNER::run<uint8_t>(__VA_ARGS__);                                      \
  case 2: return RUNNER::run<uint16_t>(__VA_ARGS__);                                     \
  case 4: return RUNNER::run<uint32_t>(__VA_ARGS__);                                     \
  case 8: return RUNNER::run<uint64_t>(__VA_ARGS__);                                     \
  case 16: return RUNNER::run<Value16>(__VA_ARGS__);                                     \
  default: break;                                                                        \
  }

} // namespace rccl_hip
