// Comparison sorts, merges and set operations for the CPU baseline (TEST
// INFRASTRUCTURE ONLY: loaded by tests/ and by the cpu_baseline leg of
// bench.py, never by the product).
//
// They restate the reference's host-side validation oracles: Rust
// slice::sort_unstable (rccl-cub/examples/device_radix_sort_keys_probe.rs:42),
// the stable sort_by_key of pairs (device_radix_sort_pairs_probe.rs:45), the
// hand-written two-pointer merge (device_ordering_probe.rs:89-102) and
// host_set_by (rccl-thrust/examples/set_operations_tests.rs:40-107), plus,
// for the multi-core baseline the north star names, rayon-style parallel
// sorts. Neither Rust nor rayon is in this image, so the substitutes are the
// C++ standard library (std::sort, std::stable_sort, std::merge, std::set_*:
// the same semantics, first input first on ties) and parallel sorts written
// here: one sort per thread over equal chunks, then rounds of pairwise
// merges, each merge split across threads along merge-path diagonals (stable
// when the chunk sorts are).
#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <thread>
#include <vector>

namespace {

// Number of items of a that precede the first `diag` outputs of merge(a, b)
// (a first on ties).
template <class T, class Less>
size_t merge_path(const T *a, size_t na, const T *b, size_t nb, size_t diag, Less less) {
  size_t lo = diag > nb ? diag - nb : 0, hi = std::min(diag, na);
  while (lo < hi) {
    const size_t mid = lo + (hi - lo) / 2;
    if (less(b[diag - 1 - mid], a[mid])) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// One merge task: merge a and b into out, producing output slice
// [d0, d1) of the merged sequence.
template <class T, class Less>
struct MergeSlice {
  const T *a, *b;
  size_t na, nb, d0, d1;
  T *out;
  Less less;
  void run() const {
    const size_t i0 = merge_path(a, na, b, nb, d0, less), i1 = merge_path(a, na, b, nb, d1, less);
    std::merge(a + i0, a + i1, b + (d0 - i0), b + (d1 - i1), out + d0, less);
  }
};

// Sort n items on `t` threads: chunk sorts with `chunk_sort`, then rounds of
// pairwise merges through a scratch buffer of n items.
template <class T, class Less, class ChunkSort>
void par_sort(T *keys, size_t n, unsigned t, Less less, ChunkSort chunk_sort) {
  if (n < 2 * size_t(t) || t == 1) {
    chunk_sort(keys, keys + n);
    return;
  }
  std::vector<size_t> bounds(t + 1);
  for (unsigned i = 0; i <= t; ++i) bounds[i] = n * i / t;
  {
    std::vector<std::thread> pool;
    for (unsigned i = 0; i < t; ++i)
      pool.emplace_back([&, i] { chunk_sort(keys + bounds[i], keys + bounds[i + 1]); });
    for (auto &th : pool) th.join();
  }
  std::vector<T> scratch(n);
  T *src = keys, *dst = scratch.data();
  // Merge runs pairwise until one run is left; each round splits every merge
  // into slices along merge-path diagonals, about `t` slices in all, and runs
  // them at once.
  while (bounds.size() > 2) {
    std::vector<size_t> next{0};
    std::vector<MergeSlice<T, Less>> tasks;
    for (size_t r = 0; r + 1 < bounds.size(); r += 2) {
      const size_t lo = bounds[r], mid = bounds[r + 1];
      const size_t hi = r + 2 < bounds.size() ? bounds[r + 2] : mid;
      const unsigned share = std::max<unsigned>(1, static_cast<unsigned>(t * (hi - lo) / n));
      for (unsigned k = 0; k < share; ++k)
        tasks.push_back(MergeSlice<T, Less>{src + lo, src + mid, mid - lo, hi - mid,
                                            (hi - lo) * k / share, (hi - lo) * (k + 1) / share,
                                            dst + lo, less});
      next.push_back(hi);
    }
    std::vector<std::thread> pool;
    for (const auto &m : tasks) pool.emplace_back([&m] { m.run(); });
    for (auto &th : pool) th.join();
    bounds.swap(next);
    std::swap(src, dst);
  }
  if (src != keys) std::copy(src, src + n, keys);
}

// A u64 key with its u32 value, ordered by key only.
struct Pair64 {
  uint64_t key;
  uint32_t value;
};
struct PairLess {
  bool operator()(const Pair64 &x, const Pair64 &y) const { return x.key < y.key; }
};
struct Pair32 {
  uint32_t key, value;
};

} // namespace

extern "C" {

// slice::sort_unstable substitute: one thread.
int oracle_sort_unstable_u32(uint32_t *keys, size_t n) {
  if (!keys && n) return -1;
  std::sort(keys, keys + n);
  return 0;
}

// Parallel sort substitute on `threads` threads (at least 1). Uses a scratch
// buffer of n keys.
int oracle_par_sort_unstable_u32(uint32_t *keys, size_t n, int threads) {
  if ((!keys && n) || threads < 1) return -1;
  par_sort(keys, n, static_cast<unsigned>(threads), std::less<uint32_t>(),
           [](uint32_t *b, uint32_t *e) { std::sort(b, e); });
  return 0;
}

// Stable sort of (u64 key, u32 value) pairs by key, the stable sort_by_key
// substitute, on `threads` threads (1: std::stable_sort). Keys and values are
// separate arrays, sorted in place; the pairs are packed into a buffer first.
int oracle_stable_sort_pairs_u64_u32(uint64_t *keys, uint32_t *values, size_t n, int threads) {
  if (((!keys || !values) && n) || threads < 1) return -1;
  std::vector<Pair64> p(n);
  for (size_t i = 0; i < n; ++i) p[i] = Pair64{keys[i], values[i]};
  par_sort(p.data(), n, static_cast<unsigned>(threads), PairLess(),
           [](Pair64 *b, Pair64 *e) { std::stable_sort(b, e, PairLess()); });
  for (size_t i = 0; i < n; ++i) {
    keys[i] = p[i].key;
    values[i] = p[i].value;
  }
  return 0;
}

// The reference's two-pointer merge of keys with payloads (first input first
// on equal keys), as std::merge over (key, value) records; one thread.
int oracle_merge_pairs_u32(const uint32_t *a, const uint32_t *av, size_t na, const uint32_t *b,
                           const uint32_t *bv, size_t nb, uint32_t *out, uint32_t *outv) {
  if (((!a || !av) && na) || ((!b || !bv) && nb) || ((!out || !outv) && na + nb)) return -1;
  std::vector<Pair32> pa(na), pb(nb), po(na + nb);
  for (size_t i = 0; i < na; ++i) pa[i] = Pair32{a[i], av[i]};
  for (size_t i = 0; i < nb; ++i) pb[i] = Pair32{b[i], bv[i]};
  std::merge(pa.begin(), pa.end(), pb.begin(), pb.end(), po.begin(),
             [](const Pair32 &x, const Pair32 &y) { return x.key < y.key; });
  for (size_t i = 0; i < na + nb; ++i) {
    out[i] = po[i].key;
    outv[i] = po[i].value;
  }
  return 0;
}

// host_set_by substitute for sorted u64 multisets: std::set_union (op 0),
// set_intersection (1), set_difference (2), set_symmetric_difference (3);
// one thread. Returns the output length, or -1.
long long oracle_std_set_op_u64(int op, const uint64_t *a, size_t na, const uint64_t *b,
                                size_t nb, uint64_t *out) {
  if ((!a && na) || (!b && nb) || (!out && na + nb)) return -1;
  uint64_t *end = out;
  switch (op) {
  case 0: end = std::set_union(a, a + na, b, b + nb, out); break;
  case 1: end = std::set_intersection(a, a + na, b, b + nb, out); break;
  case 2: end = std::set_difference(a, a + na, b, b + nb, out); break;
  case 3: end = std::set_symmetric_difference(a, a + na, b, b + nb, out); break;
  default: return -1;
  }
  return static_cast<long long>(end - out);
}

} // extern "C"
