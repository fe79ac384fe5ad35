// Comparison sorts for the CPU baseline (TEST INFRASTRUCTURE ONLY: loaded by
// tests/ and by the cpu_baseline leg of bench.py, never by the product).
//
// They restate the reference's host-side validation oracles for the keys-only
// radix sort: Rust slice::sort_unstable (rccl-cub/examples/
// device_radix_sort_keys_probe.rs:42) and, for the multi-core baseline the
// north star names, a rayon-style parallel sort. Neither Rust nor rayon is in
// this image, so the substitutes are std::sort (introsort; the order of u32
// keys is total, so any correct sort gives the same output) and a parallel
// sort written here: one std::sort per thread over equal chunks, then rounds
// of pairwise merges, each merge split across threads along merge-path
// diagonals.
#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <thread>
#include <vector>

namespace {

// Number of items of a that precede the first `diag` outputs of merge(a, b)
// (a first on ties).
size_t merge_path(const uint32_t *a, size_t na, const uint32_t *b, size_t nb, size_t diag) {
  size_t lo = diag > nb ? diag - nb : 0, hi = std::min(diag, na);
  while (lo < hi) {
    const size_t mid = lo + (hi - lo) / 2;
    if (b[diag - 1 - mid] < a[mid]) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// One merge task: merge a and b into out, producing output slice
// [d0, d1) of the merged sequence.
struct MergeSlice {
  const uint32_t *a, *b;
  size_t na, nb, d0, d1;
  uint32_t *out;
  void run() const {
    const size_t i0 = merge_path(a, na, b, nb, d0), i1 = merge_path(a, na, b, nb, d1);
    std::merge(a + i0, a + i1, b + (d0 - i0), b + (d1 - i1), out + d0);
  }
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
  const unsigned t = static_cast<unsigned>(threads);
  if (n < 2 * size_t(t) || t == 1) {
    std::sort(keys, keys + n);
    return 0;
  }
  std::vector<size_t> bounds(t + 1);
  for (unsigned i = 0; i <= t; ++i) bounds[i] = n * i / t;
  {
    std::vector<std::thread> pool;
    for (unsigned i = 0; i < t; ++i)
      pool.emplace_back([&, i] { std::sort(keys + bounds[i], keys + bounds[i + 1]); });
    for (auto &th : pool) th.join();
  }
  std::vector<uint32_t> scratch(n);
  uint32_t *src = keys, *dst = scratch.data();
  // Merge runs pairwise until one run is left; each round splits every merge
  // into slices along merge-path diagonals, about `threads` slices in all, and
  // runs them at once.
  while (bounds.size() > 2) {
    std::vector<size_t> next{0};
    std::vector<MergeSlice> tasks;
    for (size_t r = 0; r + 1 < bounds.size(); r += 2) {
      const size_t lo = bounds[r], mid = bounds[r + 1];
      const size_t hi = r + 2 < bounds.size() ? bounds[r + 2] : mid;
      const unsigned share = std::max<unsigned>(1, static_cast<unsigned>(t * (hi - lo) / n));
      for (unsigned k = 0; k < share; ++k)
        tasks.push_back(MergeSlice{src + lo, src + mid, mid - lo, hi - mid,
                                   (hi - lo) * k / share, (hi - lo) * (k + 1) / share, dst + lo});
      next.push_back(hi);
    }
    std::vector<std::thread> pool;
    for (const MergeSlice &m : tasks) pool.emplace_back([&m] { m.run(); });
    for (auto &th : pool) th.join();
    bounds.swap(next);
    std::swap(src, dst);
  }
  if (src != keys) std::copy(src, src + n, keys);
  return 0;
}

} // extern "C"
