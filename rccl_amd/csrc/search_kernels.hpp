// Vectorized binary search for gfx950: lower_bound / upper_bound of many
// needles in one sorted haystack (thrust::lower_bound / upper_bound over a
// range of values, which the reference's datalog callers use and
// rccl-thrust does not export: CCCL_RUST_CAPABILITY_CHECKLIST.md:107).
//
// lower_bound(x) = the first index i with !(h[i] < x); upper_bound(x) = the
// first i with x < h[i]; n when there is none. `<` is the natural order, its
// reverse, or the lexicographic order of [u32; N] rows.
//
// Design: one thread per needle, blocks striding over the needles. Every
// block first copies a sample of the haystack into LDS, element
// (s + 1) * step - 1 for s < SAMPLES with step = ceil(n / SAMPLES): the
// boundaries of an implicit search tree's top levels. A thread searches the sample in LDS, which brackets its answer in
// one step-long span, then finishes with a binary search over that span in
// global memory: ceil(log2(step)) dependent global loads instead of
// ceil(log2(n)).
#pragma once

#include <type_traits>

#include "ordering_common.hpp"
#include "record_rows.hpp"

namespace rccl_hip {
namespace search {

constexpr int THREADS = 256;

template <class K>
constexpr uint32_t samples_for() {
  // 16 KB of LDS per block at most.
  return static_cast<uint32_t>(16384 / sizeof(K));
}

// Predicate "item i belongs before the answer": h < x for lower_bound,
// !(x < h) for upper_bound. True on a prefix of a sorted haystack.
template <class K, class Cmp, bool UPPER>
struct Before {
  __device__ __forceinline__ bool operator()(const K &h, const K &x) const {
    const Cmp less{};
    if constexpr (UPPER) return !less(x, h);
    else return less(h, x);
  }
};

template <class K, class Cmp, bool UPPER, uint32_t SAMPLES>
__global__ void __launch_bounds__(THREADS)
search_kernel(const K *__restrict__ hay, size_t n, const K *__restrict__ needles, size_t m,
              uint64_t *__restrict__ out, size_t step) {
  __shared__ K sample[SAMPLES];
  const Before<K, Cmp, UPPER> before{};
  // Sample s is hay[(s + 1) * step - 1]; samples past the end are unused.
  const uint32_t used = static_cast<uint32_t>(std::min<size_t>(SAMPLES, n / step));
  for (uint32_t s = threadIdx.x; s < used; s += THREADS)
    sample[s] = hay[(size_t(s) + 1) * step - 1];
  __syncthreads();
  // Blocks stride over the needles, so the sample is loaded once per block.
  for (size_t q = size_t(blockIdx.x) * THREADS + threadIdx.x; q < m;
       q += size_t(gridDim.x) * THREADS) {
    const K x = needles[q];
    // First sample not before x.
    uint32_t lo = 0, hi = used;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      if (before(sample[mid], x)) lo = mid + 1;
      else hi = mid;
    }
    // Items [lo * step, (lo + 1) * step - 1) remain (to n past the last
    // sample); the item at (lo + 1) * step - 1, sample lo, is not before x.
    size_t a = size_t(lo) * step;
    size_t b = lo < used ? (size_t(lo) + 1) * step - 1 : n;
    while (a < b) {
      const size_t mid = a + (b - a) / 2;
      if (before(hay[mid], x)) a = mid + 1;
      else b = mid;
    }
    out[q] = a;
  }
}

struct SearchArgs {
  const void *hay, *needles;
  size_t n, m;
  uint64_t *out;
  bool upper;
  hipStream_t stream;
};

// Blocks per CU of the grid-striding search (enough waves to hide the
// global loads' latency).
constexpr size_t BLOCKS_PER_CU = 8;

template <class K, class Cmp>
rccl_hip_status run(const SearchArgs &a) {
  if (a.m == 0) return ok();
  constexpr uint32_t SAMPLES = samples_for<K>();
  const size_t step = std::max<size_t>(1, (a.n + SAMPLES - 1) / SAMPLES);
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess)
      err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_DRIVER, "search device", err);
  }
  const dim3 grid(static_cast<uint32_t>(
      std::min<size_t>((a.m + THREADS - 1) / THREADS, size_t(cus) * BLOCKS_PER_CU)));
  KernelTimer t("search", a.stream, a.m);
  if (a.upper)
    search_kernel<K, Cmp, true, SAMPLES><<<grid, THREADS, 0, a.stream>>>(
        static_cast<const K *>(a.hay), a.n, static_cast<const K *>(a.needles), a.m, a.out, step);
  else
    search_kernel<K, Cmp, false, SAMPLES><<<grid, THREADS, 0, a.stream>>>(
        static_cast<const K *>(a.hay), a.n, static_cast<const K *>(a.needles), a.m, a.out, step);
  return check_launch("search");
}

} // namespace search
} // namespace rccl_hip
