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
// block first copies a sample of the searched array into LDS, element
// (s + 1) * step - 1 for s < SAMPLES with step = ceil(len / SAMPLES): the
// boundaries of an implicit search tree's top levels. A thread searches the
// sample in LDS, which brackets its answer in one step-long span, then
// finishes with a binary search over that span in global memory.
//
// Large haystacks with many needles are searched through a two-level index
// built per call, a B+-tree over cache lines: index[c] is the last item of
// the haystack's c-th 128-byte chunk (CHUNK items), and lines[j] the last
// item of its j-th run of CHUNK chunks (the last entry of index line j). The
// sampled search above runs over `lines` (a CHUNK^2-th of the haystack, hot
// in L2) and yields the first index line whose last entry is not before x;
// a search inside that index line gives the chunk, and one inside the chunk
// the answer: one cache line of each level. Searching the haystack directly
// costs a cache line per level below the LDS sample (about ten at 2^26
// items), and random needles share almost none of them.
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

// Haystack items per index entry: one 128-byte cache line's worth.
template <class K>
constexpr size_t chunk_items() {
  return sizeof(K) >= 128 ? 1 : 128 / sizeof(K);
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

// index[c] = hay[min((c + 1) * CHUNK, n) - 1] for c < chunks, and
// lines[j] = index[min((j + 1) * CHUNK, chunks) - 1] for j < ceil(chunks /
// CHUNK), written by the thread of that index entry.
template <class K>
__global__ void __launch_bounds__(THREADS)
index_kernel(const K *__restrict__ hay, size_t n, K *__restrict__ index, size_t chunks,
             K *__restrict__ lines) {
  constexpr size_t CHUNK = chunk_items<K>();
  for (size_t c = size_t(blockIdx.x) * THREADS + threadIdx.x; c < chunks;
       c += size_t(gridDim.x) * THREADS) {
    const K v = hay[std::min((c + 1) * CHUNK, n) - 1];
    index[c] = v;
    if ((c + 1) % CHUNK == 0 || c + 1 == chunks) lines[c / CHUNK] = v;
  }
}

// First position in [a, b] whose item is not before x, given that arr[b] is
// not before x (a sorted run inside one cache line).
template <class K, class B>
__device__ __forceinline__ size_t first_in_line(const K *__restrict__ arr, size_t a, size_t b,
                                                const K &x, B before) {
  while (a < b) {
    const size_t mid = a + (b - a) / 2;
    if (before(arr[mid], x)) a = mid + 1;
    else b = mid;
  }
  return a;
}

// First position p < len with !before(arr[p], x), or len: the LDS sample
// (sample[s] = arr[(s + 1) * step - 1], s < used) brackets p in one span,
// searched in global memory.
template <class K, class B, uint32_t SAMPLES>
__device__ __forceinline__ size_t first_not_before(const K *__restrict__ arr, size_t len,
                                                   const K *sample, uint32_t used, size_t step,
                                                   const K &x, B before) {
  uint32_t lo = 0, hi = used;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (before(sample[mid], x)) lo = mid + 1;
    else hi = mid;
  }
  // Items [lo * step, (lo + 1) * step - 1) remain (to len past the last
  // sample); the item at (lo + 1) * step - 1, sample lo, is not before x.
  size_t a = size_t(lo) * step;
  size_t b = lo < used ? (size_t(lo) + 1) * step - 1 : len;
  while (a < b) {
    const size_t mid = a + (b - a) / 2;
    if (before(arr[mid], x)) a = mid + 1;
    else b = mid;
  }
  return a;
}

// Items searched a whole line at a time: 4, 8 or 16 bytes, a whole number
// per 16-byte lane read (narrower ones would need a register per item).
template <class K>
constexpr bool line_items() {
  return sizeof(K) >= 4 && 16 % sizeof(K) == 0;
}

// Shuffle of a trivially copyable item, one 32-bit word at a time.
template <class T>
__device__ __forceinline__ T shfl_item(const T &v, int src) {
  static_assert(sizeof(T) % 4 == 0, "whole words");
  uint32_t w[sizeof(T) / 4];
  __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 4; ++i)
    w[i] = static_cast<uint32_t>(__shfl(static_cast<int>(w[i]), src, 64));
  T r;
  __builtin_memcpy(&r, w, sizeof(T));
  return r;
}

// For every lane of the (fully active) wave: how many of the first `valid`
// items of the 128-byte line at base + start are before the lane's x. Eight
// lanes read each line together, 16 bytes a lane, and add their counts with
// three butterfly shuffles; eight rounds cover the wave's 64 lines, all eight
// loads issued before the first is used. A load instruction so touches eight
// lines (one per needle) instead of 64: lane-private reads of whole lines
// (eight 16-byte loads per lane per line) were bound by the address
// processing of 64 lines per instruction. `base` is 16-byte aligned and
// every line lies inside its array (a lane with nothing to search passes
// start 0 and valid 0).
template <class K, class B>
__device__ __forceinline__ uint32_t group_count_before(const K *__restrict__ base, size_t start,
                                                       uint32_t valid, const K &x, B before,
                                                       uint32_t lane) {
  static_assert(16 % sizeof(K) == 0, "whole items per 16 bytes");
  constexpr int PER = 16 / sizeof(K);
  const uint32_t sub = lane & 7u, grp = lane >> 3;
  uint4 raw[8];
  uint32_t vld[8];
  K xr[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int src = r * 8 + static_cast<int>(grp);
    const size_t st = shfl_item(start, src);
    vld[r] = static_cast<uint32_t>(__shfl(static_cast<int>(valid), src, 64));
    xr[r] = shfl_item(x, src);
    raw[r] = reinterpret_cast<const uint4 *>(base + st)[sub];
  }
  uint32_t mine = 0;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    K v[PER];
    __builtin_memcpy(v, &raw[r], 16);
    uint32_t c = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      c += (sub * PER + uint32_t(i) < vld[r] && before(v[i], xr[r])) ? 1u : 0u;
    c += static_cast<uint32_t>(__shfl_xor(static_cast<int>(c), 1, 64));
    c += static_cast<uint32_t>(__shfl_xor(static_cast<int>(c), 2, 64));
    c += static_cast<uint32_t>(__shfl_xor(static_cast<int>(c), 4, 64));
    // Group g now holds the count of lane 8r + g's line; lane 8r + g takes
    // it from the group's first lane.
    const uint32_t got = static_cast<uint32_t>(__shfl(static_cast<int>(c), int((lane & 7u) << 3), 64));
    if ((lane >> 3) == uint32_t(r)) mine = got;
  }
  return mine;
}

// Indexed search for items of 4, 8 or 16 bytes (all keys of 4 or 8 bytes,
// rows of arity 2 and 4) whose `lines` array the LDS sample covers: the
// sample (the last entry of every 128-byte line of `lines`) brackets the line
// of `lines`, and each level below is one line read cooperatively
// (group_count_before): the line of `lines` gives the index line, that gives
// the haystack chunk, and the chunk the answer. A chunk that is not whole or
// a haystack that is not 16-byte aligned is finished by binary search. The
// needle loop is wave-uniform (the shuffles need every lane).
template <class K, class Cmp, bool UPPER, uint32_t SAMPLES>
__global__ void __launch_bounds__(THREADS)
line_search_kernel(const K *__restrict__ hay, size_t n, const K *__restrict__ index,
                   size_t chunks, const K *__restrict__ lines, size_t nlines,
                   const K *__restrict__ needles, size_t m, uint64_t *__restrict__ out,
                   bool hay16) {
  __shared__ K sample[SAMPLES];
  constexpr size_t CHUNK = chunk_items<K>();
  const Before<K, Cmp, UPPER> before{};
  const uint32_t used = static_cast<uint32_t>(std::min<size_t>(SAMPLES, nlines / CHUNK));
  for (uint32_t s = threadIdx.x; s < used; s += THREADS)
    sample[s] = lines[(size_t(s) + 1) * CHUNK - 1];
  __syncthreads();
  const uint32_t lane = threadIdx.x & 63u;
  for (size_t b0 = size_t(blockIdx.x) * THREADS; b0 < m; b0 += size_t(gridDim.x) * THREADS) {
    const size_t q = b0 + threadIdx.x;
    const K x = needles[std::min(q, m - 1)];
    // Line L of `lines`: the first whose last entry is not before x (L ==
    // used is the partial last line, or past the end).
    uint32_t lo = 0, hi = used;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      if (before(sample[mid], x)) lo = mid + 1;
      else hi = mid;
    }
    const size_t l0 = size_t(lo) * CHUNK;
    bool go = l0 < nlines;
    const size_t j =
        l0 + group_count_before(lines, go ? l0 : 0,
                                go ? uint32_t(std::min(CHUNK, nlines - l0)) : 0u, x, before,
                                lane);
    go = go && j < nlines;
    const size_t i0 = go ? j * CHUNK : 0;
    // Below chunks for a sorted haystack; clamped so that an unsorted one
    // (unspecified results) still reads in bounds.
    const size_t c = std::min(
        chunks - 1, i0 + group_count_before(index, i0,
                                            go ? uint32_t(std::min(CHUNK, chunks - i0)) : 0u,
                                            x, before, lane));
    const size_t h0 = c * CHUNK;
    const bool whole = go && h0 + CHUNK <= n;
    size_t p = n;
    if (hay16) {  // uniform
      const uint32_t k = group_count_before(hay, whole ? h0 : 0, whole ? uint32_t(CHUNK) : 0u,
                                            x, before, lane);
      if (whole) p = h0 + k;
    }
    if (go && !(hay16 && whole)) p = first_in_line(hay, h0, std::min(h0 + CHUNK, n) - 1, x, before);
    if (q < m) out[q] = p;
  }
}

// INDEXED: the sampled search runs over the index lines and finishes with
// one line of the index and one chunk of the haystack, each by binary search;
// otherwise it runs over the haystack itself.
template <class K, class Cmp, bool UPPER, uint32_t SAMPLES, bool INDEXED>
__global__ void __launch_bounds__(THREADS)
search_kernel(const K *__restrict__ hay, size_t n, const K *__restrict__ index, size_t chunks,
              const K *__restrict__ lines, size_t nlines, const K *__restrict__ needles,
              size_t m, uint64_t *__restrict__ out, size_t step) {
  __shared__ K sample[SAMPLES];
  constexpr size_t CHUNK = chunk_items<K>();
  const Before<K, Cmp, UPPER> before{};
  const K *arr = INDEXED ? lines : hay;
  const size_t len = INDEXED ? nlines : n;
  // Sample s is arr[(s + 1) * step - 1]; samples past the end are unused.
  const uint32_t used = static_cast<uint32_t>(std::min<size_t>(SAMPLES, len / step));
  for (uint32_t s = threadIdx.x; s < used; s += THREADS)
    sample[s] = arr[(size_t(s) + 1) * step - 1];
  __syncthreads();
  // Blocks stride over the needles, so the sample is loaded once per block.
  for (size_t q = size_t(blockIdx.x) * THREADS + threadIdx.x; q < m;
       q += size_t(gridDim.x) * THREADS) {
    const K x = needles[q];
    size_t p = first_not_before<K, Before<K, Cmp, UPPER>, SAMPLES>(arr, len, sample, used, step,
                                                                   x, before);
    if constexpr (INDEXED) {
      // Every index line before j ends with an entry before x, so all of its
      // chunks end before x and so do all their items; line j's last entry
      // is not. Likewise inside the line for the chunk, and inside the chunk
      // for the answer; n when no line qualifies.
      const size_t j = p;
      if (j == nlines) {
        p = n;
      } else {
        const size_t c = first_in_line(index, j * CHUNK, std::min((j + 1) * CHUNK, chunks) - 1,
                                       x, before);
        p = first_in_line(hay, c * CHUNK, std::min((c + 1) * CHUNK, n) - 1, x, before);
      }
    }
    out[q] = p;
  }
}

struct SearchArgs {
  const void *hay, *needles;
  size_t n, m;
  uint64_t *out;
  bool upper;
  void *ws;
  size_t ws_bytes;
  hipStream_t stream;
};

// Blocks per CU of the grid-striding search (enough waves to hide the
// global loads' latency).
constexpr size_t BLOCKS_PER_CU = 8;

// The index pays when the haystack is larger than the LDS sample can bracket
// to one chunk, and there are enough needles to repay reading the haystack
// once to build it (each indexed needle saves several cache lines).
template <class K>
size_t index_chunks(size_t n) {
  const size_t chunks = (n + chunk_items<K>() - 1) / chunk_items<K>();
  return chunks > samples_for<K>() ? chunks : 0;
}
template <class K>
size_t index_lines(size_t chunks) {
  return (chunks + chunk_items<K>() - 1) / chunk_items<K>();
}
template <class K>
size_t workspace_bytes(size_t n) {
  const size_t chunks = index_chunks<K>(n);
  if (chunks == 0) return 0;
  return align_up(chunks * sizeof(K), 256) + align_up(index_lines<K>(chunks) * sizeof(K), 256);
}
template <class K>
bool use_index(size_t n, size_t m) {
  const size_t chunks = index_chunks<K>(n);
  return chunks && m >= chunks / 4;
}

template <class K, class Cmp>
rccl_hip_status run(const SearchArgs &a) {
  if (a.m == 0) return ok();
  constexpr uint32_t SAMPLES = samples_for<K>();
  const bool indexed = use_index<K>(a.n, a.m);
  const size_t chunks = indexed ? index_chunks<K>(a.n) : 0;
  if (indexed && (!a.ws || a.ws_bytes < workspace_bytes<K>(a.n)))
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "search workspace",
                     workspace_bytes<K>(a.n), a.ws_bytes);
  const size_t nlines = indexed ? index_lines<K>(chunks) : 0;
  const size_t len = indexed ? nlines : a.n;
  constexpr size_t CHUNK = chunk_items<K>();
  const bool line_search =
      indexed && line_items<K>() && (nlines + CHUNK - 1) / CHUNK <= SAMPLES;
  const size_t step =
      line_search ? CHUNK : std::max<size_t>(1, (len + SAMPLES - 1) / SAMPLES);
  const bool hay16 = reinterpret_cast<uintptr_t>(a.hay) % 16 == 0;
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess)
      err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_DRIVER, "search device", err);
  }
  const K *hay = static_cast<const K *>(a.hay);
  K *index = static_cast<K *>(a.ws);
  K *lines = indexed ? reinterpret_cast<K *>(static_cast<unsigned char *>(a.ws) +
                                             align_up(chunks * sizeof(K), 256))
                     : nullptr;
  if (indexed) {
    KernelTimer t("search_index", a.stream, chunks);
    const dim3 grid(static_cast<uint32_t>(
        std::min<size_t>((chunks + THREADS - 1) / THREADS, size_t(cus) * BLOCKS_PER_CU)));
    index_kernel<K><<<grid, THREADS, 0, a.stream>>>(hay, a.n, index, chunks, lines);
    RCCL_HIP_TRY(check_launch("search index"));
  }
  const dim3 grid(static_cast<uint32_t>(
      std::min<size_t>((a.m + THREADS - 1) / THREADS, size_t(cus) * BLOCKS_PER_CU)));
  KernelTimer t("search", a.stream, a.m);
  const K *needles = static_cast<const K *>(a.needles);
  auto launch = [&](auto upper, auto idx) {
    search_kernel<K, Cmp, decltype(upper)::value, SAMPLES, decltype(idx)::value>
        <<<grid, THREADS, 0, a.stream>>>(hay, a.n, index, chunks, lines, nlines, needles, a.m,
                                         a.out, step);
  };
  using T = std::true_type;
  using F = std::false_type;
  if (line_search) {
    if constexpr (line_items<K>()) {
      if (a.upper)
        line_search_kernel<K, Cmp, true, SAMPLES><<<grid, THREADS, 0, a.stream>>>(
            hay, a.n, index, chunks, lines, nlines, needles, a.m, a.out, hay16);
      else
        line_search_kernel<K, Cmp, false, SAMPLES><<<grid, THREADS, 0, a.stream>>>(
            hay, a.n, index, chunks, lines, nlines, needles, a.m, a.out, hay16);
    }
  } else if (indexed) {
    if (a.upper) launch(T{}, T{});
    else launch(F{}, T{});
  } else {
    if (a.upper) launch(T{}, F{});
    else launch(F{}, F{});
  }
  return check_launch("search");
}

} // namespace search
} // namespace rccl_hip
