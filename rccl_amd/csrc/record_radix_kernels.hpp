// Multi-word LSD radix sort of [u32; N] rows (with an optional payload), the
// large-input path of the record sort.
//
// The reference sorts rows with DeviceMergeSort and an unrolled lexicographic
// comparator (rccl-thrust/src/record_sort.rs:88-115,144-366). A stable LSD
// radix sort over the row's bytes, least significant first (last column's low
// byte first, first column's high byte last), yields the same stable
// ascending lexicographic order with O(1) passes over the data instead of
// O(log n). Relation rows hold interned ids, so most high bytes are constant
// across the input; those passes are skipped on the device:
//   init        zero the per-pass bins and a completion count
//   histogram   one read of the rows counts all 4N byte positions' digits
//               (a wave whose lanes share a digit adds once); the last block
//               to finish then plans the passes: bins -> exclusive offsets; a
//               pass whose digit is the same for every row is inactive; each
//               active pass gets its source and destination buffer so the
//               last one writes the output (an in-place sort needs an even
//               number of active passes, an out-of-place one at least one: a
//               trivial pass is activated when needed, and is then a stable
//               copy)
//   onesweep    one launch per byte position; inactive passes return at once,
//               active ones run the scalar sort's onesweep tile with rows as
//               keys (radix_kernels.hpp)
#pragma once

#include "radix_kernels.hpp"
#include "record_rows.hpp"

namespace rccl_hip {
namespace record_sort {

using radix::BINS;
using radix::LookbackBuf;

// Source/destination buffers: 0 the input, 1 the output, 2 the scratch.
using radix::PassPlan;

// Onesweep policy for rows: 512 threads x 4 rows = 2048-row tiles for every
// arity (at most 48 KB of staged rows, two blocks per CU). At the reference
// workload's 2^20 rows this measured best among 1024- to 4096-row tiles:
// larger tiles leave CUs idle, smaller ones lengthen the look-back.
#ifndef RCCL_RECORD_RADIX_THREADS
#define RCCL_RECORD_RADIX_THREADS 512
#endif
#ifndef RCCL_RECORD_RADIX_ITEMS
#define RCCL_RECORD_RADIX_ITEMS 4
#endif
// Below this many rows the merge sort (fewer launches) is used.
#ifndef RCCL_RECORD_RADIX_MIN_ROWS
#define RCCL_RECORD_RADIX_MIN_ROWS 65536
#endif
constexpr int RADIX_THREADS = RCCL_RECORD_RADIX_THREADS;
constexpr size_t RADIX_MIN_ROWS = RCCL_RECORD_RADIX_MIN_ROWS;
// Look-back counts are 30-bit; larger inputs take the merge sort.
constexpr size_t RADIX_MAX_ROWS = (size_t(1) << 30) - 1;

template <int N, class Val>
constexpr int radix_items() {
  constexpr size_t vb = std::is_same<Val, radix::NoValue>::value ? 0 : sizeof(Val);
  constexpr size_t elem = 4 * N > vb ? 4 * N : vb;
  static_assert(size_t(RADIX_THREADS) * RCCL_RECORD_RADIX_ITEMS * elem <= 64 * 1024,
                "the staged tile must leave room for two blocks per CU");
  return RCCL_RECORD_RADIX_ITEMS;
}

// ---------------------------------------------------------------------------
// init: zero the bins and the histogram's completion counter.
// ---------------------------------------------------------------------------
namespace {
__global__ void __launch_bounds__(256) record_init_kernel(uint32_t *words, uint32_t count) {
  for (uint32_t i = threadIdx.x; i < count; i += 256) words[i] = 0;
}
} // namespace

// ---------------------------------------------------------------------------
// histogram + plan. Every block counts a share of the rows into LDS and adds
// its counts to the bins; the last block to finish then turns the bins into
// exclusive offsets and writes the pass plan.
// ---------------------------------------------------------------------------
constexpr int HIST_THREADS = 1024;
constexpr int HIST_ITEMS = 4;
static_assert(HIST_THREADS >= BINS, "the plan uses one thread per digit");

// Turns the bins into exclusive offsets and writes the pass plan. Called by
// every thread of one block; threads past BINS only join the barriers.
template <int N>
__device__ __forceinline__ void write_plan(uint32_t *__restrict__ bins, uint32_t n,
                                           PassPlan *__restrict__ plan, uint32_t plan_flags) {
  constexpr int P = 4 * N;
  __shared__ uint32_t s_wave[P][BINS / 64];
  __shared__ uint32_t s_trivial[P];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const bool digit_thread = tid < BINS;
  uint32_t c[P], inc[P];
  if (digit_thread) {
#pragma unroll
    for (int p = 0; p < P; ++p) c[p] = load_agent(&bins[p * BINS + tid]);
  }
  if (tid < P) s_trivial[tid] = 0;
  __syncthreads();
  if (digit_thread) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      inc[p] = wave_inclusive_sum(c[p], lane);
      if (lane == 63) s_wave[p][tid >> 6] = inc[p];
      if (c[p] == n) s_trivial[p] = 1;  // one digit holds every row
    }
  }
  __syncthreads();
  if (!digit_thread) return;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    uint32_t excl = inc[p] - c[p];
    for (uint32_t w = 0; w < (tid >> 6); ++w) excl += s_wave[p][w];
    bins[p * BINS + tid] = excl;
  }
  if (tid != 0) return;
  uint32_t trivial = 0;
  for (int p = 0; p < P; ++p) trivial |= s_trivial[p] ? (1u << p) : 0u;
  radix::assign_plan(P, trivial, plan_flags, plan);
}

// Adds one wave's digits of byte `byte` of a column word to the LDS
// histogram row `h`. x = w ^ w0, where w0 is the first active lane's word:
// when no lane's byte differs from w0's, the first lane adds the lane count
// once; otherwise every lane adds 1.
__device__ __forceinline__ void count_byte(uint32_t *h, uint32_t w, uint32_t w0, uint32_t x,
                                           int byte, bool leader, uint32_t cnt) {
  const uint32_t shift = 8u * uint32_t(byte);
  if (__ballot(((x >> shift) & 0xFFu) != 0u) == 0) {
    if (leader)
      __hip_atomic_fetch_add(&h[(w0 >> shift) & 0xFFu], cnt, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
  } else {
    __hip_atomic_fetch_add(&h[(w >> shift) & 0xFFu], 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

template <int N>
__global__ void __launch_bounds__(HIST_THREADS)
row_histogram_kernel(const Row<N> *__restrict__ rows, size_t n, uint32_t *__restrict__ bins,
                     uint32_t *__restrict__ done, PassPlan *__restrict__ plan, uint32_t plan_flags,
                     uint32_t *__restrict__ zero_words, size_t zero_count) {
  constexpr int P = 4 * N;
  __shared__ uint32_t hist[P * BINS];  // [pass][digit], pass 0 = last column's low byte
  __shared__ uint32_t s_last;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  for (uint32_t i = tid; i < P * BINS; i += HIST_THREADS) hist[i] = 0;
  for (size_t i = size_t(blockIdx.x) * HIST_THREADS + tid; i < zero_count;
       i += size_t(gridDim.x) * HIST_THREADS)
    zero_words[i] = 0;
  __syncthreads();

  constexpr size_t CHUNK = size_t(HIST_THREADS) * HIST_ITEMS;
  for (size_t base = size_t(blockIdx.x) * CHUNK; base < n; base += size_t(gridDim.x) * CHUNK) {
    Row<N> r[HIST_ITEMS];
#pragma unroll
    for (int j = 0; j < HIST_ITEMS; ++j)
      r[j] = rows[min(base + size_t(j) * HIST_THREADS + tid, n - 1)];
#pragma unroll
    for (int j = 0; j < HIST_ITEMS; ++j) {
      if (base + size_t(j) * HIST_THREADS + tid >= n) continue;
      // Lanes still here hold valid rows; the byte branches are wave-uniform.
      const uint64_t act = __ballot(1);
      const bool leader = lane == static_cast<uint32_t>(__builtin_ctzll(act));
      const uint32_t cnt = static_cast<uint32_t>(__popcll(act));
#pragma unroll
      for (int c = 0; c < N; ++c) {
        const uint32_t w = r[j].w[c];
        const uint32_t w0 = __builtin_amdgcn_readfirstlane(w);
        const uint32_t x = w ^ w0;
        uint32_t *h = &hist[(N - 1 - c) * 4 * BINS];
#pragma unroll
        for (int b = 0; b < 4; ++b) count_byte(h + b * BINS, w, w0, x, b, leader, cnt);
      }
    }
  }
  __syncthreads();
  for (uint32_t i = tid; i < P * BINS; i += HIST_THREADS) {
    const uint32_t v = hist[i];
    if (v) add_agent(&bins[i], v);
  }
  // Completion count. The barrier waits for the block's additions; the count
  // is a device-scope release/acquire, so the block that brings it to
  // gridDim.x sees every block's additions.
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
                     gridDim.x - 1u
                 ? 1u
                 : 0u;
  __syncthreads();
  if (!s_last) return;
  write_plan<N>(bins, static_cast<uint32_t>(n), plan, plan_flags);
}

// ---------------------------------------------------------------------------
// onesweep over rows
// ---------------------------------------------------------------------------
template <int N, class Val>
struct RowBuffers {
  const Row<N> *in;
  Row<N> *out, *scratch;
  const Val *vin;
  Val *vout, *vscratch;
};

template <int N, class Val, int ITEMS, radix::Rank RANK>
__global__ void __launch_bounds__(RADIX_THREADS, RCCL_RADIX_WAVES_PER_SIMD)
row_onesweep_kernel(RowBuffers<N, Val> b, size_t n, uint32_t num_tiles,
                    const uint32_t *__restrict__ pass_bins, const PassPlan *__restrict__ plan,
                    LookbackBuf<uint32_t> lb0, LookbackBuf<uint32_t> lb1, uint32_t nx,
                    uint32_t bit) {
  const PassPlan pl = *plan;
  if (!pl.active) return;
  const Row<N> *kin = pl.src == 0 ? b.in : (pl.src == 1 ? b.out : b.scratch);
  Row<N> *kout = pl.dst == 1 ? b.out : b.scratch;
  const Val *vin = pl.src == 0 ? b.vin : (pl.src == 1 ? b.vout : b.vscratch);
  Val *vout = pl.dst == 1 ? b.vout : b.vscratch;
  radix::onesweep_tile<Row<N>, Val, RowDigits<N>, ITEMS, uint32_t, RADIX_THREADS, RANK>(
      kin, kout, vin, vout, n, num_tiles, pass_bins, nullptr, pl.lb ? lb1 : lb0,
      pl.lb ? lb0 : lb1, nx, bit, 0xFFu, pl.conv);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct RadixLayout {
  size_t tiles = 0, groups = 0;
  size_t bins = 0, plan = 0;
  size_t lb[2] = {0, 0};
  size_t lb_ginc = 0, lb_gagg = 0, lb_ticket = 0, lb_bytes = 0;
  size_t scratch_rows = 0, scratch_vals = 0;
  size_t total = 0;
};

template <int N, class Val>
RadixLayout radix_layout(size_t n) {
  constexpr size_t VB = std::is_same<Val, radix::NoValue>::value ? 0 : sizeof(Val);
  constexpr size_t TILE = size_t(RADIX_THREADS) * radix_items<N, Val>();
  constexpr size_t P = 4 * N;
  RadixLayout l;
  l.tiles = (n + TILE - 1) / TILE;
  l.groups = (l.tiles + radix::GROUP - 1) / radix::GROUP;
  size_t off = 0;
  l.bins = off;
  off += align_up((P * BINS + 1) * sizeof(uint32_t), 256);  // bins, completion count
  l.plan = off;
  off += align_up(P * sizeof(PassPlan), 256);
  l.lb_ginc = align_up(l.tiles * BINS * sizeof(uint32_t), 256);
  l.lb_gagg = l.lb_ginc + align_up(l.groups * BINS * sizeof(uint32_t), 256);
  l.lb_ticket = l.lb_gagg + align_up(l.groups * BINS * sizeof(uint32_t), 256);
  l.lb_bytes = l.lb_ticket + align_up(XCDS * sizeof(uint32_t), 256);
  l.lb[0] = off;
  off += l.lb_bytes;
  l.lb[1] = off;
  off += l.lb_bytes;
  l.scratch_rows = off;
  off += align_up(n * sizeof(Row<N>), 256);
  l.scratch_vals = off;
  off += align_up(n * VB, 256);
  l.total = off;
  return l;
}

struct RecordArgs {
  const void *in, *in_v;
  void *out, *out_v;
  size_t n;
  void *ws;
  size_t ws_bytes;
  hipStream_t stream;
};

// The 4N onesweep launches of a row sort, in one ranking mode.
template <int N, class Val, radix::Rank RANK>
rccl_hip_status launch_row_onesweeps(const RecordArgs &a, const RadixLayout &l,
                                     const RowBuffers<N, Val> &b, const uint32_t *bins,
                                     const PassPlan *plan, const LookbackBuf<uint32_t> (&lb)[2],
                                     uint32_t nx) {
  constexpr int ITEMS = radix_items<N, Val>();
  constexpr uint32_t P = 4 * N;
  size_t resident = 0;
  RCCL_HIP_TRY(resident_blocks(
      reinterpret_cast<const void *>(&row_onesweep_kernel<N, Val, ITEMS, RANK>), RADIX_THREADS,
      &resident));
  // The XCD order needs two rows of runs resident at once; with fewer, blocks
  // claim ticketed tiles instead.
  if (nx == XCDS && resident < 2 * size_t(XCDS) * radix::XCD_RUN) nx = 1;
  const uint32_t grid = static_cast<uint32_t>(radix::onesweep_grid(l.tiles, nx));
  for (uint32_t p = 0; p < P; ++p) {
    const uint32_t word = uint32_t(N) - 1u - p / 4u;
    const uint32_t bit = 32u * word + 8u * (p % 4u);
    KernelTimer t("record_onesweep", a.stream, a.n);
    row_onesweep_kernel<N, Val, ITEMS, RANK><<<dim3(grid), RADIX_THREADS, 0, a.stream>>>(
        b, a.n, static_cast<uint32_t>(l.tiles), bins + size_t(p) * BINS, plan + p, lb[0], lb[1],
        nx, bit);
    RCCL_HIP_TRY(check_launch("record sort onesweep"));
  }
  return ok();
}

template <int N, class Val>
rccl_hip_status run_radix(const RecordArgs &a) {
  constexpr uint32_t P = 4 * N;
  const RadixLayout l = radix_layout<N, Val>(a.n);
  if (!a.ws || a.ws_bytes < l.total)
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "record sort workspace", l.total,
                     a.ws_bytes);
  unsigned char *ws = static_cast<unsigned char *>(a.ws);
  uint32_t *bins = reinterpret_cast<uint32_t *>(ws + l.bins);
  PassPlan *plan = reinterpret_cast<PassPlan *>(ws + l.plan);
  LookbackBuf<uint32_t> lb[2];
  for (int i = 0; i < 2; ++i) {
    unsigned char *base = ws + l.lb[i];
    lb[i].tile = reinterpret_cast<uint32_t *>(base);
    lb[i].ginc = reinterpret_cast<uint32_t *>(base + l.lb_ginc);
    lb[i].gagg = reinterpret_cast<uint32_t *>(base + l.lb_gagg);
    lb[i].ticket = reinterpret_cast<uint32_t *>(base + l.lb_ticket);
  }
  RowBuffers<N, Val> b;
  b.in = static_cast<const Row<N> *>(a.in);
  b.out = static_cast<Row<N> *>(a.out);
  b.scratch = reinterpret_cast<Row<N> *>(ws + l.scratch_rows);
  b.vin = static_cast<const Val *>(a.in_v);
  b.vout = static_cast<Val *>(a.out_v);
  b.vscratch = reinterpret_cast<Val *>(ws + l.scratch_vals);

  radix::DeviceCaps caps;
  RCCL_HIP_TRY(radix::device_caps(&caps, a.stream));
  const size_t cus = caps.cus;

  {
    KernelTimer t("record_init", a.stream, 0);
    record_init_kernel<<<1, 256, 0, a.stream>>>(bins, P * BINS + 1);
  }
  RCCL_HIP_TRY(check_launch("record sort init"));
  {
    KernelTimer t("record_histogram", a.stream, a.n);
    const size_t chunk = size_t(HIST_THREADS) * HIST_ITEMS;
    const size_t blocks =
        std::max<size_t>(1, std::min<size_t>((a.n + chunk - 1) / chunk, size_t(cus)));
    // Rows or payloads sorted in place: the first active pass must not write
    // the buffer it reads. Rows or payloads out of place: their output must
    // be written even when every row is equal.
    const bool has_v = a.in_v != nullptr;
    const uint32_t flags =
        (a.in == a.out || (has_v && a.in_v == a.out_v) ? radix::PLAN_IN_PLACE : 0u) |
        (a.in != a.out || (has_v && a.in_v != a.out_v) ? radix::PLAN_COPIES : 0u);
    row_histogram_kernel<N><<<dim3(static_cast<uint32_t>(blocks)), HIST_THREADS, 0, a.stream>>>(
        b.in, a.n, bins, bins + P * BINS, plan, flags, lb[0].tile,
        l.lb_bytes / sizeof(uint32_t));
  }
  RCCL_HIP_TRY(check_launch("record sort histogram"));
  return caps.rank == radix::Rank::LaneAtomic
             ? launch_row_onesweeps<N, Val, radix::Rank::LaneAtomic>(a, l, b, bins, plan, lb,
                                                                     caps.nx)
             : launch_row_onesweeps<N, Val, radix::Rank::MatchAny>(a, l, b, bins, plan, lb,
                                                                   caps.nx);
}

} // namespace record_sort
} // namespace rccl_hip
