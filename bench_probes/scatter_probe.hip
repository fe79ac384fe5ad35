// Memory-pattern probe for bench.py's hbm_reference leg: the radix onesweep's
// loads and stores without its ranking, counting or look-back, so the rate a
// pass could reach with its write pattern is measured on the same GPU in the
// same run. Not part of librccl_hip; no sort calls it.
//
// Shape, as the u32 keys-only onesweep (rccl_amd/csrc/radix_kernels.hpp):
// 512 threads x 34 keys per tile, tiles handed to the XCDs in runs of 8
// (the same block -> tile map), keys loaded wave-contiguous and lane-striped
// with non-temporal loads, staged in LDS, read back thread-striped and
// stored; the LDS array has the onesweep's footprint, so two blocks share a
// CU as in the sort.
//   mode 0  copy through LDS: staged key i of tile t goes to t * TILE + i.
//   mode 1  the write pattern of a uniform radix pass: every tile holds 68
//           keys of each of the 256 digits, staged in digit order; run r of
//           tile t goes to r * (tiles * 68) + t * 68, so each digit's bucket
//           is filled tile after tile, as a pass over uniform digits does.
//   mode 2  mode 1's output, stored in 64-key-aligned windows: wave w takes
//           runs 32w to 32w + 31, and for each run one store per aligned
//           window of 64 output positions that the run touches (two or three),
//           each lane writing the window position it owns if the run covers
//           it. Where a run covers a whole window, its two 128-byte lines
//           leave in one store; it takes about twice the store instructions.
//   mode 3  mode 1 with each store split into two of 32 lanes (staged keys
//           0-31 and 32-63 of the instruction's 64), each spanning at most
//           two cache lines of one or two runs.
//   mode 4  mode 1 with tile = block: consecutive tiles land on different
//           XCDs (round-robin placement), so the lines two neighbouring tiles
//           share at every run boundary meet in no common L2.
// The input and output hold tiles * TILE u32 words (whole tiles only).
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

constexpr uint32_t XCDS = 8;
constexpr uint32_t XCD_RUN = 8;
constexpr int THREADS = 512;
constexpr int ITEMS = 34;
constexpr int TILE = THREADS * ITEMS;
constexpr int WAVE_ITEMS = 64 * ITEMS;
constexpr int DIGITS = 256;
constexpr int RUN_KEYS = TILE / DIGITS;  // 68
static_assert(RUN_KEYS * DIGITS == TILE, "whole digit runs per tile");
constexpr int LDS_WORDS = 79360 / 4;     // the u32 onesweep's LDS bytes per block
static_assert(TILE <= LDS_WORDS, "the tile fits the staging array");

__device__ __forceinline__ uint32_t xcd_order_tile(uint32_t block) {
  const uint32_t x = block % XCDS, j = block / XCDS;
  return XCDS * XCD_RUN * (j / XCD_RUN) + XCD_RUN * x + j % XCD_RUN;
}

template <int MODE>
__global__ void __launch_bounds__(THREADS)
probe_kernel(const uint32_t *__restrict__ in, uint32_t *__restrict__ out, uint32_t tiles) {
  __shared__ uint32_t stage[LDS_WORDS];
  const uint32_t tile = MODE == 4 ? blockIdx.x : xcd_order_tile(blockIdx.x);
  if (tile >= tiles) return;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const size_t base = size_t(tile) * TILE;
  const uint32_t *src = in + base + size_t(wave) * WAVE_ITEMS;
  uint32_t key[ITEMS];
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) key[j] = __builtin_nontemporal_load(&src[j * 64 + lane]);
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) stage[wave * WAVE_ITEMS + j * 64 + lane] = key[j];
  __syncthreads();
  const size_t bucket = size_t(tiles) * RUN_KEYS;
  if constexpr (MODE == 2) {
    constexpr int RUNS_PER_WAVE = DIGITS / (THREADS / 64);
    for (int q = 0; q < RUNS_PER_WAVE; ++q) {
      const uint32_t r = wave * RUNS_PER_WAVE + q;  // wave-uniform
      const size_t g0 = size_t(r) * bucket + size_t(tile) * RUN_KEYS;
      const size_t g1 = g0 + RUN_KEYS;
      for (size_t w = g0 & ~size_t(63); w < g1; w += 64) {
        const size_t p = w + lane;
        if (p >= g0 && p < g1) out[p] = stage[r * RUN_KEYS + static_cast<uint32_t>(p - g0)];
      }
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < ITEMS; ++k) {
    const uint32_t i = uint32_t(k) * THREADS + tid;
    const uint32_t v = stage[i];
    size_t dst;
    if constexpr (MODE == 0)
      dst = base + i;
    else
      dst = size_t(i / RUN_KEYS) * bucket + size_t(tile) * RUN_KEYS + i % RUN_KEYS;
    if constexpr (MODE == 3) {
      // Two stores of 32 lanes each (the compiler may not merge them).
      if (lane < 32) out[dst] = v;
      asm volatile("" ::: "memory");
      if (lane >= 32) out[dst] = v;
    } else {
      out[dst] = v;
    }
  }
}

}  // namespace

extern "C" {

// Keys per tile: callers size the buffers to whole tiles.
__attribute__((visibility("default"))) size_t scatter_probe_tile_items() { return TILE; }

// One launch of mode 0 to 4 over `tiles` whole tiles on `stream`. Returns
// 0, or the HIP error of the launch; 1 for an invalid mode or tile count.
__attribute__((visibility("default"))) int scatter_probe_launch(const void *in, void *out,
                                                                 size_t tiles, int mode,
                                                                 void *stream) {
  if (tiles == 0 || tiles > (size_t(1) << 31) / TILE || mode < 0 || mode > 4) return 1;
  const size_t row = size_t(XCDS) * XCD_RUN;
  const dim3 grid(static_cast<uint32_t>((tiles + row - 1) / row * row));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t *src = static_cast<const uint32_t *>(in);
  uint32_t *dst = static_cast<uint32_t *>(out);
  if (mode == 0)
    probe_kernel<0><<<grid, THREADS, 0, s>>>(src, dst, static_cast<uint32_t>(tiles));
  else if (mode == 1)
    probe_kernel<1><<<grid, THREADS, 0, s>>>(src, dst, static_cast<uint32_t>(tiles));
  else if (mode == 2)
    probe_kernel<2><<<grid, THREADS, 0, s>>>(src, dst, static_cast<uint32_t>(tiles));
  else if (mode == 3)
    probe_kernel<3><<<grid, THREADS, 0, s>>>(src, dst, static_cast<uint32_t>(tiles));
  else
    probe_kernel<4><<<grid, THREADS, 0, s>>>(src, dst, static_cast<uint32_t>(tiles));
  return static_cast<int>(hipGetLastError());
}

}  // extern "C"
