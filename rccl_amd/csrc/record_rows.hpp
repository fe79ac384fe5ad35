// Padding-free [u32; N] relation rows (SRDatalog/HISA Row<N>,
// rccl-thrust/src/record_sort.rs:10-15) and their ascending unsigned
// lexicographic order (record_sort.rs:88-115).
#pragma once

#include "common.hpp"

namespace rccl_hip {
namespace record_sort {

constexpr uint32_t MIN_ARITY = 2, MAX_ARITY = 6;

template <int N>
struct Row {
  uint32_t w[N];
};

template <int N>
struct RowLess {
  __device__ __forceinline__ bool operator()(const Row<N> &a, const Row<N> &b) const {
#pragma unroll
    for (int c = 0; c < N; ++c) {
      if (a.w[c] != b.w[c]) return a.w[c] < b.w[c];
    }
    return false;
  }
};

// Per-word choice between two rows (the merge kernels call it through
// argument-dependent lookup), so the choice stays in registers.
template <int N>
__device__ __forceinline__ Row<N> pick(bool c, const Row<N> &x, const Row<N> &y) {
  Row<N> r;
#pragma unroll
  for (int i = 0; i < N; ++i) r.w[i] = c ? x.w[i] : y.w[i];
  return r;
}

// Per-word opaque copy (the onesweep tile calls it through argument-dependent
// lookup).
template <int N>
__device__ __forceinline__ void launder(Row<N> &r) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(r.w[i]));
}

// Digits of a row for LSD radix sorting. `bit` = 32 * word + 8 * byte, with
// word 0 the most significant column. The word index is uniform across a
// launch; the word is picked with masks rather than selects, which the
// compiler would turn into an indexed load and so keep rows in memory.
template <int N>
struct RowDigits {
  __device__ static __forceinline__ uint32_t word(const Row<N> &r, uint32_t w) {
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) x |= r.w[i] & (0u - static_cast<uint32_t>(w == uint32_t(i)));
    return x;
  }
  __device__ static __forceinline__ uint32_t digit(const Row<N> &r, uint32_t bit, uint32_t mask) {
    return (word(r, bit >> 5) >> (bit & 31u)) & mask;
  }
  // Rows are their own order-preserving image (the onesweep's conversions are
  // no-ops).
  __device__ static __forceinline__ Row<N> image(const Row<N> &r) { return r; }
  __device__ static __forceinline__ Row<N> raw(const Row<N> &r) { return r; }
  __device__ static __forceinline__ uint32_t image_digit(const Row<N> &r, uint32_t bit,
                                                         uint32_t mask) {
    return digit(r, bit, mask);
  }
};

} // namespace record_sort
} // namespace rccl_hip
