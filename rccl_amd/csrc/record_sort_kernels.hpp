// Stable lexicographic sort of padding-free [u32; N] rows (SRDatalog/HISA
// relation rows), optionally carrying a provenance payload per row.
//
// Reference behaviour: rccl-thrust/src/record_sort.rs:88-366. The reference
// lowers every row sort onto DeviceMergeSort with an unrolled lexicographic
// comparator over the row's columns (:88-115). Here small inputs do the same
// (rows are the keys of the merge-path merge sort, merge_sort_kernels.hpp,
// with RowLess as comparator) and larger ones take a multi-word LSD radix
// sort (record_radix_kernels.hpp); both are stable, so the output is the
// reference's. Arity 2..6 (:117-126); payloads are u64, f64 or
// BooleanProvenance (one byte), moved as opaque 8- or 1-byte values.
#pragma once

#include "merge_sort_kernels.hpp"
#include "record_radix_kernels.hpp"
#include "record_rows.hpp"

namespace rccl_hip {
namespace record_sort {

// Payload type of a width: none, BooleanProvenance (1 byte) or u64/f64 (8).
template <size_t VB> struct PayloadOf;
template <> struct PayloadOf<0> { using merge = ordering::NoValue; using radix = radix::NoValue; };
template <> struct PayloadOf<1> { using merge = uint8_t; using radix = uint8_t; };
template <> struct PayloadOf<8> { using merge = uint64_t; using radix = uint64_t; };

// Inputs of RADIX_MIN_ROWS..RADIX_MAX_ROWS rows take the LSD radix sort
// (record_radix_kernels.hpp); others the merge sort, whose few launches win
// on small inputs. Both are stable sorts in the same order, so the choice
// never changes a result.
inline bool use_radix(size_t n) { return n >= RADIX_MIN_ROWS && n <= RADIX_MAX_ROWS; }

template <int N, size_t VB>
size_t bytes_for(size_t n) {
  using P = PayloadOf<VB>;
  if (use_radix(n)) return radix_layout<N, typename P::radix>(n).total;
  return merge_sort::layout<Row<N>, typename P::merge>(n).total;
}

template <int N, size_t VB>
rccl_hip_status run_for(const RecordArgs &a) {
  using P = PayloadOf<VB>;
  if (use_radix(a.n)) return run_radix<N, typename P::radix>(a);
  const merge_sort::SortArgs s{a.in, a.in_v, a.out, a.out_v, a.n, a.ws, a.ws_bytes, a.stream};
  return merge_sort::run_sort<Row<N>, typename P::merge, RowLess<N>>(s);
}

template <int N>
size_t bytes(size_t n, size_t payload_bytes) {
  switch (payload_bytes) {
  case 0: return bytes_for<N, 0>(n);
  case 1: return bytes_for<N, 1>(n);
  default: return bytes_for<N, 8>(n);
  }
}

template <int N>
rccl_hip_status run(const RecordArgs &a, size_t payload_bytes) {
  switch (payload_bytes) {
  case 0: return run_for<N, 0>(a);
  case 1: return run_for<N, 1>(a);
  case 8: return run_for<N, 8>(a);
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "record-sort payload bytes");
}

// One arity per translation unit (record_sort_<N>.hip).
#define RCCL_RECORD_SORT_DECLARE_ARITY(N)                                                  \
  size_t bytes_##N(size_t n, size_t payload_bytes);                                      \
  rccl_hip_status run_##N(const RecordArgs &a, size_t payload_bytes);
RCCL_RECORD_SORT_DECLARE_ARITY(2)
RCCL_RECORD_SORT_DECLARE_ARITY(3)
RCCL_RECORD_SORT_DECLARE_ARITY(4)
RCCL_RECORD_SORT_DECLARE_ARITY(5)
RCCL_RECORD_SORT_DECLARE_ARITY(6)
#undef RCCL_RECORD_SORT_DECLARE_ARITY

#define RCCL_RECORD_SORT_DEFINE_ARITY(N)                                                   \
  size_t bytes_##N(size_t n, size_t payload_bytes) { return bytes<N>(n, payload_bytes); } \
  rccl_hip_status run_##N(const RecordArgs &a, size_t payload_bytes) {                   \
    return run<N>(a, payload_bytes);                                                      \
  }

} // namespace record_sort
} // namespace rccl_hip
