// DeviceMerge and DeviceMergeSort C ABI: validation (before any launch) and
// dispatch of the runtime key kind onto the per-kind instantiations in
// merge_<kind>.hip / merge_sort_<kind>.hip.
#include "merge_sort_kernels.hpp"
#include "radix_kernels.hpp"

using namespace rccl_hip;

namespace {

bool valid_kind(rccl_hip_key_kind k) { return key_bytes(k) != 0; }
bool valid_order(rccl_hip_order o) {
  return o == RCCL_HIP_ORDER_ASCENDING || o == RCCL_HIP_ORDER_DESCENDING;
}

rccl_hip_status common_checks(rccl_hip_key_kind key, size_t value_bytes, rccl_hip_order order,
                              const char *what) {
  if (!valid_kind(key)) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, what);
  if (!valid_value_bytes(value_bytes))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "value bytes");
  if (!valid_order(order)) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "order");
  return ok();
}

size_t merge_bytes(rccl_hip_key_kind key, size_t na, size_t nb, size_t vb) {
  switch (key) {
  case RCCL_HIP_KEY_U8: return merge::bytes_u8(na, nb, vb);
  case RCCL_HIP_KEY_I8: return merge::bytes_i8(na, nb, vb);
  case RCCL_HIP_KEY_U16: return merge::bytes_u16(na, nb, vb);
  case RCCL_HIP_KEY_I16: return merge::bytes_i16(na, nb, vb);
  case RCCL_HIP_KEY_U32: return merge::bytes_u32(na, nb, vb);
  case RCCL_HIP_KEY_I32: return merge::bytes_i32(na, nb, vb);
  case RCCL_HIP_KEY_F32: return merge::bytes_f32(na, nb, vb);
  case RCCL_HIP_KEY_U64: return merge::bytes_u64(na, nb, vb);
  case RCCL_HIP_KEY_I64: return merge::bytes_i64(na, nb, vb);
  case RCCL_HIP_KEY_F64: return merge::bytes_f64(na, nb, vb);
  }
  return 0;
}

rccl_hip_status merge_run(rccl_hip_key_kind key, const merge::MergeArgs &m, size_t vb, bool desc) {
  switch (key) {
  case RCCL_HIP_KEY_U8: return merge::run_u8(m, vb, desc);
  case RCCL_HIP_KEY_I8: return merge::run_i8(m, vb, desc);
  case RCCL_HIP_KEY_U16: return merge::run_u16(m, vb, desc);
  case RCCL_HIP_KEY_I16: return merge::run_i16(m, vb, desc);
  case RCCL_HIP_KEY_U32: return merge::run_u32(m, vb, desc);
  case RCCL_HIP_KEY_I32: return merge::run_i32(m, vb, desc);
  case RCCL_HIP_KEY_F32: return merge::run_f32(m, vb, desc);
  case RCCL_HIP_KEY_U64: return merge::run_u64(m, vb, desc);
  case RCCL_HIP_KEY_I64: return merge::run_i64(m, vb, desc);
  case RCCL_HIP_KEY_F64: return merge::run_f64(m, vb, desc);
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge key kind");
}

// Merge sorts of at least this many items with 32- or 64-bit keys run as a
// stable LSD radix sort (radix::merge_sort_lowering): same permutation, 36
// B/key of HBM traffic for 4-byte keys instead of 8 B per merge level. That
// holds for float keys too: the radix order is IEEE order with -0.0 and +0.0
// one key, which is the merge sort's `<`. Only NaN differs, and with NaN `<`
// is no ordering at all (a partial_cmp comparator cannot take it), so such
// inputs have no defined order either way.
#ifndef RCCL_MERGE_SORT_RADIX_MIN_ITEMS
#define RCCL_MERGE_SORT_RADIX_MIN_ITEMS 65536
#endif

bool lowers_to_radix(rccl_hip_key_kind key, size_t n) {
  const bool wide = key == RCCL_HIP_KEY_U32 || key == RCCL_HIP_KEY_I32 ||
                    key == RCCL_HIP_KEY_F32 || key == RCCL_HIP_KEY_U64 ||
                    key == RCCL_HIP_KEY_I64 || key == RCCL_HIP_KEY_F64;
  return wide && n >= RCCL_MERGE_SORT_RADIX_MIN_ITEMS && n <= radix::MAX_ITEMS;
}

size_t merge_sort_bytes(rccl_hip_key_kind key, size_t n, size_t vb) {
  switch (key) {
  case RCCL_HIP_KEY_U8: return merge_sort::bytes_u8(n, vb);
  case RCCL_HIP_KEY_I8: return merge_sort::bytes_i8(n, vb);
  case RCCL_HIP_KEY_U16: return merge_sort::bytes_u16(n, vb);
  case RCCL_HIP_KEY_I16: return merge_sort::bytes_i16(n, vb);
  case RCCL_HIP_KEY_U32: return merge_sort::bytes_u32(n, vb);
  case RCCL_HIP_KEY_I32: return merge_sort::bytes_i32(n, vb);
  case RCCL_HIP_KEY_F32: return merge_sort::bytes_f32(n, vb);
  case RCCL_HIP_KEY_U64: return merge_sort::bytes_u64(n, vb);
  case RCCL_HIP_KEY_I64: return merge_sort::bytes_i64(n, vb);
  case RCCL_HIP_KEY_F64: return merge_sort::bytes_f64(n, vb);
  }
  return 0;
}

rccl_hip_status sort_run(rccl_hip_key_kind key, const merge_sort::SortArgs &s, size_t vb,
                         bool desc) {
  switch (key) {
  case RCCL_HIP_KEY_U8: return merge_sort::run_u8(s, vb, desc);
  case RCCL_HIP_KEY_I8: return merge_sort::run_i8(s, vb, desc);
  case RCCL_HIP_KEY_U16: return merge_sort::run_u16(s, vb, desc);
  case RCCL_HIP_KEY_I16: return merge_sort::run_i16(s, vb, desc);
  case RCCL_HIP_KEY_U32: return merge_sort::run_u32(s, vb, desc);
  case RCCL_HIP_KEY_I32: return merge_sort::run_i32(s, vb, desc);
  case RCCL_HIP_KEY_F32: return merge_sort::run_f32(s, vb, desc);
  case RCCL_HIP_KEY_U64: return merge_sort::run_u64(s, vb, desc);
  case RCCL_HIP_KEY_I64: return merge_sort::run_i64(s, vb, desc);
  case RCCL_HIP_KEY_F64: return merge_sort::run_f64(s, vb, desc);
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge sort key kind");
}

size_t sort_bytes(rccl_hip_key_kind key, size_t n, size_t vb) {
  const size_t merge = merge_sort_bytes(key, n, vb);
  if (!lowers_to_radix(key, n)) return merge;
  return std::max(merge, radix::merge_sort_lowering_bytes(key_bytes(key), vb, n));
}

} // namespace

extern "C" {

rccl_hip_status rccl_hip_merge_workspace_bytes(rccl_hip_key_kind key, size_t value_bytes,
                                               size_t na, size_t nb, size_t *bytes) {
  if (!bytes) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "bytes");
  RCCL_HIP_TRY(common_checks(key, value_bytes, RCCL_HIP_ORDER_ASCENDING, "merge key kind"));
  // rccl-cub/src/workspace.rs:201-206: the combined length must not overflow.
  if (na > SIZE_MAX - nb) return set_error(RCCL_HIP_ERROR_SIZE_OVERFLOW, "merge length");
  *bytes = merge_bytes(key, na, nb, value_bytes);
  return ok();
}

rccl_hip_status rccl_hip_merge(rccl_hip_key_kind key, size_t value_bytes, rccl_hip_order order,
                               const void *a_keys, const void *a_values, size_t na,
                               const void *b_keys, const void *b_values, size_t nb,
                               void *out_keys, void *out_values, void *workspace,
                               size_t workspace_bytes, hipStream_t stream) {
  RCCL_HIP_TRY(common_checks(key, value_bytes, order, "merge key kind"));
  if (na > SIZE_MAX - nb) return set_error(RCCL_HIP_ERROR_SIZE_OVERFLOW, "merge length");
  if (na + nb == 0) return ok();
  if ((na && !a_keys) || (nb && !b_keys) || !out_keys)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge keys");
  if (value_bytes && ((na && !a_values) || (nb && !b_values) || !out_values))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge values");
  {
    const size_t kb = key_bytes(key), n = na + nb, vb = value_bytes;
    const ByteRange outs[] = {{out_keys, sat_mul(n, kb)}, {out_values, sat_mul(n, vb)}};
    const ByteRange ins[] = {{a_keys, sat_mul(na, kb)}, {b_keys, sat_mul(nb, kb)},
                             {a_values, sat_mul(na, vb)}, {b_values, sat_mul(nb, vb)}};
    if (outputs_overlap_inputs(outs, ins) ||
        ranges_overlap(out_keys, sat_mul(n, kb), out_values, sat_mul(n, vb)))
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge output overlaps an input");
  }
  merge::MergeArgs m{a_keys, a_values, b_keys, b_values, na, nb, out_keys, out_values,
                     workspace, workspace_bytes, stream};
  return merge_run(key, m, value_bytes, order == RCCL_HIP_ORDER_DESCENDING);
}

rccl_hip_status rccl_hip_merge_sort_workspace_bytes(rccl_hip_key_kind key, size_t value_bytes,
                                                    size_t n, size_t *bytes) {
  if (!bytes) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "bytes");
  RCCL_HIP_TRY(common_checks(key, value_bytes, RCCL_HIP_ORDER_ASCENDING, "merge sort key kind"));
  *bytes = sort_bytes(key, n, value_bytes);
  return ok();
}

rccl_hip_status rccl_hip_merge_sort(rccl_hip_key_kind key, size_t value_bytes, rccl_hip_order order,
                                    const void *in_keys, const void *in_values, void *out_keys,
                                    void *out_values, size_t n, void *workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  RCCL_HIP_TRY(common_checks(key, value_bytes, order, "merge sort key kind"));
  if (n == 0) return ok();
  if (!in_keys || !out_keys) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge sort keys");
  if (value_bytes && (!in_values || !out_values))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge sort values");
  {
    // Each stream is sorted in place (input == output) or into an output
    // disjoint from both inputs and the other output; anything else would be
    // read and written by one pass.
    const size_t kb = sat_mul(key_bytes(key), n), vb = sat_mul(value_bytes, n);
    if (sort_streams_overlap(in_keys, out_keys, kb, value_bytes ? in_values : nullptr,
                             value_bytes ? out_values : nullptr, vb))
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge sort buffers overlap");
  }
  if (lowers_to_radix(key, n))
    return radix::merge_sort_lowering(key, value_bytes, order == RCCL_HIP_ORDER_DESCENDING,
                                      in_keys, in_values, out_keys, out_values, n, workspace,
                                      workspace_bytes, stream);
  merge_sort::SortArgs s{in_keys, in_values, out_keys, out_values, n,
                         workspace, workspace_bytes, stream};
  return sort_run(key, s, value_bytes, order == RCCL_HIP_ORDER_DESCENDING);
}

} // extern "C"
