// Vectorized lower_bound / upper_bound C ABI: validation and dispatch of the
// runtime key (kind, arity) and order onto search_kernels.hpp.
#include "search_kernels.hpp"

using namespace rccl_hip;

namespace {

template <class K>
rccl_hip_status run_order(const search::SearchArgs &a, bool desc) {
  return desc ? search::run<K, ordering::Less<K, true>>(a)
              : search::run<K, ordering::Less<K, false>>(a);
}

rccl_hip_status dispatch(rccl_hip_key_kind key, uint32_t arity, bool desc,
                         const search::SearchArgs &a) {
  if (arity > 1) {
    switch (arity) {
    case 2: return search::run<record_sort::Row<2>, record_sort::RowLess<2>>(a);
    case 3: return search::run<record_sort::Row<3>, record_sort::RowLess<3>>(a);
    case 4: return search::run<record_sort::Row<4>, record_sort::RowLess<4>>(a);
    case 5: return search::run<record_sort::Row<5>, record_sort::RowLess<5>>(a);
    default: return search::run<record_sort::Row<6>, record_sort::RowLess<6>>(a);
    }
  }
  switch (key) {
  case RCCL_HIP_KEY_U32: return run_order<uint32_t>(a, desc);
  case RCCL_HIP_KEY_I32: return run_order<int32_t>(a, desc);
  case RCCL_HIP_KEY_F32: return run_order<float>(a, desc);
  case RCCL_HIP_KEY_U64: return run_order<uint64_t>(a, desc);
  case RCCL_HIP_KEY_I64: return run_order<int64_t>(a, desc);
  case RCCL_HIP_KEY_F64: return run_order<double>(a, desc);
  case RCCL_HIP_KEY_U8: return run_order<uint8_t>(a, desc);
  case RCCL_HIP_KEY_I8: return run_order<int8_t>(a, desc);
  case RCCL_HIP_KEY_U16: return run_order<uint16_t>(a, desc);
  case RCCL_HIP_KEY_I16: return run_order<int16_t>(a, desc);
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "search key kind");
}

// Workspace bytes of the chunk index for a haystack of n keys (or rows).
size_t index_bytes(rccl_hip_key_kind key, uint32_t arity, size_t n) {
  if (arity > 1) {
    switch (arity) {
    case 2: return search::workspace_bytes<record_sort::Row<2>>(n);
    case 3: return search::workspace_bytes<record_sort::Row<3>>(n);
    case 4: return search::workspace_bytes<record_sort::Row<4>>(n);
    case 5: return search::workspace_bytes<record_sort::Row<5>>(n);
    default: return search::workspace_bytes<record_sort::Row<6>>(n);
    }
  }
  switch (key) {
  case RCCL_HIP_KEY_U32: return search::workspace_bytes<uint32_t>(n);
  case RCCL_HIP_KEY_I32: return search::workspace_bytes<int32_t>(n);
  case RCCL_HIP_KEY_F32: return search::workspace_bytes<float>(n);
  case RCCL_HIP_KEY_U64: return search::workspace_bytes<uint64_t>(n);
  case RCCL_HIP_KEY_I64: return search::workspace_bytes<int64_t>(n);
  case RCCL_HIP_KEY_F64: return search::workspace_bytes<double>(n);
  case RCCL_HIP_KEY_U8: return search::workspace_bytes<uint8_t>(n);
  case RCCL_HIP_KEY_I8: return search::workspace_bytes<int8_t>(n);
  case RCCL_HIP_KEY_U16: return search::workspace_bytes<uint16_t>(n);
  case RCCL_HIP_KEY_I16: return search::workspace_bytes<int16_t>(n);
  }
  return 0;
}

rccl_hip_status check_key(rccl_hip_key_kind key, uint32_t arity) {
  if (arity == 1) {
    if (key_bytes(key) == 0) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "search key kind");
  } else if (key != RCCL_HIP_KEY_U32 || arity < 2 || arity > 6) {
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "search key kind or arity");
  }
  return ok();
}

} // namespace

extern "C" {

rccl_hip_status rccl_hip_bound_search_workspace_bytes(rccl_hip_key_kind key, uint32_t arity,
                                                      size_t n, size_t *bytes) {
  if (!bytes) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "bytes");
  RCCL_HIP_TRY(check_key(key, arity));
  *bytes = index_bytes(key, arity, n);
  return ok();
}


rccl_hip_status rccl_hip_bound_search(rccl_hip_key_kind key, uint32_t arity, rccl_hip_order order,
                                      int upper, const void *haystack, size_t n,
                                      const void *needles, size_t m, uint64_t *out_indices,
                                      void *workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
  RCCL_HIP_TRY(check_key(key, arity));
  if (order != RCCL_HIP_ORDER_ASCENDING && order != RCCL_HIP_ORDER_DESCENDING)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "order");
  if (arity > 1 && order != RCCL_HIP_ORDER_ASCENDING)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "rows are searched in ascending order");
  if (m && (!needles || !out_indices))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "search needles or output");
  if (m && n && !haystack) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "search haystack");
  {
    const size_t item = arity > 1 ? 4u * size_t(arity) : key_bytes(key);
    const ByteRange outs[] = {{out_indices, sat_mul(m, sizeof(uint64_t))}};
    const ByteRange ins[] = {{haystack, sat_mul(n, item)}, {needles, sat_mul(m, item)}};
    if (outputs_overlap_inputs(outs, ins))
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "search output overlaps an input");
  }
  const search::SearchArgs a{haystack, needles, n,         m, out_indices, upper != 0,
                            workspace, workspace_bytes, stream};
  return dispatch(key, arity, order == RCCL_HIP_ORDER_DESCENDING, a);
}

} // extern "C"
