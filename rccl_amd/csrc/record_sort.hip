// Record sort C ABI: validation (before any launch) and dispatch of the
// runtime arity onto record_sort_<N>.hip (rccl-thrust/src/record_sort.rs:117-366).
#include "record_sort_kernels.hpp"

using namespace rccl_hip;

namespace {

rccl_hip_status check_shape(uint32_t arity, size_t payload_bytes) {
  // rccl-thrust/src/record_sort.rs:117-126
  if (arity < record_sort::MIN_ARITY || arity > record_sort::MAX_ARITY)
    return set_error(RCCL_HIP_ERROR_UNSUPPORTED_TARGET,
                     "record sort supports audited workload arities 2 through 6; use radix "
                     "sort for scalar keys",
                     record_sort::MAX_ARITY, arity);
  if (payload_bytes != 0 && payload_bytes != 1 && payload_bytes != 8)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "record-sort payload bytes", 8,
                     payload_bytes);
  return ok();
}

} // namespace

extern "C" {

rccl_hip_status rccl_hip_record_sort_workspace_bytes(uint32_t arity, size_t payload_bytes,
                                                     size_t n, size_t *bytes) {
  if (!bytes) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "bytes");
  RCCL_HIP_TRY(check_shape(arity, payload_bytes));
  switch (arity) {
  case 2: *bytes = record_sort::bytes_2(n, payload_bytes); break;
  case 3: *bytes = record_sort::bytes_3(n, payload_bytes); break;
  case 4: *bytes = record_sort::bytes_4(n, payload_bytes); break;
  case 5: *bytes = record_sort::bytes_5(n, payload_bytes); break;
  default: *bytes = record_sort::bytes_6(n, payload_bytes); break;
  }
  return ok();
}

rccl_hip_status rccl_hip_record_sort(uint32_t arity, size_t payload_bytes, const void *in_rows,
                                     const void *in_payloads, void *out_rows,
                                     void *out_payloads, size_t n, void *workspace,
                                     size_t workspace_bytes, hipStream_t stream) {
  RCCL_HIP_TRY(check_shape(arity, payload_bytes));
  if (n == 0) return ok();
  if (!in_rows || !out_rows) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "record-sort rows");
  if (payload_bytes && (!in_payloads || !out_payloads))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "record-sort payload");
  {
    // Each stream in place (input == output) or into an output disjoint from
    // both inputs and the other output.
    const size_t rb = sat_mul(n, 4u * size_t(arity)), pb = sat_mul(n, payload_bytes);
    if (sort_streams_overlap(in_rows, out_rows, rb, payload_bytes ? in_payloads : nullptr,
                             payload_bytes ? out_payloads : nullptr, pb))
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "record-sort buffers overlap");
  }
  const record_sort::RecordArgs s{in_rows, in_payloads, out_rows, out_payloads, n,
                                  workspace, workspace_bytes, stream};
  switch (arity) {
  case 2: return record_sort::run_2(s, payload_bytes);
  case 3: return record_sort::run_3(s, payload_bytes);
  case 4: return record_sort::run_4(s, payload_bytes);
  case 5: return record_sort::run_5(s, payload_bytes);
  default: return record_sort::run_6(s, payload_bytes);
  }
}

} // extern "C"
