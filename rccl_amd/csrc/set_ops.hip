// Set operation C ABI: validation (before any launch) and dispatch of the
// runtime key kind onto the per-kind instantiations in set_<kind>.hip.
#include <cstring>

#include "set_ops_kernels.hpp"

using namespace rccl_hip;

namespace {

bool valid_op(rccl_hip_set_operation op) {
  return op == RCCL_HIP_SET_UNION || op == RCCL_HIP_SET_INTERSECTION ||
         op == RCCL_HIP_SET_DIFFERENCE || op == RCCL_HIP_SET_SYMMETRIC_DIFFERENCE;
}

rccl_hip_status checks(rccl_hip_set_operation op, rccl_hip_key_kind key, size_t value_bytes,
                       rccl_hip_order order, size_t na, size_t nb) {
  if (!valid_op(op)) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "set operation");
  if (key_bytes(key) == 0) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "set key kind");
  if (!valid_value_bytes(value_bytes))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "value bytes");
  if (order != RCCL_HIP_ORDER_ASCENDING && order != RCCL_HIP_ORDER_DESCENDING)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "order");
  // rccl-cub/src/set_operation.rs:309-312: the combined length must not overflow.
  if (na > SIZE_MAX - nb) return set_error(RCCL_HIP_ERROR_SIZE_OVERFLOW, "set length");
  return ok();
}

size_t set_bytes(rccl_hip_key_kind key, size_t na, size_t nb, size_t vb) {
  switch (key) {
  case RCCL_HIP_KEY_U8: return set_ops::bytes_u8(na, nb, vb);
  case RCCL_HIP_KEY_I8: return set_ops::bytes_i8(na, nb, vb);
  case RCCL_HIP_KEY_U16: return set_ops::bytes_u16(na, nb, vb);
  case RCCL_HIP_KEY_I16: return set_ops::bytes_i16(na, nb, vb);
  case RCCL_HIP_KEY_U32: return set_ops::bytes_u32(na, nb, vb);
  case RCCL_HIP_KEY_I32: return set_ops::bytes_i32(na, nb, vb);
  case RCCL_HIP_KEY_F32: return set_ops::bytes_f32(na, nb, vb);
  case RCCL_HIP_KEY_U64: return set_ops::bytes_u64(na, nb, vb);
  case RCCL_HIP_KEY_I64: return set_ops::bytes_i64(na, nb, vb);
  case RCCL_HIP_KEY_F64: return set_ops::bytes_f64(na, nb, vb);
  }
  return 0;
}

rccl_hip_status set_run(rccl_hip_key_kind key, const set_ops::SetArgs &s, size_t vb, bool desc) {
  switch (key) {
  case RCCL_HIP_KEY_U8: return set_ops::run_u8(s, vb, desc);
  case RCCL_HIP_KEY_I8: return set_ops::run_i8(s, vb, desc);
  case RCCL_HIP_KEY_U16: return set_ops::run_u16(s, vb, desc);
  case RCCL_HIP_KEY_I16: return set_ops::run_i16(s, vb, desc);
  case RCCL_HIP_KEY_U32: return set_ops::run_u32(s, vb, desc);
  case RCCL_HIP_KEY_I32: return set_ops::run_i32(s, vb, desc);
  case RCCL_HIP_KEY_F32: return set_ops::run_f32(s, vb, desc);
  case RCCL_HIP_KEY_U64: return set_ops::run_u64(s, vb, desc);
  case RCCL_HIP_KEY_I64: return set_ops::run_i64(s, vb, desc);
  case RCCL_HIP_KEY_F64: return set_ops::run_f64(s, vb, desc);
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "set key kind");
}

// Largest index an arithmetic range of `key` can address: the reference converts
// each index to the key type and traps when it does not fit
// (rccl-cub/src/ordering_backend/set.rs:72-80).
uint64_t max_arith_index(rccl_hip_key_kind key) {
  switch (key) {
  case RCCL_HIP_KEY_U8: return 0xFFu;
  case RCCL_HIP_KEY_I8: return 0x7Fu;
  case RCCL_HIP_KEY_U16: return 0xFFFFu;
  case RCCL_HIP_KEY_I16: return 0x7FFFu;
  case RCCL_HIP_KEY_U32: return 0xFFFFFFFFu;
  case RCCL_HIP_KEY_I32: return 0x7FFFFFFFu;
  case RCCL_HIP_KEY_U64: return ~0ull;
  case RCCL_HIP_KEY_I64: return 0x7FFFFFFFFFFFFFFFull;
  default: return 0;  // floating keys have no arithmetic ranges
  }
}

} // namespace

extern "C" {

rccl_hip_status rccl_hip_set_op_workspace_bytes(rccl_hip_set_operation op, rccl_hip_key_kind key,
                                                size_t value_bytes, size_t na, size_t nb,
                                                size_t *bytes) {
  if (!bytes) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "bytes");
  RCCL_HIP_TRY(checks(op, key, value_bytes, RCCL_HIP_ORDER_ASCENDING, na, nb));
  *bytes = set_bytes(key, na, nb, value_bytes);
  return ok();
}

rccl_hip_status rccl_hip_set_op(rccl_hip_set_operation op, rccl_hip_key_kind key,
                                size_t value_bytes, rccl_hip_order order, const void *a_keys,
                                const void *a_values, size_t na, const void *b_keys,
                                const void *b_values, size_t nb, void *out_keys,
                                void *out_values, size_t out_capacity, uint64_t *d_out_count,
                                void *workspace, size_t workspace_bytes, hipStream_t stream) {
  RCCL_HIP_TRY(checks(op, key, value_bytes, order, na, nb));
  if ((na && !a_keys) || (nb && !b_keys))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "set input keys");
  if (!out_keys && !d_out_count)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "set output count");
  // Counting reads keys only; value ranges are checked when they are written.
  const size_t vb = out_keys ? value_bytes : 0;
  const bool reads_b_values =
      op == RCCL_HIP_SET_UNION || op == RCCL_HIP_SET_SYMMETRIC_DIFFERENCE;
  if (vb && ((na && !a_values) || (reads_b_values && nb && !b_values) || !out_values))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "set values");
  if (out_keys) {
    const size_t kb = key_bytes(key), cap = out_capacity;
    const ByteRange outs[] = {{out_keys, sat_mul(cap, kb)}, {out_values, sat_mul(cap, vb)}};
    const ByteRange ins[] = {{a_keys, sat_mul(na, kb)}, {b_keys, sat_mul(nb, kb)},
                             {a_values, sat_mul(na, vb)},
                             {reads_b_values ? b_values : nullptr, sat_mul(nb, vb)}};
    if (outputs_overlap_inputs(outs, ins) ||
        ranges_overlap(out_keys, sat_mul(cap, kb), out_values, sat_mul(cap, vb)))
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "set output overlaps an input");
  }
  set_ops::SetArgs s{};
  s.op = static_cast<int>(op);
  s.a = a_keys;
  s.av = a_values;
  s.b = b_keys;
  s.bv = b_values;
  s.na = na;
  s.nb = nb;
  s.out = out_keys;
  s.outv = out_values;
  s.out_cap = out_keys ? out_capacity : 0;
  s.out_count = d_out_count;
  s.ws = workspace;
  s.ws_bytes = workspace_bytes;
  s.stream = stream;
  return set_run(key, s, vb, order == RCCL_HIP_ORDER_DESCENDING);
}

rccl_hip_status rccl_hip_set_op_arithmetic(rccl_hip_set_operation op, rccl_hip_key_kind key,
                                           rccl_hip_order order, const void *a_start,
                                           const void *a_step, size_t na, const void *b_start,
                                           const void *b_step, size_t nb, void *out_keys,
                                           size_t out_capacity, uint64_t *d_out_count,
                                           void *workspace, size_t workspace_bytes,
                                           hipStream_t stream) {
  RCCL_HIP_TRY(checks(op, key, 0, order, na, nb));
  if (key == RCCL_HIP_KEY_F32 || key == RCCL_HIP_KEY_F64)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "arithmetic range key kind");
  if ((na && (!a_start || !a_step)) || (nb && (!b_start || !b_step)))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "arithmetic range start or step");
  const uint64_t max_index = max_arith_index(key);
  if (na > 0 && uint64_t(na - 1) > max_index)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "first arithmetic range index",
                     max_index + 1, na);
  if (nb > 0 && uint64_t(nb - 1) > max_index)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "second arithmetic range index",
                     max_index + 1, nb);
  if (!out_keys && !d_out_count)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "set output count");
  set_ops::SetArgs s{};
  s.op = static_cast<int>(op);
  s.na = na;
  s.nb = nb;
  s.out = out_keys;
  s.out_cap = out_keys ? out_capacity : 0;
  s.out_count = d_out_count;
  s.ws = workspace;
  s.ws_bytes = workspace_bytes;
  s.stream = stream;
  s.arith = true;
  const size_t kb = key_bytes(key);
  if (na) {
    std::memcpy(&s.a_start, a_start, kb);
    std::memcpy(&s.a_step, a_step, kb);
  }
  if (nb) {
    std::memcpy(&s.b_start, b_start, kb);
    std::memcpy(&s.b_step, b_step, kb);
  }
  return set_run(key, s, 0, order == RCCL_HIP_ORDER_DESCENDING);
}

} // extern "C"
