// Adjacent-run compaction C ABI: validation (before any launch) and dispatch
// of the runtime key (kind, arity) onto group_<key>.hip.
#include "group_kernels.hpp"

using namespace rccl_hip;

namespace rccl_hip {
namespace group {

namespace {
__global__ void zero_count_kernel(uint64_t *p) { *p = 0; }
} // namespace

rccl_hip_status write_zero_count(uint64_t *out_count, hipStream_t stream) {
  KernelTimer t("group_clear", stream, 1);
  zero_count_kernel<<<1, 1, 0, stream>>>(out_count);
  return check_launch("group count");
}

} // namespace group
} // namespace rccl_hip

namespace {

// Key slot: 0..9 the scalar kinds in rccl_hip_key_kind order, 10..14 rows of
// arity 2..6; -1 when the pair is not supported.
int key_slot(rccl_hip_key_kind key, uint32_t arity) {
  if (arity == 1) return key_bytes(key) ? static_cast<int>(key) : -1;
  if (key == RCCL_HIP_KEY_U32 && arity >= 2 && arity <= 6) return 8 + static_cast<int>(arity);
  return -1;
}

bool valid_op(rccl_hip_group_op op) {
  return op == RCCL_HIP_GROUP_UNIQUE || op == RCCL_HIP_GROUP_NATURAL_BAG_ADD ||
         op == RCCL_HIP_GROUP_BOOLEAN_OR || op == RCCL_HIP_GROUP_INDEPENDENT_PROBABILITY_OR;
}

bool valid_payload(rccl_hip_group_op op, size_t pb) {
  if (op == RCCL_HIP_GROUP_UNIQUE) return pb == 0 || pb == 1 || pb == 2 || pb == 4 || pb == 8;
  return pb == 0 || pb == 4 || pb == 8;
}

rccl_hip_status checks(rccl_hip_key_kind key, uint32_t arity, rccl_hip_group_op op, size_t pb,
                       int &slot) {
  slot = key_slot(key, arity);
  if (slot < 0) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "group key kind or arity");
  if (!valid_op(op)) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "group operator");
  if (!valid_payload(op, pb))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "group payload bytes");
  return ok();
}

size_t bytes_for(int slot, size_t n, rccl_hip_group_op op, size_t pb) {
  using namespace group;
  switch (slot) {
  case RCCL_HIP_KEY_U32: return bytes_u32(n, op, pb);
  case RCCL_HIP_KEY_I32: return bytes_i32(n, op, pb);
  case RCCL_HIP_KEY_F32: return bytes_f32(n, op, pb);
  case RCCL_HIP_KEY_U64: return bytes_u64(n, op, pb);
  case RCCL_HIP_KEY_I64: return bytes_i64(n, op, pb);
  case RCCL_HIP_KEY_F64: return bytes_f64(n, op, pb);
  case RCCL_HIP_KEY_U8: return bytes_u8(n, op, pb);
  case RCCL_HIP_KEY_I8: return bytes_i8(n, op, pb);
  case RCCL_HIP_KEY_U16: return bytes_u16(n, op, pb);
  case RCCL_HIP_KEY_I16: return bytes_i16(n, op, pb);
  case 10: return bytes_row2(n, op, pb);
  case 11: return bytes_row3(n, op, pb);
  case 12: return bytes_row4(n, op, pb);
  case 13: return bytes_row5(n, op, pb);
  default: return bytes_row6(n, op, pb);
  }
}

rccl_hip_status run_for(int slot, const group::GroupArgs &a, rccl_hip_group_op op, size_t pb) {
  using namespace group;
  switch (slot) {
  case RCCL_HIP_KEY_U32: return run_u32(a, op, pb);
  case RCCL_HIP_KEY_I32: return run_i32(a, op, pb);
  case RCCL_HIP_KEY_F32: return run_f32(a, op, pb);
  case RCCL_HIP_KEY_U64: return run_u64(a, op, pb);
  case RCCL_HIP_KEY_I64: return run_i64(a, op, pb);
  case RCCL_HIP_KEY_F64: return run_f64(a, op, pb);
  case RCCL_HIP_KEY_U8: return run_u8(a, op, pb);
  case RCCL_HIP_KEY_I8: return run_i8(a, op, pb);
  case RCCL_HIP_KEY_U16: return run_u16(a, op, pb);
  case RCCL_HIP_KEY_I16: return run_i16(a, op, pb);
  case 10: return run_row2(a, op, pb);
  case 11: return run_row3(a, op, pb);
  case 12: return run_row4(a, op, pb);
  case 13: return run_row5(a, op, pb);
  default: return run_row6(a, op, pb);
  }
}

// Bytes of one key ([u32; arity] rows from arity 2) and of one reduced value.
size_t key_item_bytes(rccl_hip_key_kind key, uint32_t arity) {
  return arity > 1 ? 4u * size_t(arity) : key_bytes(key);
}
size_t value_item_bytes(rccl_hip_group_op op) {
  return op == RCCL_HIP_GROUP_BOOLEAN_OR ? 1u : 8u;
}

} // namespace

extern "C" {

rccl_hip_status rccl_hip_group_workspace_bytes(rccl_hip_key_kind key, uint32_t arity,
                                               rccl_hip_group_op op, size_t payload_bytes,
                                               size_t n, size_t *bytes) {
  if (!bytes) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "bytes");
  int slot;
  RCCL_HIP_TRY(checks(key, arity, op, payload_bytes, slot));
  *bytes = bytes_for(slot, n, op, payload_bytes);
  return ok();
}

rccl_hip_status rccl_hip_unique_copy(rccl_hip_key_kind key, uint32_t arity, size_t payload_bytes,
                                     const void *in_keys, const void *in_payloads,
                                     void *out_keys, void *out_payloads, size_t n,
                                     uint64_t *d_count, void *workspace, size_t workspace_bytes,
                                     hipStream_t stream) {
  int slot;
  RCCL_HIP_TRY(checks(key, arity, RCCL_HIP_GROUP_UNIQUE, payload_bytes, slot));
  if (!d_count) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "selected-count output");
  if (n && (!in_keys || !out_keys))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "unique keys");
  if (n && payload_bytes && (!in_payloads || !out_payloads))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "unique payloads");
  {
    const size_t kb = sat_mul(n, key_item_bytes(key, arity)), pb = sat_mul(n, payload_bytes);
    const ByteRange outs[] = {{out_keys, kb}, {out_payloads, pb}};
    const ByteRange ins[] = {{in_keys, kb}, {in_payloads, pb}};
    if (outputs_overlap_inputs(outs, ins) || ranges_overlap(out_keys, kb, out_payloads, pb))
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "unique output overlaps an input");
  }
  const group::GroupArgs a{in_keys, in_payloads, nullptr, out_keys, out_payloads, nullptr,
                           n, d_count, workspace, workspace_bytes, stream};
  return run_for(slot, a, RCCL_HIP_GROUP_UNIQUE, payload_bytes);
}

rccl_hip_status rccl_hip_reduce_by_key(rccl_hip_key_kind key, uint32_t arity,
                                       rccl_hip_group_op op, size_t payload_bytes,
                                       const void *keys, const void *key_payloads,
                                       const void *values, void *out_keys,
                                       void *out_key_payloads, void *out_values, size_t n,
                                       uint64_t *d_group_count, void *workspace,
                                       size_t workspace_bytes, hipStream_t stream) {
  int slot;
  RCCL_HIP_TRY(checks(key, arity, op, payload_bytes, slot));
  if (op == RCCL_HIP_GROUP_UNIQUE)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "reduce-by-key operator");
  if (!d_group_count) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "group-count output");
  if (n && (!keys || !values || !out_keys || !out_values))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "reduce-by-key ranges");
  if (n && payload_bytes && (!key_payloads || !out_key_payloads))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "reduce-by-key key payloads");
  {
    const size_t kb = sat_mul(n, key_item_bytes(key, arity)), pb = sat_mul(n, payload_bytes),
                 vb = sat_mul(n, value_item_bytes(op));
    const ByteRange outs[] = {{out_keys, kb}, {out_key_payloads, pb}, {out_values, vb}};
    const ByteRange ins[] = {{keys, kb}, {key_payloads, pb}, {values, vb}};
    if (outputs_overlap_inputs(outs, ins) || ranges_overlap(out_keys, kb, out_key_payloads, pb) ||
        ranges_overlap(out_keys, kb, out_values, vb) ||
        ranges_overlap(out_key_payloads, pb, out_values, vb))
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "reduce-by-key output overlaps");
  }
  const group::GroupArgs a{keys,     key_payloads,     values,        out_keys,
                           out_key_payloads, out_values, n, d_group_count,
                           workspace, workspace_bytes, stream};
  return run_for(slot, a, op, payload_bytes);
}

} // extern "C"
