// DeviceRadixSort host entry points: validation, workspace layout and the C
// ABI (rccl-cub/src/radix.rs:364-876 behaviour). Kernels and pass control are
// in radix_kernels.hpp; each key kind is instantiated in its own
// radix_<kind>.hip.
#include <atomic>
#include <mutex>
#include <utility>
#include <vector>

#include "radix_kernels.hpp"

// Control workspace (bins and the two look-back buffers) of
// rccl_hip_radix_sort_static: one copy per device, held until the process
// ends. Host code never uses this name as an address: the device address
// comes from hipGetSymbolAddress (static_workspace below).
static __device__ __align__(256) unsigned char scratch[RCCL_HIP_STATIC_RADIX_WORKSPACE_BYTES];

namespace rccl_hip {
namespace radix {

namespace {
std::mutex g_static_mu;
std::vector<std::pair<int, void *>> g_static_ptr;  // (device, device address of scratch)
} // namespace

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
rccl_hip_status static_workspace(void **out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_DRIVER, "current device", err);
  std::lock_guard<std::mutex> lock(g_static_mu);
  for (const auto &e : g_static_ptr) {
    if (e.first == dev) {
      *out = e.second;
      return ok();
    }
  }
  void *ptr = nullptr;
  err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (err != hipSuccess || !ptr)
    return set_hip_error(RCCL_HIP_ERROR_DRIVER, "static radix workspace address", err);
  g_static_ptr.emplace_back(dev, ptr);
  *out = ptr;
  return ok();
}


namespace {

// Lane-order self-check (see the onesweep notes): each wave repeatedly adds 1
// to per-wave LDS counters chosen by a hash of (block, round, lane)
// restricted to 1, 2, 16 or 256 counters, and checks that lanes hitting the
// same counter received consecutive values in lane order. CHECK_BLOCKS
// blocks of CHECK_THREADS run at once, several per CU on every CU, so the
// property is checked on the LDS of every CU under load; block b writes its
// number of violations to bad[b].
constexpr int CHECK_THREADS = 256;
constexpr int CHECK_BLOCKS = 1024;

// Outputs of the one-time device probes below (no allocation needed): the
// XCD of each placement-probe block, then each lane-order block's violations.
constexpr int XCC_PROBE_BLOCKS = 256;
__device__ uint32_t probe_out[XCC_PROBE_BLOCKS + CHECK_BLOCKS];

__global__ void __launch_bounds__(CHECK_THREADS) lane_order_check_kernel(uint32_t *bad) {
  const uint32_t salt = blockIdx.x * 0x27d4eb2fu;
  __shared__ uint32_t c[CHECK_THREADS / 64][BINS];
  __shared__ uint32_t total;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  for (uint32_t i = tid; i < (CHECK_THREADS / 64) * BINS; i += CHECK_THREADS) (&c[0][0])[i] = 0;
  if (tid == 0) total = 0;
  __syncthreads();
  uint32_t nbad = 0;
  for (uint32_t round = 0; round < 64; ++round) {
    uint32_t h = (round * 0x9e3779b9u) ^ (tid * 0x85ebca6bu) ^ salt;
    h ^= h >> 15;
    h *= 0x2c1b3c6du;
    h ^= h >> 12;
    const uint32_t mask = round % 4 == 0 ? 0u : round % 4 == 1 ? 1u : round % 4 == 2 ? 15u : 255u;
    const uint32_t d = h & mask;
    const uint32_t got =
        __hip_atomic_fetch_add(&c[wave][d], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    // Lanes below with the same counter, and the lowest such lane.
    uint32_t below = 0, first = lane;
    for (int l = 63; l >= 0; --l) {
      const uint32_t dl = static_cast<uint32_t>(__shfl(static_cast<int>(d), l, 64));
      if (dl == d && static_cast<uint32_t>(l) < lane) {
        ++below;
        first = static_cast<uint32_t>(l);
      }
    }
    const uint32_t base = got - below;
    nbad += static_cast<uint32_t>(__shfl(static_cast<int>(base), static_cast<int>(first), 64)) !=
            base;
  }
  if (nbad) atomicAdd(&total, nbad);
  __syncthreads();
  if (tid == 0) bad[blockIdx.x] = total;
}

// Where blocks land: block b records its XCD (HW_REG_XCC_ID, all 4 bits).
__global__ void __launch_bounds__(64) xcc_probe_kernel(uint32_t *out) {
  if (threadIdx.x == 0)
    out[blockIdx.x] = static_cast<uint32_t>(__builtin_amdgcn_s_getreg((3 << 11) | 20));
}

// Modes requested with rccl_hip_radix_configure (RCCL_HIP_RANKING_*,
// RCCL_HIP_TILE_ORDER_*).
std::atomic<int> g_ranking{0};
std::atomic<int> g_tile_order{0};

struct CapsEntry {
  int device;
  DeviceCaps caps;
};
std::mutex g_caps_mu;
std::vector<CapsEntry> g_caps;

rccl_hip_status probe_device(DeviceCaps *caps) {
  uint32_t *out = nullptr;
  hipError_t err = hipGetSymbolAddress(reinterpret_cast<void **>(&out), HIP_SYMBOL(probe_out));
  std::vector<uint32_t> host(XCC_PROBE_BLOCKS + CHECK_BLOCKS, 0u);
  if (err == hipSuccess) {
    xcc_probe_kernel<<<XCC_PROBE_BLOCKS, 64>>>(out);
    lane_order_check_kernel<<<CHECK_BLOCKS, CHECK_THREADS>>>(out + XCC_PROBE_BLOCKS);
    err = hipGetLastError();
  }
  if (err == hipSuccess)
    err = hipMemcpy(host.data(), out, host.size() * sizeof(uint32_t), hipMemcpyDeviceToHost);
  if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_DRIVER, "radix device probe", err);
  uint64_t violations = 0;
  for (int b = 0; b < CHECK_BLOCKS; ++b) violations += host[XCC_PROBE_BLOCKS + b];
  caps->lane_order = violations == 0;
  bool round_robin = true;
  for (int b = 0; b < XCC_PROBE_BLOCKS; ++b) round_robin &= host[b] == uint32_t(b) % XCDS;
  caps->nx = round_robin ? XCDS : 1u;
  caps->rank = caps->lane_order ? Rank::LaneAtomic : Rank::MatchAny;
  int dev = 0, cus = 0;
  err = hipGetDevice(&dev);
  if (err == hipSuccess)
    err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (err != hipSuccess || cus <= 0)
    return set_hip_error(RCCL_HIP_ERROR_DRIVER, "radix device CU count", err);
  caps->cus = static_cast<uint32_t>(cus);
  return ok();
}

} // namespace

namespace {
// The current device's probed caps, probing it on first use. The probe
// launches on the null stream and copies its result back synchronously, which
// a stream under graph capture does not allow: a first use from a capturing
// `stream` is refused (load the program on the device before capturing).
rccl_hip_status probed_caps(DeviceCaps *caps, hipStream_t stream, bool check_capture) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_DRIVER, "current device", err);
  std::lock_guard<std::mutex> lock(g_caps_mu);
  for (const CapsEntry &e : g_caps) {
    if (e.device == dev) {
      *caps = e.caps;
      return ok();
    }
  }
  if (check_capture) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    err = hipStreamIsCapturing(stream, &status);
    if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_DRIVER, "stream capture status", err);
    if (status != hipStreamCaptureStatusNone)
      return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT,
                       "device not loaded before stream capture (rccl_hip_program_load)");
  }
  RCCL_HIP_TRY(probe_device(caps));
  g_caps.push_back(CapsEntry{dev, *caps});
  return ok();
}
} // namespace

rccl_hip_status probe_current_device() {
  DeviceCaps caps;
  return probed_caps(&caps, nullptr, false);
}

rccl_hip_status device_caps(DeviceCaps *caps, hipStream_t stream) {
  DeviceCaps c;
  RCCL_HIP_TRY(probed_caps(&c, stream, true));
  switch (g_ranking.load(std::memory_order_relaxed)) {
  case RCCL_HIP_RANKING_LANE_ATOMIC:
    if (!c.lane_order)
      return set_error(RCCL_HIP_ERROR_UNSUPPORTED_TARGET, "lane-ordered LDS atomics");
    c.rank = Rank::LaneAtomic;
    break;
  case RCCL_HIP_RANKING_MATCH_ANY: c.rank = Rank::MatchAny; break;
  default: break;
  }
  if (g_tile_order.load(std::memory_order_relaxed) == RCCL_HIP_TILE_ORDER_TICKET) c.nx = 1;
  *caps = c;
  return ok();
}

} // namespace radix

rccl_hip_status tile_order(uint32_t *nx, hipStream_t stream) {
  radix::DeviceCaps c;
  RCCL_HIP_TRY(radix::device_caps(&c, stream));
  *nx = c.nx;
  return ok();
}

namespace radix {

namespace {

bool radix_kind(rccl_hip_key_kind k) { return k >= RCCL_HIP_KEY_U32 && k <= RCCL_HIP_KEY_F64; }

// Shared validation + launch for both ABI entry points; every check runs
// before the first launch.
rccl_hip_status sort_buffer(rccl_hip_key_kind key, size_t value_bytes, rccl_hip_order order,
                            SortArgs &a, size_t workspace_bytes) {
  if (!radix_kind(key)) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix key kind");
  if (!valid_value_bytes(value_bytes))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix value bytes");
  if (order != RCCL_HIP_ORDER_ASCENDING && order != RCCL_HIP_ORDER_DESCENDING)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix order");
  const uint32_t key_bits = static_cast<uint32_t>(key_bytes(key) * 8);
  // rccl-cub/src/radix.rs:370-376
  if (a.begin_bit > a.end_bit || a.end_bit > key_bits)
    return set_bit_range_error(a.begin_bit, a.end_bit, key_bits);
  if (a.n > MAX_ITEMS)
    return set_error(RCCL_HIP_ERROR_LENGTH_MISMATCH, "radix item count", MAX_ITEMS, a.n);
  const uint32_t passes = (a.end_bit - a.begin_bit + 7u) / 8u;
  // rccl-cub/src/radix.rs:467-469: an empty input or bit window is a no-op.
  if (a.n == 0 || passes == 0) return ok();
  if (!a.keys[0] || !a.keys[1]) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix keys");
  if (value_bytes && (!a.vals[0] || !a.vals[1]))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix values");
  if (!a.planned) {
    // Every pass reads one buffer of each pair and writes the other: the
    // four buffers must not share a byte (the reference's borrows make them
    // distinct; here an aliased scratch would race silently).
    const size_t kb = key_bytes(key) * a.n, vb = value_bytes * a.n;
    const void *p[4] = {a.keys[0], a.keys[1], a.vals[0], a.vals[1]};
    const size_t s[4] = {kb, kb, vb, vb};
    for (int i = 0; i < 4; ++i)
      for (int j = i + 1; j < 4; ++j)
        if (ranges_overlap(p[i], s[i], p[j], s[j]))
          return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix buffers overlap");
  }
  const Layout l = layout(key_bytes(key), value_bytes, a.n, a.planned);
  if (!a.ws || workspace_bytes < l.total)
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "radix workspace", l.total,
                     workspace_bytes);
  const bool desc = order == RCCL_HIP_ORDER_DESCENDING;
  switch (key) {
  case RCCL_HIP_KEY_U32: return run_u32(a, value_bytes, l, passes, desc);
  case RCCL_HIP_KEY_I32: return run_i32(a, value_bytes, l, passes, desc);
  case RCCL_HIP_KEY_F32: return run_f32(a, value_bytes, l, passes, desc);
  case RCCL_HIP_KEY_U64: return run_u64(a, value_bytes, l, passes, desc);
  case RCCL_HIP_KEY_I64: return run_i64(a, value_bytes, l, passes, desc);
  case RCCL_HIP_KEY_F64: return run_f64(a, value_bytes, l, passes, desc);
  default: break;
  }
  return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix key kind");
}

} // namespace

size_t merge_sort_lowering_bytes(size_t key_bytes_, size_t value_bytes, size_t n) {
  return align_up(n * key_bytes_, 256) + align_up(n * value_bytes, 256) +
         layout(key_bytes_, value_bytes, n, true).total + plan_bytes();
}

// A stable LSD radix sort under the natural order or its reverse yields
// exactly the stable merge sort's permutation: digit order is integer order,
// or for floats IEEE order with -0.0 and +0.0 one key (the merge sort's `<`;
// inputs with NaN, which `<` cannot order, have no defined order), and equal
// keys keep their input order. The output buffers
// are the first half of the double buffer and the workspace's scratch the
// second; a copy form reads its input in the histogram and its first active
// pass only. The sort is planned: passes whose byte is the same in every key
// (a digit holding all n keys) are skipped, and the plan routes the active
// ones so that the last writes the output.
rccl_hip_status merge_sort_lowering(rccl_hip_key_kind key, size_t value_bytes, bool descending,
                                    const void *in_keys, const void *in_vals, void *out_keys,
                                    void *out_vals, size_t n, void *workspace,
                                    size_t workspace_bytes, hipStream_t stream) {
  const size_t kb = key_bytes(key);
  if (key != RCCL_HIP_KEY_U32 && key != RCCL_HIP_KEY_I32 && key != RCCL_HIP_KEY_F32 &&
      key != RCCL_HIP_KEY_U64 && key != RCCL_HIP_KEY_I64 && key != RCCL_HIP_KEY_F64)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "merge sort radix key kind");
  const size_t scratch = align_up(n * kb, 256) + align_up(n * value_bytes, 256);
  if (!workspace || workspace_bytes < merge_sort_lowering_bytes(kb, value_bytes, n))
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "merge sort workspace",
                     merge_sort_lowering_bytes(kb, value_bytes, n), workspace_bytes);
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  SortArgs a{};
  a.keys[0] = out_keys;
  a.keys[1] = ws;
  a.vals[0] = value_bytes ? out_vals : nullptr;
  a.vals[1] = value_bytes ? ws + align_up(n * kb, 256) : nullptr;
  a.n = n;
  a.cur = 0;
  a.begin_bit = 0;
  a.end_bit = static_cast<uint32_t>(kb * 8);
  a.ws = ws + scratch;
  a.stream = stream;
  // Keys and values may each be in place or not: the histogram and the first
  // active pass read the input, and the plan keeps an in-place stream from
  // being read and written by one pass.
  a.src_keys = in_keys;
  a.src_vals = value_bytes ? in_vals : nullptr;
  a.planned = true;
  const bool vals_aliased = value_bytes && in_vals == out_vals;
  const bool vals_copied = value_bytes && in_vals != out_vals;
  a.plan_flags = (in_keys == out_keys || vals_aliased ? PLAN_IN_PLACE : 0u) |
                 (in_keys != out_keys || vals_copied ? PLAN_COPIES : 0u);
  return sort_buffer(key, value_bytes,
                     descending ? RCCL_HIP_ORDER_DESCENDING : RCCL_HIP_ORDER_ASCENDING, a,
                     workspace_bytes - scratch - plan_bytes());
}
} // namespace radix
} // namespace rccl_hip

using namespace rccl_hip;

extern "C" {

rccl_hip_status rccl_hip_radix_configure(int ranking, int tile_order) {
  if (ranking != RCCL_HIP_RANKING_AUTO && ranking != RCCL_HIP_RANKING_LANE_ATOMIC &&
      ranking != RCCL_HIP_RANKING_MATCH_ANY)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix ranking mode");
  if (tile_order != RCCL_HIP_TILE_ORDER_AUTO && tile_order != RCCL_HIP_TILE_ORDER_TICKET)
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix tile order");
  radix::g_ranking.store(ranking);
  radix::g_tile_order.store(tile_order);
  return ok();
}

rccl_hip_status rccl_hip_radix_sort_workspace_bytes(rccl_hip_key_kind key, size_t value_bytes,
                                                    size_t n, size_t *bytes) {
  if (!bytes) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "bytes");
  if (!radix::radix_kind(key)) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix key kind");
  if (!valid_value_bytes(value_bytes))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix value bytes");
  if (n > radix::MAX_ITEMS)
    return set_error(RCCL_HIP_ERROR_LENGTH_MISMATCH, "radix item count", radix::MAX_ITEMS, n);
  *bytes = radix::layout(key_bytes(key), value_bytes, n, false).total;
  return ok();
}

rccl_hip_status rccl_hip_radix_sort_buffer(rccl_hip_key_kind key, size_t value_bytes,
                                           rccl_hip_order order, void *keys_first,
                                           void *keys_second, void *values_first,
                                           void *values_second, size_t n,
                                           int *current_is_first, uint32_t begin_bit,
                                           uint32_t end_bit, void *workspace,
                                           size_t workspace_bytes, hipStream_t stream) {
  if (!current_is_first) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "current_is_first");
  radix::SortArgs a{};
  a.keys[0] = keys_first;
  a.keys[1] = keys_second;
  a.vals[0] = values_first;
  a.vals[1] = values_second;
  a.n = n;
  a.cur = *current_is_first ? 0 : 1;
  a.begin_bit = begin_bit;
  a.end_bit = end_bit;
  a.ws = static_cast<unsigned char *>(workspace);
  a.stream = stream;
  // Every onesweep pass flips the selector; the single-tile route (one
  // launch) flips it once, as the reference's does.
  a.single_to_other = true;
  RCCL_HIP_TRY(radix::sort_buffer(key, value_bytes, order, a, workspace_bytes));
  *current_is_first = a.cur == 0 ? 1 : 0;
  return ok();
}

rccl_hip_status rccl_hip_radix_sort_static(rccl_hip_key_kind key, size_t value_bytes,
                                           rccl_hip_order order, void *keys, void *values,
                                           void *scratch_keys, void *scratch_values, size_t n,
                                           hipStream_t stream) {
  if (!radix::radix_kind(key)) return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix key kind");
  if (!valid_value_bytes(value_bytes))
    return set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "radix value bytes");
  if (n > radix::MAX_ITEMS)
    return set_error(RCCL_HIP_ERROR_LENGTH_MISMATCH, "radix item count", radix::MAX_ITEMS, n);
  const size_t need = radix::layout(key_bytes(key), value_bytes, n, false).total;
  if (need > RCCL_HIP_STATIC_RADIX_WORKSPACE_BYTES)
    return set_error(RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL, "static radix workspace", need,
                     RCCL_HIP_STATIC_RADIX_WORKSPACE_BYTES);
  if (n == 0) return ok();
  void *ws = nullptr;
  RCCL_HIP_TRY(radix::static_workspace(&ws));
  return rccl_hip_radix_sort(key, value_bytes, order, keys, values, scratch_keys, scratch_values,
                             n, ws, RCCL_HIP_STATIC_RADIX_WORKSPACE_BYTES, stream);
}

rccl_hip_status rccl_hip_radix_sort(rccl_hip_key_kind key, size_t value_bytes,
                                    rccl_hip_order order, void *keys, void *values,
                                    void *scratch_keys, void *scratch_values, size_t n,
                                    void *workspace, size_t workspace_bytes, hipStream_t stream) {
  radix::SortArgs a{};
  a.keys[0] = keys;
  a.keys[1] = scratch_keys;
  a.vals[0] = values;
  a.vals[1] = scratch_values;
  a.n = n;
  a.cur = 0;
  a.begin_bit = 0;
  a.end_bit = static_cast<uint32_t>(key_bytes(key) * 8);
  a.ws = static_cast<unsigned char *>(workspace);
  a.stream = stream;
  RCCL_HIP_TRY(radix::sort_buffer(key, value_bytes, order, a, workspace_bytes));
  // rccl-cub/src/radix.rs:617-621: copy back when the result is in scratch.
  if (a.cur == 1) {
    hipError_t err = hipMemcpyAsync(keys, scratch_keys, n * key_bytes(key),
                                    hipMemcpyDeviceToDevice, stream);
    if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_MEMORY, "radix copy back", err);
    if (value_bytes) {
      err = hipMemcpyAsync(values, scratch_values, n * value_bytes, hipMemcpyDeviceToDevice,
                           stream);
      if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_MEMORY, "radix copy back", err);
    }
  }
  return ok();
}

} // extern "C"
