// Error state, status strings and target check of the rccl_hip C ABI.
#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace rccl_hip {
namespace radix {
struct DeviceCaps;
rccl_hip_status static_workspace(void **out);
rccl_hip_status probe_current_device();
} // namespace radix
} // namespace rccl_hip

namespace rccl_hip {

namespace {
struct TimingRecord {
  const char *name;
  hipEvent_t start;
  hipEvent_t stop;
  uint64_t items;
};
std::atomic<bool> g_timing_on{false};
std::mutex g_timing_mu;
std::vector<TimingRecord> g_records;
std::vector<std::pair<hipEvent_t, hipEvent_t>> g_event_pool;
} // namespace

KernelTimer::KernelTimer(const char *name, hipStream_t stream, uint64_t items) : stream_(stream) {
  if (!g_timing_on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  std::pair<hipEvent_t, hipEvent_t> ev{};
  if (!g_event_pool.empty()) {
    ev = g_event_pool.back();
    g_event_pool.pop_back();
  } else if (hipEventCreate(&ev.first) != hipSuccess || hipEventCreate(&ev.second) != hipSuccess) {
    return;
  }
  if (hipEventRecord(ev.first, stream) != hipSuccess) {
    g_event_pool.push_back(ev);
    return;
  }
  g_records.push_back(TimingRecord{name, ev.first, ev.second, items});
  slot_ = static_cast<int>(g_records.size()) - 1;
}

KernelTimer::~KernelTimer() {
  if (slot_ < 0) return;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (slot_ < static_cast<int>(g_records.size()))
    (void)hipEventRecord(g_records[slot_].stop, stream_);
}

namespace {
thread_local rccl_hip_error_info g_last_error = {RCCL_HIP_SUCCESS, "", 0, 0, 0, 0, 0, 0};
} // namespace

rccl_hip_status set_error(rccl_hip_status status, const char *role, uint64_t expected,
                          uint64_t actual) {
  g_last_error = rccl_hip_error_info{status, role ? role : "", expected, actual, 0, 0, 0, 0};
  return status;
}

rccl_hip_status set_bit_range_error(uint32_t begin, uint32_t end, uint32_t key_bits) {
  g_last_error = rccl_hip_error_info{RCCL_HIP_ERROR_INVALID_BIT_RANGE, "radix bit range", 0, 0,
                                     begin, end, key_bits, 0};
  return RCCL_HIP_ERROR_INVALID_BIT_RANGE;
}

rccl_hip_status set_hip_error(rccl_hip_status status, const char *role, hipError_t err) {
  g_last_error = rccl_hip_error_info{status, role ? role : "", 0, 0, 0, 0, 0,
                                     static_cast<int>(err)};
  return status;
}

rccl_hip_status ok() { return RCCL_HIP_SUCCESS; }

rccl_hip_status check_launch(const char *role) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_LAUNCH, role, err);
  return RCCL_HIP_SUCCESS;
}

rccl_hip_status resident_blocks(const void *kernel, int threads, size_t *blocks) {
  struct Entry {
    int device;
    const void *kernel;
    int threads;
    size_t blocks;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_DRIVER, "current device", err);
  std::lock_guard<std::mutex> lock(mu);
  for (const Entry &e : cache) {
    if (e.device == dev && e.kernel == kernel && e.threads == threads) {
      *blocks = e.blocks;
      return ok();
    }
  }
  int cus = 0, per_cu = 0;
  err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (err == hipSuccess)
    err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0);
  if (err != hipSuccess) return set_hip_error(RCCL_HIP_ERROR_DRIVER, "occupancy", err);
  *blocks = size_t(cus) * size_t(per_cu > 0 ? per_cu : 0);
  cache.push_back(Entry{dev, kernel, threads, *blocks});
  return ok();
}

rccl_hip_status fit_tile_order(const void *kernel, int threads, uint32_t run, uint32_t *nx) {
  if (*nx != XCDS) return ok();
  size_t blocks = 0;
  RCCL_HIP_TRY(resident_blocks(kernel, threads, &blocks));
  if (blocks < 2 * size_t(XCDS) * run) *nx = 1;
  return ok();
}

} // namespace rccl_hip

extern "C" {

void rccl_hip_last_error(rccl_hip_error_info *info) {
  if (info) *info = rccl_hip::g_last_error;
}

const char *rccl_hip_status_string(rccl_hip_status status) {
  switch (status) {
  case RCCL_HIP_SUCCESS: return "success";
  case RCCL_HIP_ERROR_LENGTH_MISMATCH: return "length does not match required length";
  case RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL: return "workspace is smaller than required";
  case RCCL_HIP_ERROR_INVALID_BIT_RANGE: return "radix bit range is outside the key or reversed";
  case RCCL_HIP_ERROR_UNSUPPORTED_TARGET: return "unsupported target: kernels are built for gfx950";
  case RCCL_HIP_ERROR_SIZE_OVERFLOW: return "combined device range length overflowed";
  case RCCL_HIP_ERROR_MEMORY: return "device memory error";
  case RCCL_HIP_ERROR_DRIVER: return "HIP runtime call failed";
  case RCCL_HIP_ERROR_LAUNCH: return "kernel launch failed";
  case RCCL_HIP_ERROR_INVALID_ARGUMENT: return "invalid argument";
  }
  return "unknown status";
}

int rccl_hip_abi_version(void) { return RCCL_HIP_ABI_VERSION; }

rccl_hip_status rccl_hip_timing_enable(int enable) {
  rccl_hip::g_timing_on.store(enable != 0);
  return rccl_hip::ok();
}

rccl_hip_status rccl_hip_timing_read(rccl_hip_kernel_timing *out, size_t capacity, size_t *count) {
  if (!count) return rccl_hip::set_error(RCCL_HIP_ERROR_INVALID_ARGUMENT, "count");
  std::lock_guard<std::mutex> lock(rccl_hip::g_timing_mu);
  auto &recs = rccl_hip::g_records;
  *count = recs.size();
  rccl_hip_status status = rccl_hip::ok();
  for (size_t i = 0; i < recs.size(); ++i) {
    float ms = 0.0f;
    hipError_t err = hipEventSynchronize(recs[i].stop);
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, recs[i].start, recs[i].stop);
    if (err != hipSuccess && status == RCCL_HIP_SUCCESS)
      status = rccl_hip::set_hip_error(RCCL_HIP_ERROR_DRIVER, "kernel timing", err);
    if (out && i < capacity) out[i] = rccl_hip_kernel_timing{recs[i].name, ms, recs[i].items};
    rccl_hip::g_event_pool.emplace_back(recs[i].start, recs[i].stop);
  }
  recs.clear();
  return status;
}

rccl_hip_status rccl_hip_program_load(int device) {
  hipDeviceProp_t prop;
  hipError_t err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) return rccl_hip::set_hip_error(RCCL_HIP_ERROR_DRIVER, "device properties", err);
  // gcnArchName looks like "gfx950:sramecc+:xnack-".
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0 ||
      (prop.gcnArchName[6] != '\0' && prop.gcnArchName[6] != ':'))
    return rccl_hip::set_error(RCCL_HIP_ERROR_UNSUPPORTED_TARGET, "gfx950 kernels");
  // Once per device, on that device: probe the LDS lane order and the XCD
  // placement the radix sort relies on, and find the static workspace.
  static std::mutex mu;
  static std::vector<int> checked;
  std::lock_guard<std::mutex> lock(mu);
  for (int d : checked)
    if (d == device) return rccl_hip::ok();
  int current = 0;
  err = hipGetDevice(&current);
  if (err == hipSuccess) err = hipSetDevice(device);
  if (err != hipSuccess) return rccl_hip::set_hip_error(RCCL_HIP_ERROR_DRIVER, "set device", err);
  rccl_hip_status st = rccl_hip::radix::probe_current_device();
  // The static radix workspace's device address, looked up with the device
  // current (rccl_hip_radix_sort_static).
  void *static_ws = nullptr;
  if (st == RCCL_HIP_SUCCESS) st = rccl_hip::radix::static_workspace(&static_ws);
  err = hipSetDevice(current);
  if (st != RCCL_HIP_SUCCESS) return st;
  if (err != hipSuccess) return rccl_hip::set_hip_error(RCCL_HIP_ERROR_DRIVER, "set device", err);
  checked.push_back(device);
  return rccl_hip::ok();
}

} // extern "C"
