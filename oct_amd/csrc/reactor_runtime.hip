// Runtime lifecycle, probe, diagnostics, device memory and stream timing.
//
// Reference semantics followed:
//   create/destroy/probe   internal/prometheus/native/reactor_sgemm.cpp:2955-3203
//                          (second destroy -> PROM_INVALID_HANDLE; probe of a
//                          runtime without a device -> available 0, backend
//                          UNKNOWN, reason VULKAN_UNAVAILABLE, as asserted by
//                          Marionette/reactor_stub_tests.cpp:164-185)
//   config struct_size gating  reactor_api.h:1751-1769
#include <stddef.h>
#include <string.h>
#include <time.h>

#include <unordered_set>

#include "reactor_internal.h"

namespace prom {

namespace {
std::mutex g_registry_mu;
std::unordered_set<void*>& registry() {
  static std::unordered_set<void*> handles;
  return handles;
}
}  // namespace

DeviceContext& ctx() {
  static DeviceContext context;
  return context;
}

uint64_t wall_ns() {
  timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

bool ensure_device() {
  DeviceContext& c = ctx();
  std::lock_guard<std::mutex> lock(c.mu);
  if (c.probed) return c.available;
  c.probed = true;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    (void)hipGetLastError();
    return false;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  if (hipSetDevice(dev) != hipSuccess) return false;
  if (hipGetDeviceProperties(&c.props, dev) != hipSuccess) return false;
  if (c.props.name[0] == '\0' && hipDeviceGetName(c.props.name, (int)sizeof(c.props.name), dev) != hipSuccess) {
    c.props.name[0] = '\0';
  }
  // One non-blocking stream at the default priority carries every launch.
  if (hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking) != hipSuccess) return false;
  for (uint32_t i = 0; i < kEventSlots; ++i) {
    if (hipEventCreate(&c.events[i]) != hipSuccess) return false;
  }
  if (hipEventCreate(&c.op_begin) != hipSuccess || hipEventCreate(&c.op_end) != hipSuccess) return false;
  c.device = dev;
  c.available = true;
  // Device address of the allocation-free SGEMM's scratch array; on failure
  // only that entry reports PROM_DETAIL_SCRATCH_UNAVAILABLE.
  (void)init_sgemm_scratch(dev);
  return true;
}

Runtime* lookup(void* handle) {
  if (handle == nullptr) return nullptr;
  std::lock_guard<std::mutex> lock(g_registry_mu);
  if (registry().count(handle) == 0) return nullptr;
  Runtime* rt = static_cast<Runtime*>(handle);
  return rt->magic == kRuntimeMagic ? rt : nullptr;
}

void* staging(uint32_t slot, size_t bytes) {
  DeviceContext& c = ctx();
  if (slot >= kStagingSlots) return nullptr;
  if (bytes == 0) bytes = 256;
  if (c.staging_bytes[slot] >= bytes) return c.staging[slot];
  if (c.staging[slot] != nullptr) {
    // The stream may still use the old buffer.
    if (hipStreamSynchronize(c.stream) != hipSuccess) return nullptr;
    (void)hipFree(c.staging[slot]);
    c.staging[slot] = nullptr;
    c.staging_bytes[slot] = 0;
  }
  // Round up to 2 MiB so that a sweep of growing shapes does not reallocate each call.
  const size_t rounded = (bytes + (2u << 20) - 1) & ~(size_t)((2u << 20) - 1);
  void* p = nullptr;
  if (hipMalloc(&p, rounded) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  c.staging[slot] = p;
  c.staging_bytes[slot] = rounded;
  ++c.staging_allocations;
  return p;
}

}  // namespace prom

using namespace prom;

extern "C" {

PROM_REACTOR_API uint32_t prometheus_reactor_abi_version(void) { return PROM_REACTOR_ABI_V1; }

PROM_REACTOR_API int prometheus_reactor_runtime_create(void* config, void** out_handle) {
  if (out_handle == nullptr) return PROM_ERROR;
  *out_handle = nullptr;
  uint32_t test_flags = 0, reduction_flags = 0, ring_depth = 0;
  if (config != nullptr) {
    const PrometheusReactorConfig* cfg = static_cast<const PrometheusReactorConfig*>(config);
    if (cfg->struct_size >= offsetof(PrometheusReactorConfig, p15_shadow_disabled)) test_flags = cfg->test_flags;
    if (cfg->struct_size >= offsetof(PrometheusReactorConfig, reduction_test_flags)) ring_depth = cfg->batch_ring_depth;
    if (cfg->struct_size >= offsetof(PrometheusReactorConfig, reduction_ring_depth))
      reduction_flags = cfg->reduction_test_flags;
  }
  Runtime* rt = new (std::nothrow) Runtime();
  if (rt == nullptr) return PROM_INTERNAL_ERROR;
  memset(rt, 0, sizeof(*rt));
  rt->magic = kRuntimeMagic;
  rt->test_flags = test_flags;
  rt->reduction_test_flags = reduction_flags;
  // reactor_api.h:1759-1760: zero keeps the default depth of two; at most four.
  rt->batch_ring_depth = ring_depth == 0u ? 2u : (ring_depth > 4u ? 4u : ring_depth);
  if ((test_flags & (PROM_TESTCFG_SKIP_VULKAN_INIT | PROM_TESTCFG_FAIL_DEVICE_CREATE)) != 0u) {
    rt->available = 0;
    rt->init_detail = PROM_DETAIL_HIP_UNAVAILABLE;
  } else if (ensure_device()) {
    rt->available = 1;
    rt->init_detail = 0;
  } else {
    rt->available = 0;
    rt->init_detail = PROM_DETAIL_HIP_UNAVAILABLE;
  }
  {
    std::lock_guard<std::mutex> lock(g_registry_mu);
    registry().insert(rt);
  }
  *out_handle = rt;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_destroy(void* handle) {
  Runtime* rt = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_registry_mu);
    if (handle == nullptr || registry().count(handle) == 0) return PROM_INVALID_HANDLE;
    registry().erase(handle);
    rt = static_cast<Runtime*>(handle);
  }
  if (rt->available) {
    DeviceContext& c = ctx();
    std::lock_guard<std::mutex> lock(c.mu);
    (void)hipStreamSynchronize(c.stream);
  }
  async_release(rt);
  model_release(rt);
  rt->magic = 0;
  delete rt;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_probe(void* handle, PrometheusCaps* out_caps) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (out_caps == nullptr) return PROM_ERROR;
  if (rt->available) {
    out_caps->available = 1;
    out_caps->backend_type = PROM_BACKEND_HARDWARE_GPU;
    out_caps->reason_code = PROM_REASON_NONE;
  } else {
    out_caps->available = 0;
    out_caps->backend_type = PROM_BACKEND_UNKNOWN;
    out_caps->reason_code = PROM_REASON_VULKAN_UNAVAILABLE;
  }
  return PROM_OK;
}

// reactor_api.c:801-812: the earlier contract drafts' names forward unchanged.
PROM_REACTOR_API int prometheus_runtime_create(void* config, void** out_handle) {
  return prometheus_reactor_runtime_create(config, out_handle);
}

PROM_REACTOR_API int prometheus_runtime_destroy(void* handle) { return prometheus_reactor_runtime_destroy(handle); }

PROM_REACTOR_API int prometheus_runtime_probe(void* handle, PrometheusCaps* out_caps) {
  return prometheus_reactor_runtime_probe(handle, out_caps);
}

PROM_REACTOR_API int prometheus_reactor_runtime_vulkan_device_diagnostics(void* handle,
                                                                           PrometheusVulkanDeviceDiagnostics* out_diag) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (out_diag == nullptr) return PROM_ERROR;
  memset(out_diag, 0, sizeof(*out_diag));
  if (!rt->available) return PROM_ERROR;
  const hipDeviceProp_t& p = ctx().props;
  strncpy(out_diag->device_name, p.name, sizeof(out_diag->device_name) - 1);
  out_diag->vendor_id = 0x1002u;  // AMD PCI vendor id
  out_diag->device_id = (uint32_t)p.pciDeviceID;
  out_diag->device_type = 2u;     // discrete GPU
  int runtime_version = 0;
  (void)hipRuntimeGetVersion(&runtime_version);
  out_diag->api_version = (uint32_t)runtime_version;
  int driver_version = 0;
  (void)hipDriverGetVersion(&driver_version);
  out_diag->driver_version = (uint32_t)driver_version;
  out_diag->software_vulkan = 0;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_hip_device_diagnostics(void* handle,
                                                                        PrometheusHipDeviceDiagnostics* out_diag) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (out_diag == nullptr || out_diag->struct_size < offsetof(PrometheusHipDeviceDiagnostics, staging_allocations))
    return PROM_ERROR;
  const uint32_t size = out_diag->struct_size;
  const bool has_staging = size >= sizeof(PrometheusHipDeviceDiagnostics);
  memset(out_diag, 0, has_staging ? sizeof(*out_diag) : offsetof(PrometheusHipDeviceDiagnostics, staging_allocations));
  out_diag->struct_size = size;
  if (!rt->available) return PROM_ERROR;
  const DeviceContext& c = ctx();
  const hipDeviceProp_t& p = c.props;
  strncpy(out_diag->device_name, p.name, sizeof(out_diag->device_name) - 1);
  strncpy(out_diag->gcn_arch_name, p.gcnArchName, sizeof(out_diag->gcn_arch_name) - 1);
  out_diag->compute_units = (uint32_t)p.multiProcessorCount;
  out_diag->clock_khz = (uint32_t)p.clockRate;
  out_diag->memory_clock_khz = (uint32_t)p.memoryClockRate;
  out_diag->memory_bus_width = (uint32_t)p.memoryBusWidth;
  out_diag->total_global_mem = (uint64_t)p.totalGlobalMem;
  out_diag->lds_bytes_per_workgroup = (uint32_t)p.sharedMemPerBlock;
  out_diag->wavefront_size = (uint32_t)p.warpSize;
  int runtime_version = 0;
  (void)hipRuntimeGetVersion(&runtime_version);
  out_diag->hip_runtime_version = runtime_version;
  out_diag->device_ordinal = c.device;
  if (has_staging) {
    std::lock_guard<std::mutex> lock(ctx().mu);
    out_diag->staging_allocations = c.staging_allocations;
    for (uint32_t i = 0; i < kStagingSlots; ++i) out_diag->staging_bytes += c.staging_bytes[i];
  }
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_device_alloc(void* handle, uint64_t bytes, void** out_device_ptr) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (out_device_ptr == nullptr || bytes == 0) return PROM_ERROR;
  *out_device_ptr = nullptr;
  if (!rt->available || (rt->test_flags & PROM_TESTCFG_FAIL_BUFFER_ALLOC)) return PROM_ERROR;
  void* p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return PROM_ERROR;
  }
  *out_device_ptr = p;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_device_free(void* handle, void* device_ptr) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (!rt->available) return PROM_ERROR;
  if (device_ptr == nullptr) return PROM_OK;
  DeviceContext& c = ctx();
  if (hipStreamSynchronize(c.stream) != hipSuccess) return PROM_ERROR;
  return hipFree(device_ptr) == hipSuccess ? PROM_OK : PROM_ERROR;
}

PROM_REACTOR_API int prometheus_reactor_runtime_device_upload(void* handle, void* device_dst, const void* host_src,
                                                              uint64_t bytes) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (!rt->available || device_dst == nullptr || host_src == nullptr) return PROM_ERROR;
  DeviceContext& c = ctx();
  if (hipMemcpyAsync(device_dst, host_src, bytes, hipMemcpyHostToDevice, c.stream) != hipSuccess) return PROM_ERROR;
  return hipStreamSynchronize(c.stream) == hipSuccess ? PROM_OK : PROM_ERROR;
}

PROM_REACTOR_API int prometheus_reactor_runtime_device_download(void* handle, void* host_dst, const void* device_src,
                                                                uint64_t bytes) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (!rt->available || host_dst == nullptr || device_src == nullptr) return PROM_ERROR;
  DeviceContext& c = ctx();
  if (hipMemcpyAsync(host_dst, device_src, bytes, hipMemcpyDeviceToHost, c.stream) != hipSuccess) return PROM_ERROR;
  return hipStreamSynchronize(c.stream) == hipSuccess ? PROM_OK : PROM_ERROR;
}

PROM_REACTOR_API int prometheus_reactor_runtime_synchronize(void* handle) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (!rt->available) return PROM_ERROR;
  return hipStreamSynchronize(ctx().stream) == hipSuccess ? PROM_OK : PROM_ERROR;
}

PROM_REACTOR_API int prometheus_reactor_runtime_event_record(void* handle, uint32_t slot) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (!rt->available || slot >= kEventSlots) return PROM_ERROR;
  DeviceContext& c = ctx();
  return hipEventRecord(c.events[slot], c.stream) == hipSuccess ? PROM_OK : PROM_ERROR;
}

PROM_REACTOR_API int prometheus_reactor_runtime_event_elapsed_ms(void* handle, uint32_t start_slot, uint32_t end_slot,
                                                                 float* out_ms) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (!rt->available || out_ms == nullptr || start_slot >= kEventSlots || end_slot >= kEventSlots) return PROM_ERROR;
  DeviceContext& c = ctx();
  if (hipEventSynchronize(c.events[end_slot]) != hipSuccess) return PROM_ERROR;
  return hipEventElapsedTime(out_ms, c.events[start_slot], c.events[end_slot]) == hipSuccess ? PROM_OK : PROM_ERROR;
}

}  // extern "C"
