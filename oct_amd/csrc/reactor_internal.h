// Internal declarations shared by the reactor's translation units.
//
// One process-wide device context owns the HIP device, a single stream on
// which every launch is queued, grow-only staging buffers for host-pointer
// calls and a ring of timing events.  Runtime handles are cheap records in a
// registry (the reference keeps a global handle registry too:
// internal/prometheus/native/reactor_sgemm.cpp:1370-1565).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/prometheus_reactor.h"

namespace prom {

constexpr uint64_t kRuntimeMagic = 0x4F43544D49333535ull;  // "OCTMI355"
constexpr uint32_t kEventSlots = 64;
// Staging slots: 0-3 operand staging, 4 block workspace, 5 block host staging,
// 6 split-K partials, 7 FFT twiddle table.
constexpr uint32_t kStagingSlots = 8;

struct AsyncState;  // async task table, submission slots and batch arenas (sgemm_async.hip)

struct Runtime {
  uint64_t magic;
  uint32_t test_flags;
  uint32_t reduction_test_flags;
  uint32_t available;       // 1 when a HIP device is usable by this handle
  int32_t init_detail;      // reason when unavailable
  uint64_t requests;
  uint64_t successes;
  uint32_t batch_ring_depth;  // 1..4 (config batch_ring_depth; 0 selects 2)
  AsyncState* async;          // created on first async or batch call
  // Gemma-4-E2B M1 committed RMSNorm weight (generation 0: none committed yet).
  uint64_t m1_weight_generation;
  uint64_t m1_weight_hash;
  uint32_t m1_weight_width;
};

struct DeviceContext {
  std::mutex mu;            // serialises host-pointer calls and staging reuse
  bool probed = false;
  bool available = false;
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t events[kEventSlots] = {};
  hipEvent_t op_begin = nullptr, op_end = nullptr;
  void* staging[kStagingSlots] = {};
  size_t staging_bytes[kStagingSlots] = {};
  void* fft_roots = nullptr;  // twiddle table in staging slot 7 for length fft_roots_n
  uint32_t fft_roots_n = 0;
  hipDeviceProp_t props{};
};

DeviceContext& ctx();
// Initialises the device context once; returns true when a device is usable.
bool ensure_device();
// Validates a handle against the registry; returns nullptr when invalid.
Runtime* lookup(void* handle);
// Grow-only device staging buffer `slot` of at least `bytes`.
void* staging(uint32_t slot, size_t bytes);

// Unconsumed async tasks of a runtime (READY and FAILED count until consumed
// or abandoned); the synchronous SGEMM is rejected while this is non-zero.
uint32_t async_outstanding(Runtime* rt);
// Waits for the runtime's queued work and frees its async/batch resources.
void async_release(Runtime* rt);

inline void set_status(uint32_t* stage, int* detail, uint32_t s, int d) {
  if (stage) *stage = s;
  if (detail) *detail = d;
}

uint64_t wall_ns();

// ---- kernel launchers (enqueue on `stream`; return hipSuccess or the launch error)
hipError_t launch_sgemm_f32(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                            hipStream_t stream, int* path_detail);
// Strided forms used by the transformer blocks (leading dimensions in elements;
// residual may be null or alias c; gemm_bf16 writes bf16 to cb when non-null).
hipError_t launch_sgemm_f32_ex(const float* a, int lda, const float* b, int ldb, float* c, int ldc, uint32_t m,
                               uint32_t n, uint32_t k, const float* residual, int ldr, hipStream_t stream,
                               int* path_detail);
hipError_t launch_gemm_bf16_ex(const uint16_t* a, int lda, const uint16_t* b, int ldb, float* c, uint16_t* cb,
                               int ldc, uint32_t m, uint32_t n, uint32_t k, const float* residual, int ldr,
                               hipStream_t stream, int* path_detail);
hipError_t launch_gemm_bf16(const uint16_t* a, const uint16_t* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                            hipStream_t stream, int* path_detail);
// h[m, f] (bf16) = silu(a @ w13[:, :f]) * (a @ w13[:, f:]) in one GEMM; returns
// hipErrorNotSupported, launching nothing, when the shape is outside the fused path.
hipError_t launch_gemm_bf16_swiglu(const uint16_t* a, int lda, const uint16_t* w13, uint16_t* h, int ldh, uint32_t m,
                                   uint32_t f, uint32_t k, hipStream_t stream);
// Binary64 FFT of n = 2^k <= 2^20 points (interleaved complex); temp holds n
// points and is used when n > 4096.  roots comes from fft64_roots(n).
hipError_t launch_fft64(const double2* in, double2* out, double2* temp, const double2* roots, uint32_t n,
                        hipStream_t stream);
// Device twiddle table for length n (cached; caller holds ctx().mu).
const double2* fft64_roots(uint32_t n);
hipError_t launch_row_reduction(const float* in, float* out, uint32_t rows, uint32_t width, uint32_t op,
                                hipStream_t stream);
hipError_t launch_rmsnorm(const float* in, const float* w, float* out, float* inv_rms, uint32_t tokens,
                          uint32_t width, uint32_t stride, float eps, hipStream_t stream);

}  // namespace prom
