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

#include <algorithm>
#include <mutex>

#include "../../include/prometheus_reactor.h"

namespace prom {

// Workgroups of a launch are dealt to the 8 XCDs round-robin (workgroup b to
// XCD b % 8).  xcd_pid(b, n) renumbers a grid of n workgroups so that XCD x
// runs the contiguous range of ids starting at x * (n / 8) + min(x, n % 8)
// (n / 8 or n / 8 + 1 of them, for any n), in increasing order: work items
// with neighbouring ids share their operands in that XCD's L2.
__device__ __forceinline__ int xcd_pid(int b, int n) {
  const int x = b & 7, q = n >> 3, r = n & 7;
  return x * q + min(x, r) + (b >> 3);
}

// max / sum of v over lanes l and l ^ 32 of a wave64 (the attention kernels
// keep a query's scores in the two 32-lane halves).  v_permlane32_swap with v
// as both operands returns v[l & 31] and v[l | 32] in every lane l, in
// registers; __shfl_xor(v, 32) is an LDS permute round trip.
__device__ __forceinline__ float max_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// silu(g) * u = g / (1 + e^-g) * u with the hardware base-2 exponential and
// reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each, so ~3e-7 relative
// error before the bf16 rounding of the result); every bf16 SwiGLU of the DiT
// block uses this form: the fused GEMM epilogues, the K-split sum and the
// separate elementwise kernel.  e^-g overflows to infinity for g < -88 and
// the product goes to -0, as silu does.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// Tanh-approximate GELU of the fp32 Gemma-style layer's GeGLU (the reference
// has none; Gemma uses this form): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  return 0.5f * x * (1.0f + tanhf(k0 * (x + k1 * x * x * x)));
}

constexpr uint64_t kRuntimeMagic = 0x4F43544D49333535ull;  // "OCTMI355"
constexpr uint32_t kEventSlots = 64;
// Staging slots: 0-3 operand staging, 4 block workspace, 5 block host staging,
// 6 split-K partials, 7 FFT twiddle table, 8-9 padded SGEMM operand copies.
constexpr uint32_t kStagingSlots = 10;

struct AsyncState;  // async task table, submission slots and batch arenas (sgemm_async.hip)
struct ModelState;  // resident model block and compiled session (model_block.hip)

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
  ModelState* model;  // created by the first model-block or session call
  PrometheusFftDiagnostics fft_diag;  // the last fp32 FFT call (struct_size 0 before the first)
  // Row-reduction calls (reduction, reduction_v2, row_wise_softmax) for the diagnostics entry.
  uint64_t reduction_total, reduction_successes, reduction_failures;
  uint64_t reduction_last_replay, reduction_last_gpu_ns, reduction_last_e2e_ns;
  uint32_t reduction_last_stages;
  int32_t reduction_last_detail;
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
  uint64_t staging_allocations = 0;  // hipMalloc calls made by staging(), for the diagnostics
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
// Copies of caller-owned pageable host buffers (host_copy.hip).  upload_host
// returns once `src` has been read (the device side completes in stream
// order); download_host returns once `dst` holds the data.
hipError_t upload_host(void* dst, const void* src, size_t bytes, hipStream_t stream);
// memcpy between host buffers on the same host threads (1 MiB and more).
void host_memcpy(void* dst, const void* src, size_t bytes);
hipError_t download_host(void* dst, const void* src, size_t bytes, hipStream_t stream);

// Unconsumed async tasks of a runtime (READY and FAILED count until consumed
// or abandoned); the synchronous SGEMM is rejected while this is non-zero.
uint32_t async_outstanding(Runtime* rt);
// Waits for the runtime's queued work and frees its async/batch resources.
void async_release(Runtime* rt);
// Frees the runtime's resident model block, session and their device memory.
void model_release(Runtime* rt);

// GEMM admission: every dimension fits the kernels' signed 32-bit index type
// and each operand holds fewer than 2^32 elements.  The reference refuses
// m*n*k >= 2^32 (reactor_sgemm.cpp:4186-4191), which excludes 4096^3; this
// limit admits it and still rejects any shape whose leading dimension or
// tile count would wrap an int.
inline bool gemm_shape_fits(uint32_t m, uint32_t n, uint32_t k) {
  const uint64_t lim = 1ull << 32;
  if (m > 0x7fffffffu || n > 0x7fffffffu || k > 0x7fffffffu) return false;
  return (uint64_t)m * k < lim && (uint64_t)k * n < lim && (uint64_t)m * n < lim;
}

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
// C = A @ B with the K-split slices left unreduced for a consumer that adds
// them itself: when the product's schedule is one K-split product of at most
// max_slices slices (no GEMV, padded copies or tail split) and `partial` holds
// them, slice z goes to partial + z*m*n ([m, n], row pitch n), *slices is set
// and nothing is written to c; otherwise c is computed in full and *slices is
// 1.  The slices are those launch_sgemm_f32_ex's reduce would add, in the
// same plan, so adding them in slice order reproduces its output bit for bit.
hipError_t launch_sgemm_f32_unreduced(const float* a, int lda, const float* b, int ldb, float* c, int ldc,
                                      uint32_t m, uint32_t n, uint32_t k, float* partial, size_t partial_floats,
                                      int max_slices, hipStream_t stream, int* slices);
// The slices launch_sgemm_f32_unreduced leaves for 16-byte aligned operands (1: none).
int sgemm_f32_unreduced_slices(int lda, int ldb, uint32_t m, uint32_t n, uint32_t k, int max_slices);
// H[m, f] = gelu_tanh(A @ W[:, :f]) * (A @ W[:, f:]) for W = [gate | up]
// ([k, 2f], row pitch 2f): one launch of the 128x128 direct-to-LDS kernel
// whose tiles take 64 gate and the matching 64 up columns.  Returns
// hipErrorNotSupported when the shape does not fit it (f % 64, k % 16,
// 16-byte aligned operands and rows, byte offsets below 2^31); the caller
// then runs the GEMM and the elementwise GeGLU.
hipError_t launch_sgemm_f32_geglu(const float* a, int lda, const float* w, float* h, int ldh, uint32_t m, uint32_t f,
                                  uint32_t k, hipStream_t stream);
// C_z = A_z @ B_z for z < batch, A_z = a + z*sa etc. (elements); no residual, no split-K.
// Allocation-free SGEMM: split-K partials in the library's static scratch
// array.  init_sgemm_scratch(device) runs once per device at set-up (device
// current).  launch_sgemm_f32_noalloc returns PROM_OK,
// PROM_DETAIL_SCRATCH_LIMIT, PROM_DETAIL_SCRATCH_UNAVAILABLE or
// PROM_DETAIL_HIP_LAUNCH_FAILED.
hipError_t init_sgemm_scratch(int device);
int launch_sgemm_f32_noalloc(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                             int device, hipStream_t stream, int* path_detail);
// One product with a caller-chosen kernel variant (tile index as in
// PrometheusSgemmPlanInfo's tables, K slices); hipErrorInvalidValue when the
// variant cannot run this shape.  Caller holds ctx().mu (split-K staging).
hipError_t launch_sgemm_f32_variant(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                                    uint32_t tile, uint32_t k_slices, hipStream_t stream);
hipError_t launch_sgemm_f32_batched(const float* a, int lda, long long sa, const float* b, int ldb, long long sb,
                                    float* c, int ldc, long long sc, uint32_t m, uint32_t n, uint32_t k,
                                    uint32_t batch, hipStream_t stream);
// K-blocked A: a_slice > 0 says A is stored as [k/32][a_slice][32] (the 32
// consecutive k of one row are 64 contiguous bytes, rows of a slice adjacent,
// a_slice >= m rounded up to 256), so every HBM -> LDS transfer of A moves
// whole 128-byte lines; only the four-stage kernel reads it, and
// gemm_bf16_takes_blocked_a says whether a shape runs there (with a_slice == 0
// A is row-major with row stride lda).  hipErrorNotSupported otherwise.
hipError_t launch_gemm_bf16_ex(const uint16_t* a, int lda, const uint16_t* b, int ldb, float* c, uint16_t* cb,
                               int ldc, uint32_t m, uint32_t n, uint32_t k, const float* residual, int ldr,
                               hipStream_t stream, int* path_detail, int a_slice = 0);
// True when launch_gemm_bf16_ex runs this shape on the four-stage kernel (a:
// 16-byte aligned, lda its row-major stride).
bool gemm_bf16_takes_blocked_a(const uint16_t* a, int lda, const uint16_t* b, int ldb, uint32_t m, uint32_t n,
                               uint32_t k);
// The same for the fused SwiGLU GEMM, whose four-stage kernel also writes H
// K-blocked ([f/32][h_slice][32]) for a following GEMM when h_slice > 0.
bool gemm_bf16_swiglu_takes_blocked_a(const uint16_t* a, int lda, const uint16_t* w13, uint32_t m, uint32_t f,
                                      uint32_t k);
hipError_t launch_gemm_bf16(const uint16_t* a, const uint16_t* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                            hipStream_t stream, int* path_detail);
// h[m, f] (bf16) = silu(a @ w13[:, :f]) * (a @ w13[:, f:]) in one GEMM; returns
// hipErrorNotSupported, launching nothing, when the shape is outside the fused path.
// part_ws (part_bytes, may be null) takes the K-slice sums of the tiles of a
// final partial wave, which are then split along K; their fixed slice order
// keeps the result deterministic.  *launches (when given) receives the number
// of kernels queued.
// a_slice / h_slice > 0 (K-blocked A or H) only where
// gemm_bf16_swiglu_takes_blocked_a holds; hipErrorInvalidValue otherwise.
hipError_t launch_gemm_bf16_swiglu(const uint16_t* a, int lda, const uint16_t* w13, uint16_t* h, int ldh, uint32_t m,
                                   uint32_t f, uint32_t k, hipStream_t stream, void* part_ws, size_t part_bytes,
                                   uint32_t* launches = nullptr, int a_slice = 0, int h_slice = 0);
// bf16 flash attention, head dim 128, full (non-causal): Q/K/V/O [T, ld*] with
// head h at column 128 h.  variant 0: K/V tiles moved HBM -> LDS by DMA (64 KiB
// of dynamic LDS); 1: tiles staged through registers.  hipErrorInvalidValue for
// other variants.
hipError_t launch_flash_attn_bf16(const uint16_t* q, int ldq, const uint16_t* k, int ldk, const uint16_t* v, int ldv,
                                  uint16_t* o, int ldo, int T, int heads, float scale, hipStream_t stream,
                                  int variant);
// Variant 0 with the DiT block's per-head RMSNorm (weights qn [128], eps) and
// RoPE (rope [T][64] (cos, sin) per pair) applied to the raw Q rows as they
// are loaded, with k_norm_rope_kernel's arithmetic (dit_block.hip).  o_slice
// > 0 writes O K-blocked ([128 heads / 32][o_slice][32], o_slice >= T) for a
// following launch_gemm_bf16_ex with that a_slice; 0 writes rows of stride ldo.
hipError_t launch_flash_attn_bf16_qnorm_rope(const uint16_t* q, int ldq, const uint16_t* k, int ldk, const uint16_t* v,
                                            int ldv, uint16_t* o, int ldo, int T, int heads, float scale,
                                            const float2* rope, const float* qn, const float* kn, float eps,
                                            hipStream_t stream, int o_slice = 0);
// Binary64 FFT of n = 2^k <= 2^20 points (interleaved complex); temp holds n
// points and is used when n > 4096.  roots comes from fft64_roots(n).
hipError_t launch_fft64(const double2* in, double2* out, double2* temp, const double2* roots, uint32_t n,
                        hipStream_t stream);
// Device twiddle table for length n (cached; caller holds ctx().mu): the n/2
// roots, followed for n > 4096 by the four-step passes' compact tables.
const double2* fft64_roots(uint32_t n);
hipError_t launch_row_reduction(const float* in, float* out, uint32_t rows, uint32_t width, uint32_t op,
                                hipStream_t stream);
// Binary64 reference of the same row reduction (the benchmark's correctness check).
hipError_t launch_row_reduction_check(const float* in, float* out, uint32_t rows, uint32_t width, uint32_t op,
                                      hipStream_t stream);
hipError_t launch_rmsnorm(const float* in, const float* w, float* out, float* inv_rms, uint32_t tokens,
                          uint32_t width, uint32_t stride, float eps, hipStream_t stream);

// ---- fp32 flash attention (attention_f32.hip)
// O[t][hq*d + c] = sum_s softmax_s(scale * Q[hq][t] . K[hkv][s]) V[hkv][s][c] with
// hkv = hq / group, keys s <= t when causal.  Element strides: Q[hq][t][c] at
// q + hq*q_hs + t*q_rs + c; K^T[hkv][c][s] at kt + hkv*kt_hs + c*kt_rs + s;
// V[hkv][s][c] at v + hkv*v_hs + s*v_rs + c; O[t][hq*d + c] at o + t*o_rs + hq*d + c.
// part_o / part_ml hold key-split partials when flash_attn_f32_partial_bytes > 0.
struct AttnF32Params {
  const float* q;
  const float* kt;
  const float* v;
  float* o;
  float* part_o;
  float* part_ml;
  long long q_hs, kt_hs, v_hs;
  int q_rs, kt_rs, v_rs, o_rs;
  int T, q_heads, group, causal;
};
bool flash_attn_f32_supported(int head_dim);
// Partial buffer bytes the launch needs (0: none); flash_attn_f32_bind_partials
// points part_o and part_ml into such a buffer.
size_t flash_attn_f32_partial_bytes(int T, int q_heads, int group, int head_dim, int causal);
void flash_attn_f32_bind_partials(AttnF32Params& p, int head_dim, void* buffer);
hipError_t launch_flash_attn_f32(const AttnF32Params& p, int head_dim, float scale, hipStream_t stream);

// ---- fp32 Z-Image transformer block on resident weights (zimage_f32.hip)
constexpr int kZImageConditionWidth = 256;  // timestep embedding width (adaLN input)

// Workspace buffers of one block execution (byte offsets from zimage_workspace_layout).
enum ZImageWorkspace {
  kZModRaw,  // [4D] adaLN projection before adjustment
  kZMod,     // [4D] scaleA+1 | tanh gateA | scaleM+1 | tanh gateM
  kZA,       // [T, D] RMSNorm(x; n1) * scaleA
  kZQkv,     // [T, 3D]
  kZQ,       // [H, T, 128] normalized, rotated, scaled by 1/sqrt(128)
  kZKt,      // [H, 128, T] normalized, rotated, transposed
  kZV,       // [H, T, 128]
  kZS,       // flash-attention key-split partials (no score matrix)
  kZO,       // [T, D] attention aggregation
  kZProj,    // [T, D] attention projection
  kZR,       // [T, D] attention residual
  kZF,       // [T, D] RMSNorm(r; n3) * scaleM
  kZG,       // [T, 2F] w1 | w3
  kZH,       // [T, F] gated hidden
  kZW2,      // [T, D]
  kZRope,    // [T, 64] (cos, sin), filled by launch_zimage_rope_table
  kZCount
};

struct ZImageBlockWeights {
  const float* adaln_w;  // [256, 4D]; null for the unmodulated ContextRefiner
  const float* adaln_b;  // [4D]
  const float* attn_norm1;
  const float* attn_norm2;
  const float* ffn_norm1;
  const float* ffn_norm2;  // [D] each
  const float* q_norm;
  const float* k_norm;  // [128] each
  const float* w_qkv;   // [D, 3D]
  const float* w_out;   // [D, D]
  const float* w_13;    // [D, 2F]: w1 in columns [0, F), w3 in [F, 2F)
  const float* w_2;     // [F, D]
};

size_t zimage_workspace_layout(int T, int D, int H, int F, size_t off[kZCount]);
// dst[r * dst_ld + c] = (float) fp16 src[r * cols + c]
hipError_t launch_widen_f16(const uint16_t* src, float* dst, size_t rows, size_t cols, size_t dst_ld,
                            hipStream_t stream);
hipError_t launch_widen_bf16(const uint16_t* src, float* dst, size_t n, hipStream_t stream);
// coords [T, 3] (frame, row, column) -> workspace rope table
hipError_t launch_zimage_rope_table(const float* coords, float2* tab, int T, hipStream_t stream);
// One block: out = block(x); cond [256] is read only when w.adaln_w is set;
// the workspace rope table must already hold this sequence's coordinates.
// The block runs in three phases, first_phase..last_phase of: 1 adaLN to the
// Q/K/V split (pre-attention), 2 attention to the gated residual and FFN
// input, 3 the FFN and final residual.  A later phase reads the workspace the
// earlier ones left, so 2..2 re-runs the attention of the last phase 1.
// stage_events (null: none; else 14 events) are recorded before the first of
// the 13 stages (adaLN, norm, QKV, head norm + RoPE, scores, softmax, P.V,
// projection, gated residual + FFN norm, W1|W3, SwiGLU, W2, final residual)
// and after each one.
hipError_t enqueue_zimage_block_f32(const ZImageBlockWeights& w, const float* x, const float* cond, float* out,
                                    char* ws, const size_t off[kZCount], int T, int D, int F, float eps,
                                    hipStream_t st, uint32_t* launches, int first_phase, int last_phase,
                                    const hipEvent_t* stage_events = nullptr);
// Audit recomputations: out = RMSNorm(x; w) (no modulation), and q or k
// (which 0 / 1) after the head RMSNorm and optionally RoPE, [T, H*128].
hipError_t launch_zimage_norm(const float* x, const float* w, float* out, int T, int D, float eps, hipStream_t stream);
hipError_t launch_zimage_qk_audit(const float* qkv, const float2* tab, const float* norm_w, float* out, int T, int H,
                                  float eps, int which, bool rope, hipStream_t stream);

// One 256-byte (64-word) audit summary record of the fp32 view
// v[e] = src[(e / cols) * ld + e % cols], 0 <= e < count: words 0 stage,
// 1 generation, 2 count, 3 all-finite flag, 4 NaN count, 5 infinity count,
// 6 finite count, 7 key count, 8 min, 9 max, 10 sum of squares, 11 RMS (finite
// values; quiet NaN when none), 12 completion (1), 13 status (1 if a key is out
// of range), 16 + 2i / 17 + 2i (key i, v[key i]); other words zero
// (shaders/sdslv/production/zimage/nr0_persistent_audit_summary.sdslv:56-217).
struct ZImageAuditJob {
  const float* src;
  uint32_t count, cols, ld, stage_id;
  uint32_t generation, dest_word, key_count, reserved;
  uint32_t keys[16];
};
constexpr uint32_t kZImageAuditMaxKeys = 15u;
// One workgroup per job; jobs and arena are device memory.
hipError_t launch_zimage_audit_summary(const ZImageAuditJob* jobs, uint32_t job_count, uint32_t* arena,
                                       hipStream_t stream);
// The 64-float streaming-attention witness of (token 0, head 0) at out[0..31]
// and (token T-1, head H-1) at out[32..63] from the split Q (scaled by
// q_scale) [H, T, 128], K^T [H, 128, T], V [H, T, 128] and the attention
// output O [T, H*128].  image_format selects the NoiseRefiner record
// (nr0_attention_streaming.sdslv:24-116) over the ContextRefiner one
// (context_refiner_attention_streaming.sdslv:44-73).  T <= kZImageWitnessMaxTokens.
constexpr int kZImageWitnessMaxTokens = 1056;
hipError_t launch_zimage_attention_witness(const float* Q, const float* Kt, const float* V, const float* O, int T,
                                           int H, float q_scale, bool image_format, float* out, hipStream_t stream);

}  // namespace prom
