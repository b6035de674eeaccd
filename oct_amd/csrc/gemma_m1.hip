// Gemma-4-E2B M1 entry points: input / projection-activation / per-head
// RMSNorm, half-split RoPE, head RMSNorm + RoPE and raw attention scores.
//
// Reference call chain (internal/prometheus/native):
//   reactor_api.c:250-587          public wrappers and their validation
//   reactor_concept_rmsnorm.cpp    weight preparation (:85-108), execution
//                                  checks (:50-70, :110-146), RoPE (:157-189),
//                                  scores (:191-211)
//   reactors/PrometheusRmsNorm.concept:199-213  weight replacement requires a
//                                  strictly newer generation (-7406 otherwise)
//   shaders/sdslv/production/gemma4e2b/{bf16_roundtrip,rope_half_split,
//   attention_scores}.sdslv        the arithmetic of each stage
// The Go witnesses (gemma4e2b_m1_rtx.go:811-883) state the same functions on
// the CPU.
//
// MI355X design: these are 15-token model-private shapes (at most 120 rows of
// 256 channels for the head stages, 1024 x 4096 for the input norm), so each
// stage is one small launch on the runtime stream with all intermediates kept
// in device staging: one wave64 per row for the norms (row sum of squares in
// binary64), one thread per element for RoPE and per score for the scores.
#include <math.h>
#include <string.h>

#include "reactor_internal.h"

namespace prom {
namespace {

constexpr uint32_t kM1Tokens = 15;
constexpr uint32_t kM1HeadWidth = 256;
constexpr uint32_t kM1QueryHeads = 8;
constexpr uint32_t kM1Scores = kM1QueryHeads * kM1Tokens * kM1Tokens;  // 1800
constexpr uint64_t kM46CapacityBytes = (uint64_t)1024 * 4096 * 4;         // tokens x width x fp32

// Round to nearest even at bit 16 (finite inputs; gemma4e2b_m1_rtx.go:1009-1014).
__device__ __forceinline__ float bf16_round(float v) {
  const uint32_t bits = __float_as_uint(v);
  return __uint_as_float((bits + 0x7FFFu + ((bits >> 16) & 1u)) & 0xFFFF0000u);
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One wave64 per row: inv = 1/sqrt(sum(x^2)/W + eps) with the sum in binary64,
// y = x * inv * w; optional BF16 rounding of x before the norm and of y after.
__global__ __launch_bounds__(256) void m1_rmsnorm_kernel(const float* __restrict__ in, int stride,
                                                         const float* __restrict__ w, float* __restrict__ out,
                                                         float* __restrict__ inv_out, int rows, int width, float eps,
                                                         int round_in, int round_out) {
#pragma clang fp contract(off)
  const int row = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* x = in + (size_t)row * stride;
  double acc = 0.0;
  for (int c = lane; c < width; c += 64) {
    const double v = round_in ? bf16_round(x[c]) : x[c];
    acc += v * v;
  }
  acc = wave_sum_f64(acc);
  const float inv = (float)(1.0 / sqrt(acc / (double)width + (double)eps));
  float* y = out + (size_t)row * width;
  for (int c = lane; c < width; c += 64) {
    const float v = round_in ? bf16_round(x[c]) : x[c];
    const float o = v * inv * w[c];
    y[c] = round_out ? bf16_round(o) : o;
  }
  if (inv_out != nullptr && lane == 0) inv_out[row] = inv;
}

// gemma4e2b/rope_half_split.sdslv: element (t, h, c) of [T, H, 256].
__global__ __launch_bounds__(256) void m1_rope_kernel(const float* __restrict__ in, const float* __restrict__ cosine,
                                                      const float* __restrict__ sine, float* __restrict__ out,
                                                      int tokens, int heads) {
#pragma clang fp contract(off)
  const int e = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  const int total = tokens * heads * (int)kM1HeadWidth;
  if (e >= total) return;
  const int half = (int)kM1HeadWidth / 2;
  const int c = e % (int)kM1HeadWidth;
  const int f = c % half;
  const int t = e / (heads * (int)kM1HeadWidth);
  const int pair = c < half ? e + half : e - half;
  const float a = bf16_round(in[e] * cosine[t * (int)kM1HeadWidth + f]);
  const float b = bf16_round(in[pair] * sine[t * (int)kM1HeadWidth + f]);
  out[e] = bf16_round(c < half ? a - b : a + b);
}

// gemma4e2b/attention_scores.sdslv: score (h, i, j) = (sum_c Q[i,h,c] K[j,0,c]) * scale,
// accumulated in fp32 in channel order.
__global__ __launch_bounds__(256) void m1_scores_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                        float* __restrict__ scores, float scale) {
#pragma clang fp contract(off)
  const int s = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (s >= (int)kM1Scores) return;
  const int j = s % (int)kM1Tokens;
  const int row = s / (int)kM1Tokens;
  const int i = row % (int)kM1Tokens;
  const int h = row / (int)kM1Tokens;
  const float* qr = q + ((size_t)i * kM1QueryHeads + h) * kM1HeadWidth;
  const float* kr = k + (size_t)j * kM1HeadWidth;
  float acc = 0.0f;
  for (int c = 0; c < (int)kM1HeadWidth; ++c) acc = acc + qr[c] * kr[c];
  scores[s] = acc * scale;
}

// ---- host helpers -------------------------------------------------------------
bool all_finite(const float* v, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i)
    if (!isfinite(v[i])) return false;
  return true;
}

// reactor_vulkan_common.c:399-418: FNV-1a over each value's bits widened to 8 bytes.
uint64_t hash_float_bits(const float* v, uint64_t n) {
  uint64_t h = 1469598103934665603ull;
  if (v == nullptr && n != 0) return 0;
  for (uint64_t i = 0; i < n; ++i) {
    uint32_t bits;
    memcpy(&bits, v + i, 4);
    const uint64_t value = bits;
    for (int b = 0; b < 8; ++b) {
      h ^= (value >> (b * 8)) & 0xFFu;
      h *= 1099511628211ull;
    }
  }
  return h;
}

// reactor_concept_rmsnorm.cpp:42-49: FNV-1a over the 4 bytes of each value.
uint64_t hash_float_bytes(const float* v, uint64_t n) {
  uint64_t h = 1469598103934665603ull;
  for (uint64_t i = 0; i < n; ++i) {
    uint32_t bits;
    memcpy(&bits, v + i, 4);
    for (int b = 0; b < 4; ++b) {
      h ^= (uint8_t)(bits >> (b * 8));
      h *= 1099511628211ull;
    }
  }
  return h;
}

struct WeightCommit {
  uint32_t stage;
  int32_t detail;
  uint64_t hash, observed, requested;
};

// reactor_concept_rmsnorm.cpp:85-108 + PrometheusRmsNorm.concept:199-213.
int commit_weight(Runtime* rt, const float* values, uint64_t count, uint32_t width, uint64_t generation,
                  WeightCommit* out) {
  *out = WeightCommit{PROM_STAGE_INIT, PROM_M46_DETAIL_INVALID_REQUEST, 0, 0, generation};
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (values == nullptr || width == 0u || width > PROM_M42_MAX_MODEL_WIDTH || generation == 0u || count != width)
    return PROM_ERROR;
  if (!all_finite(values, count)) {
    out->detail = PROM_M46_DETAIL_NONFINITE_INPUT;
    return PROM_ERROR;
  }
  out->hash = hash_float_bytes(values, count);
  if (!rt->available) return PROM_ERROR;
  out->observed = rt->m1_weight_generation;
  if (generation <= rt->m1_weight_generation) {
    out->stage = PROM_STAGE_TRANSFER_IN;
    out->detail = PROM_M46_DETAIL_STALE_WEIGHT_GENERATION;
    return PROM_ERROR;
  }
  rt->m1_weight_generation = generation;
  rt->m1_weight_hash = out->hash;
  rt->m1_weight_width = width;
  out->stage = 0;
  out->detail = 0;
  return PROM_OK;
}

bool upload(void* dst, const void* src, size_t bytes, hipStream_t s) {
  return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s) == hipSuccess;
}

// Device scratch for the head chain: [in | rounded norm | rope | weight | cos | sin]
// (staging slot 0), and a second region for the key chain and scores (slot 1).
struct ChainBuffers {
  float *in, *norm, *rope, *w, *cos, *sin;
};

bool chain_buffers(uint32_t slot, uint32_t rows, ChainBuffers* b) {
  const size_t act = (size_t)rows * kM1HeadWidth;
  const size_t table = (size_t)kM1Tokens * kM1HeadWidth;
  float* base = static_cast<float*>(staging(slot, (3 * act + kM1HeadWidth + 2 * table) * sizeof(float)));
  if (base == nullptr) return false;
  b->in = base;
  b->norm = b->in + act;
  b->rope = b->norm + act;
  b->w = b->rope + act;
  b->cos = b->w + kM1HeadWidth;
  b->sin = b->cos + table;
  return true;
}

// Head RMSNorm (BF16 in and out) then RoPE for tokens x heads rows; the result
// stays in b.rope.
bool enqueue_head_chain(const ChainBuffers& b, const float* input, const float* weight, const float* cosine,
                        const float* sine, uint32_t heads, float eps, hipStream_t s) {
  const uint32_t rows = kM1Tokens * heads;
  const size_t act = (size_t)rows * kM1HeadWidth * sizeof(float);
  const size_t table = (size_t)kM1Tokens * kM1HeadWidth * sizeof(float);
  if (!upload(b.in, input, act, s) || !upload(b.w, weight, kM1HeadWidth * sizeof(float), s) ||
      !upload(b.cos, cosine, table, s) || !upload(b.sin, sine, table, s))
    return false;
  hipLaunchKernelGGL(m1_rmsnorm_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, b.in, (int)kM1HeadWidth, b.w, b.norm,
                     nullptr, (int)rows, (int)kM1HeadWidth, eps, 1, 1);
  const int total = (int)(rows * kM1HeadWidth);
  hipLaunchKernelGGL(m1_rope_kernel, dim3((total + 255) / 256), dim3(256), 0, s, b.norm, b.cos, b.sin, b.rope,
                     (int)kM1Tokens, (int)heads);
  return hipGetLastError() == hipSuccess;
}

// ---- the RMSNorm family (reactor_api.c:250-395) -----------------------------------
int m1_rmsnorm(void* handle, const PrometheusGemma4E2BM1InputRmsNormRequest* r,
               PrometheusGemma4E2BM1InputRmsNormResult* out, int round_in, int round_out) {
  const uint64_t t0 = wall_ns();
  if (r == nullptr || r->struct_size < sizeof(*r) || r->input == nullptr || r->weight == nullptr ||
      r->output == nullptr || r->inv_rms_output == nullptr || r->tokens == 0u || r->model_width == 0u ||
      r->input_row_stride < r->model_width || r->input_generation == 0u || r->weight_generation == 0u ||
      r->exact_source_hash == 0u) {
    out->stage = PROM_STAGE_INIT;
    out->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
    return PROM_ERROR;
  }
  Runtime* rt = lookup(handle);
  WeightCommit wc;
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  if (commit_weight(rt, r->weight, r->weight_element_count, r->model_width, r->weight_generation, &wc) != PROM_OK) {
    out->stage = wc.stage;
    out->detail_code = wc.detail;
    out->weight_hash = wc.hash;
    out->end_to_end_ns = wall_ns() - t0;
    return PROM_ERROR;
  }
  // reactor_concept_rmsnorm.cpp:50-62 (execution admission) and :117-121 (finite input)
  const uint64_t storage = (uint64_t)r->tokens * r->input_row_stride;
  const uint64_t logical = (uint64_t)r->tokens * r->model_width;
  out->stage = 0;
  out->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
  if (r->tokens > PROM_M42_MAX_TOKENS || r->model_width > PROM_M42_MAX_MODEL_WIDTH || !isfinite(r->epsilon) ||
      r->epsilon <= 0.0f || storage != r->input_element_count || storage * sizeof(float) > kM46CapacityBytes ||
      r->output_element_count != logical || r->inv_rms_output_element_count != r->tokens)
    return PROM_ERROR;
  out->input_hash = hash_float_bits(r->input, r->input_element_count);
  if (!all_finite(r->input, storage)) {
    out->detail_code = PROM_M46_DETAIL_NONFINITE_INPUT;
    return PROM_ERROR;
  }
  float* din = static_cast<float*>(staging(0, storage * sizeof(float)));
  float* dw = static_cast<float*>(staging(1, (size_t)r->model_width * sizeof(float)));
  float* dout = static_cast<float*>(staging(2, (logical + r->tokens) * sizeof(float)));
  if (din == nullptr || dw == nullptr || dout == nullptr) {
    out->detail_code = PROM_M46_DETAIL_RESOURCE;
    return PROM_ERROR;
  }
  float* dinv = dout + logical;
  bool ok = upload(din, r->input, storage * sizeof(float), cx.stream) &&
            upload(dw, r->weight, (size_t)r->model_width * sizeof(float), cx.stream) &&
            hipEventRecord(cx.op_begin, cx.stream) == hipSuccess;
  if (ok) {
    hipLaunchKernelGGL(m1_rmsnorm_kernel, dim3((r->tokens + 3) / 4), dim3(256), 0, cx.stream, din,
                       (int)r->input_row_stride, dw, dout, dinv, (int)r->tokens, (int)r->model_width, r->epsilon,
                       round_in, round_out);
    ok = hipGetLastError() == hipSuccess && hipEventRecord(cx.op_end, cx.stream) == hipSuccess &&
         hipMemcpyAsync(r->output, dout, logical * sizeof(float), hipMemcpyDeviceToHost, cx.stream) == hipSuccess &&
         hipMemcpyAsync(r->inv_rms_output, dinv, r->tokens * sizeof(float), hipMemcpyDeviceToHost, cx.stream) ==
             hipSuccess &&
         hipStreamSynchronize(cx.stream) == hipSuccess;
  }
  if (!ok) {
    (void)hipGetLastError();
    out->detail_code = PROM_M46_DETAIL_READBACK;
    return PROM_ERROR;
  }
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, cx.op_begin, cx.op_end) == hipSuccess) out->apply_gpu_ns = (uint64_t)(ms * 1.0e6);
  out->detail_code = 0;
  out->output_written = 1;
  out->matched_input = 1;
  out->weight_hash = rt->m1_weight_hash;
  out->output_hash = hash_float_bits(r->output, logical);
  out->inv_rms_hash = hash_float_bits(r->inv_rms_output, r->tokens);
  out->submit_count = 1;
  out->final_readback_count = 1;
  out->no_product_intermediate_readback_change = 1;
  out->retained_bytes = (uint64_t)r->model_width * sizeof(float);
  out->pipeline_create_count = 1;
  out->end_to_end_ns = wall_ns() - t0;
  rt->successes++;
  return PROM_OK;
}

int rope_status(PrometheusGemma4E2BM1RopeResult* out, int detail) {
  out->detail_code = detail;
  return PROM_ERROR;
}

int head_rmsnorm_rope(void* handle, const PrometheusGemma4E2BM1HeadRmsNormRopeRequest* r,
                      PrometheusGemma4E2BM1HeadRmsNormRopeResult* out, ChainBuffers* keep, uint32_t slot) {
  if (r == nullptr || r->struct_size < sizeof(*r) || r->input == nullptr || r->weight == nullptr ||
      r->cosine == nullptr || r->sine == nullptr || (r->output == nullptr && r->output_element_count != 0u) ||
      r->tokens != kM1Tokens || (r->heads != 1u && r->heads != kM1QueryHeads) || r->head_width != kM1HeadWidth ||
      r->epsilon != 0.000001f || r->input_generation == 0u || r->weight_generation == 0u ||
      r->table_generation == 0u || r->exact_source_hash == 0u) {
    out->stage = PROM_STAGE_INIT;
    out->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
    return PROM_ERROR;
  }
  const uint64_t rows = (uint64_t)r->tokens * r->heads;
  const uint64_t table = (uint64_t)r->tokens * r->head_width;
  if (r->input_element_count != rows * r->head_width || r->weight_element_count != r->head_width ||
      r->cosine_element_count != table || r->sine_element_count != table ||
      (r->output != nullptr && r->output_element_count != r->input_element_count)) {
    out->stage = PROM_STAGE_INIT;
    out->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
    return PROM_ERROR;
  }
  Runtime* rt = lookup(handle);
  WeightCommit wc;
  if (commit_weight(rt, r->weight, r->weight_element_count, r->head_width, r->weight_generation, &wc) != PROM_OK) {
    out->stage = wc.stage;
    out->detail_code = wc.detail;
    out->weight_hash = wc.hash;
    out->observed_weight_generation = wc.observed;
    out->requested_weight_generation = wc.requested;
    return PROM_ERROR;
  }
  out->stage = 0;
  out->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
  out->input_hash = hash_float_bits(r->input, r->input_element_count);
  if (!all_finite(r->input, r->input_element_count) || !all_finite(r->cosine, table) || !all_finite(r->sine, table)) {
    out->detail_code = PROM_M46_DETAIL_NONFINITE_INPUT;
    return PROM_ERROR;
  }
  DeviceContext& cx = ctx();
  ChainBuffers b;
  if (!chain_buffers(slot, (uint32_t)rows, &b)) {
    out->detail_code = PROM_M46_DETAIL_RESOURCE;
    return PROM_ERROR;
  }
  bool ok = enqueue_head_chain(b, r->input, r->weight, r->cosine, r->sine, r->heads, r->epsilon, cx.stream);
  if (ok && r->output != nullptr)
    ok = hipMemcpyAsync(r->output, b.rope, rows * kM1HeadWidth * sizeof(float), hipMemcpyDeviceToHost, cx.stream) ==
         hipSuccess;
  ok = ok && hipStreamSynchronize(cx.stream) == hipSuccess;
  if (!ok) {
    (void)hipGetLastError();
    out->detail_code = PROM_M46_DETAIL_READBACK;
    return PROM_ERROR;
  }
  if (keep != nullptr) *keep = b;
  out->detail_code = 0;
  out->output_written = r->output != nullptr ? 1u : 0u;
  out->dispatch_count = 1;
  out->resident_source_bound = 1;
  out->normalized_readback_count = 0;
  out->source_byte_range = rows * kM1HeadWidth * sizeof(float);
  out->destination_byte_range = out->source_byte_range;
  out->weight_hash = rt->m1_weight_hash;
  out->output_hash = r->output != nullptr ? hash_float_bits(r->output, r->output_element_count) : 1u;
  out->pipeline_create_count = 1;
  out->observed_weight_generation = wc.observed;
  out->requested_weight_generation = wc.requested;
  return PROM_OK;
}

}  // namespace
}  // namespace prom

using namespace prom;

extern "C" {

PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm(
    void* handle, const PrometheusGemma4E2BM1InputRmsNormRequest* request,
    PrometheusGemma4E2BM1InputRmsNormResult* out_result) {
  if (out_result == nullptr) return PROM_ERROR;
  memset(out_result, 0, sizeof(*out_result));
  out_result->struct_size = sizeof(*out_result);
  return m1_rmsnorm(handle, request, out_result, 0, 0);
}

PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_projection_activation_rmsnorm(
    void* handle, const PrometheusGemma4E2BM1InputRmsNormRequest* request,
    PrometheusGemma4E2BM1InputRmsNormResult* out_result) {
  if (out_result == nullptr) return PROM_ERROR;
  memset(out_result, 0, sizeof(*out_result));
  out_result->struct_size = sizeof(*out_result);
  return m1_rmsnorm(handle, request, out_result, 0, 1);
}

PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm(
    void* handle, const PrometheusGemma4E2BM1HeadRmsNormRequest* request,
    PrometheusGemma4E2BM1HeadRmsNormResult* out_result) {
  if (out_result == nullptr) return PROM_ERROR;
  memset(out_result, 0, sizeof(*out_result));
  out_result->struct_size = sizeof(*out_result);
  const PrometheusGemma4E2BM1HeadRmsNormRequest* r = request;
  if (r == nullptr || r->struct_size < sizeof(*r) || r->input == nullptr || r->weight == nullptr ||
      r->output == nullptr || r->inv_rms_output == nullptr || r->tokens == 0u || r->tokens > 120u ||
      r->model_width != kM1HeadWidth || r->input_row_stride != kM1HeadWidth ||
      r->input_element_count != (uint64_t)r->tokens * kM1HeadWidth || r->weight_element_count != kM1HeadWidth ||
      r->output_element_count != (uint64_t)r->tokens * kM1HeadWidth ||
      r->inv_rms_output_element_count != r->tokens || r->epsilon != 0.000001f) {
    out_result->stage = PROM_STAGE_INIT;
    out_result->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
    return PROM_ERROR;
  }
  return m1_rmsnorm(handle, request, out_result, 1, 1);
}

PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_rope(void* handle,
                                                                  const PrometheusGemma4E2BM1RopeRequest* r,
                                                                  PrometheusGemma4E2BM1RopeResult* out) {
  if (out == nullptr) return PROM_ERROR;
  memset(out, 0, sizeof(*out));
  out->struct_size = sizeof(*out);
  out->stage = PROM_STAGE_INIT;
  out->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (r == nullptr || r->struct_size < sizeof(*r) || r->source == nullptr || r->cosine == nullptr ||
      r->sine == nullptr || r->output == nullptr || r->source == r->output || r->cosine == r->output ||
      r->sine == r->output || r->cosine == r->sine || r->tokens != kM1Tokens ||
      (r->heads != 1u && r->heads != kM1QueryHeads) || r->head_width != kM1HeadWidth || r->source_generation == 0u ||
      r->table_generation == 0u || r->source_element_count != (uint64_t)kM1Tokens * r->heads * kM1HeadWidth ||
      r->output_element_count != r->source_element_count || r->cosine_element_count != 3840u ||
      r->sine_element_count != 3840u)
    return PROM_ERROR;
  if (!all_finite(r->source, r->source_element_count) || !all_finite(r->cosine, 3840u) ||
      !all_finite(r->sine, 3840u))
    return rope_status(out, PROM_M46_DETAIL_NONFINITE_INPUT);
  out->source_hash = hash_float_bytes(r->source, r->source_element_count);
  out->cosine_hash = hash_float_bytes(r->cosine, 3840u);
  out->sine_hash = hash_float_bytes(r->sine, 3840u);
  if (!rt->available) return rope_status(out, PROM_M46_DETAIL_RESOURCE);
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  out->stage = 0;
  out->detail_code = 0;
  ChainBuffers b;
  if (!chain_buffers(0, kM1Tokens * r->heads, &b)) {
    out->stage = PROM_STAGE_INIT;
    return rope_status(out, PROM_M46_DETAIL_RESOURCE);
  }
  const size_t act = (size_t)r->source_element_count * sizeof(float);
  bool ok = upload(b.in, r->source, act, cx.stream) && upload(b.cos, r->cosine, 3840u * sizeof(float), cx.stream) &&
            upload(b.sin, r->sine, 3840u * sizeof(float), cx.stream);
  if (ok) {
    const int total = (int)r->source_element_count;
    hipLaunchKernelGGL(m1_rope_kernel, dim3((total + 255) / 256), dim3(256), 0, cx.stream, b.in, b.cos, b.sin, b.rope,
                       (int)kM1Tokens, (int)r->heads);
    ok = hipGetLastError() == hipSuccess &&
         hipMemcpyAsync(r->output, b.rope, act, hipMemcpyDeviceToHost, cx.stream) == hipSuccess &&
         hipStreamSynchronize(cx.stream) == hipSuccess;
  }
  if (!ok) {
    (void)hipGetLastError();
    out->stage = PROM_STAGE_TRANSFER_OUT;
    return rope_status(out, PROM_M46_DETAIL_READBACK);
  }
  out->output_written = 1;
  out->dispatch_count = 1;
  out->pipeline_create_count = 1;
  out->output_hash = hash_float_bytes(r->output, r->output_element_count);
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm_rope(
    void* handle, const PrometheusGemma4E2BM1HeadRmsNormRopeRequest* request,
    PrometheusGemma4E2BM1HeadRmsNormRopeResult* out_result) {
  if (out_result == nullptr) return PROM_ERROR;
  memset(out_result, 0, sizeof(*out_result));
  out_result->struct_size = sizeof(*out_result);
  std::lock_guard<std::mutex> lock(ctx().mu);
  return head_rmsnorm_rope(handle, request, out_result, nullptr, 0);
}

PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_attention_scores(
    void* handle, const PrometheusGemma4E2BM1AttentionScoresRequest* r,
    PrometheusGemma4E2BM1AttentionScoresResult* out) {
  if (out == nullptr) return PROM_ERROR;
  memset(out, 0, sizeof(*out));
  out->struct_size = sizeof(*out);
  const uint64_t q_elems = (uint64_t)kM1Tokens * kM1QueryHeads * kM1HeadWidth;
  const uint64_t k_elems = (uint64_t)kM1Tokens * kM1HeadWidth;
  const uint64_t table = (uint64_t)kM1Tokens * kM1HeadWidth;
  if (r == nullptr || r->struct_size < sizeof(*r) || r->query_input == nullptr || r->key_input == nullptr ||
      r->query_weight == nullptr || r->key_weight == nullptr || r->cosine == nullptr || r->sine == nullptr ||
      r->scores == nullptr || r->tokens != kM1Tokens || r->query_heads != kM1QueryHeads || r->key_heads != 1u ||
      r->head_width != kM1HeadWidth || r->epsilon != 0.000001f || r->scale != 0.0625f ||
      r->preparation_order > 1u || r->query_input_generation == 0u || r->key_input_generation == 0u ||
      r->query_weight_generation == 0u || r->key_weight_generation == 0u || r->table_generation == 0u ||
      r->query_exact_source_hash == 0u || r->key_exact_source_hash == 0u || r->query_input_element_count != q_elems ||
      r->key_input_element_count != k_elems || r->query_weight_element_count != kM1HeadWidth ||
      r->key_weight_element_count != kM1HeadWidth || r->cosine_element_count != table ||
      r->sine_element_count != table || r->score_element_count != kM1Scores) {
    out->stage = PROM_STAGE_INIT;
    out->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
    return PROM_ERROR;
  }
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  PrometheusGemma4E2BM1HeadRmsNormRopeRequest pos{};
  pos.struct_size = sizeof(pos);
  pos.cosine = r->cosine;
  pos.sine = r->sine;
  pos.cosine_element_count = r->cosine_element_count;
  pos.sine_element_count = r->sine_element_count;
  pos.tokens = r->tokens;
  pos.head_width = r->head_width;
  pos.epsilon = r->epsilon;
  pos.table_generation = r->table_generation;
  ChainBuffers qb{}, kb{};
  for (uint32_t step = 0; step < 2; ++step) {
    // reactor_api.c:563-580: order 0 prepares the query first, order 1 the key first.
    const bool key = r->preparation_order == 0u ? step == 1u : step == 0u;
    pos.input = key ? r->key_input : r->query_input;
    pos.weight = key ? r->key_weight : r->query_weight;
    pos.input_element_count = key ? k_elems : q_elems;
    pos.weight_element_count = r->head_width;
    pos.heads = key ? r->key_heads : r->query_heads;
    pos.input_generation = key ? r->key_input_generation : r->query_input_generation;
    pos.weight_generation = key ? r->key_weight_generation : r->query_weight_generation;
    pos.exact_source_hash = key ? r->key_exact_source_hash : r->query_exact_source_hash;
    PrometheusGemma4E2BM1HeadRmsNormRopeResult pr{};
    pr.struct_size = sizeof(pr);
    if (head_rmsnorm_rope(handle, &pos, &pr, key ? &kb : &qb, key ? 1u : 0u) != PROM_OK) {
      out->stage = pr.stage;
      out->detail_code = pr.detail_code;
      out->observed_weight_generation = pr.observed_weight_generation;
      out->requested_weight_generation = pr.requested_weight_generation;
      return PROM_ERROR;
    }
    out->positional_dispatch_count = step + 1;
    out->observed_weight_generation = pr.observed_weight_generation;
    out->requested_weight_generation = pr.requested_weight_generation;
  }
  // Scores into the key chain's free region (after its sine table).
  float* dscores = static_cast<float*>(staging(3, kM1Scores * sizeof(float)));
  if (dscores == nullptr) {
    out->stage = PROM_STAGE_INIT;
    out->detail_code = PROM_M46_DETAIL_RESOURCE;
    return PROM_ERROR;
  }
  hipLaunchKernelGGL(m1_scores_kernel, dim3((kM1Scores + 255) / 256), dim3(256), 0, cx.stream, qb.rope, kb.rope,
                     dscores, r->scale);
  const bool ok = hipGetLastError() == hipSuccess &&
                  hipMemcpyAsync(r->scores, dscores, kM1Scores * sizeof(float), hipMemcpyDeviceToHost, cx.stream) ==
                      hipSuccess &&
                  hipStreamSynchronize(cx.stream) == hipSuccess;
  if (!ok) {
    (void)hipGetLastError();
    out->stage = PROM_STAGE_TRANSFER_OUT;
    out->detail_code = PROM_M46_DETAIL_READBACK;
    return PROM_ERROR;
  }
  out->stage = 0;
  out->detail_code = 0;
  out->score_written = 1;
  out->positional_dispatch_count = 2;
  out->score_dispatch_count = 1;
  out->score_readback_count = 1;
  out->host_detour_count = 0;
  out->query_slot_id = 0x40000001u;
  out->key_slot_id = 0x40000002u;
  out->score_slot_id = 0x40000003u;
  out->query_byte_range = q_elems * sizeof(float);
  out->key_byte_range = k_elems * sizeof(float);
  out->score_byte_range = kM1Scores * sizeof(float);
  out->score_hash = hash_float_bits(r->scores, kM1Scores);
  out->pipeline_create_count = 1;
  return PROM_OK;
}

}  // extern "C"
