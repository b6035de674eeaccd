// Gemma-style fp32 decoder layer (T=512, width 2048, FFN 16384) on one HIP stream.
//
// The reference has no Gemma-2B layer; its Gemma-4-E2B pieces fix
// the conventions used here: RMSNorm y = x*inv*w with no mean subtraction
// (reactor_vulkan_gemma4e2b.c:286-319), half-split RoPE pairing
// (gemma4e2b_m1_rtx.go:834-861), multi-query scores with every query head on
// KV head 0 and scale 1/sqrt(head_dim) = 0.0625 (gemma4e2b_m1_rtx.go:863-883).
// GeGLU uses the tanh-approximate GELU Gemma uses; the causal mask is textbook.
//
// MI355X design: every matrix product is the fp32 MFMA SGEMM
// (sgemm_f32.hip) on row-major operands with strides:
//   1 RMSNorm                       x -> n1                        (reduction.hip)
//   2 QKV projection, fused         n1 @ Wqkv -> qkv [T, (Hq+2)d], or its K-split
//                                   slices left unreduced
//   3 RoPE + split                  qkv (or the slices, added in slice order) ->
//                                   Q [T, Hq*d] (scaled by 1/sqrt d, exact
//                                   power of two), K^T [d, T], V [T, d]
//   4 causal flash attention        Q, K^T, V -> O [T, Hq*d] (attention_f32.hip:
//     the query heads of a workgroup share each K/V tile; no score matrix;
//     the key range is split over the grid at T = 512, then combined).  For
//     head dims other than 64/128/256: scores as one GEMM [T*Hq, d] @ K^T ->
//     S [T*Hq, T], a causal softmax over row (t, h)'s keys 0..t, and P @ V
//   7 output projection + residual  x + O @ Wo -> h   (residual fused in the epilogue)
//   8 RMSNorm                       h -> n2
//   9 gate|up projection, fused     n2 @ Wgu -> G [T, 2F]
//  10 GeGLU                         gelu_tanh(G[:, :F]) * G[:, F:] -> A [T, F]
//  11 down projection + residual    h + A @ Wdown -> out
#include <math.h>
#include <algorithm>
#include <string.h>

#include "reactor_internal.h"

namespace prom {
namespace {

// qkv [T, ldq]: Q heads at column h*d, K at Hq*d, V at (Hq+1)*d.
// K^T rows are ldkt (>= T) apart.
__global__ __launch_bounds__(256) void gemma_rope_split_kernel(const float* __restrict__ qkv, int ldq, int T, int Hq,
                                                               int d, int pos0, float base, float q_scale,
                                                               float* __restrict__ Q, float* __restrict__ Kt,
                                                               int ldkt, float* __restrict__ V) {
  const int half = d >> 1;
  const int idx = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (idx < T * half) {
    const int t = idx / half;
    const int i = idx - t * half;
    // angle = position * base^(-2i/d), evaluated in binary64 then rounded.
    const double inv_freq = pow((double)base, -2.0 * (double)i / (double)d);
    const double angle = (double)(pos0 + t) * inv_freq;
    const float c = (float)cos(angle);
    const float s = (float)sin(angle);
    const float* row = qkv + (size_t)t * ldq;
    for (int h = 0; h < Hq; ++h) {
      const float x1 = row[h * d + i];
      const float x2 = row[h * d + i + half];
      Q[(size_t)t * Hq * d + h * d + i] = (x1 * c - x2 * s) * q_scale;
      Q[(size_t)t * Hq * d + h * d + i + half] = (x2 * c + x1 * s) * q_scale;
    }
    const float k1 = row[Hq * d + i];
    const float k2 = row[Hq * d + i + half];
    Kt[(size_t)i * ldkt + t] = k1 * c - k2 * s;
    Kt[(size_t)(i + half) * ldkt + t] = k2 * c + k1 * s;
  }
  if (idx < T * d) {
    const int t = idx / d;
    const int j = idx - t * d;
    V[(size_t)t * d + j] = qkv[(size_t)t * ldq + (Hq + 1) * d + j];
  }
}

// The same split, one token per workgroup, reading the QKV projection as
// `slices` K-split slices `slab` floats apart (1: the reduced product) and
// adding them in slice order, as the split-K reduce does.  The token's
// angles are evaluated once into LDS (half * 8 bytes).
constexpr int kRopeMaxSlices = 4;

__device__ __forceinline__ float add_slices(const float* __restrict__ P, size_t off, int slices, size_t slab) {
  float p[kRopeMaxSlices];
#pragma unroll
  for (int z = 0; z < kRopeMaxSlices; ++z) p[z] = z < slices ? P[z * slab + off] : 0.0f;
  float v = p[0];
#pragma unroll
  for (int z = 1; z < kRopeMaxSlices; ++z)
    if (z < slices) v += p[z];
  return v;
}

__global__ __launch_bounds__(256) void qkv_rope_split_kernel(const float* __restrict__ P, int ldq, int slices,
                                                             size_t slab, int Hq, int d, int pos0, float base,
                                                             float q_scale, float* __restrict__ Q,
                                                             float* __restrict__ Kt, int ldkt, float* __restrict__ V) {
  extern __shared__ float2 rope_cs[];  // [half] (cos, sin) of this token
  const int half = d >> 1;
  const int t = (int)blockIdx.x;
  const int tid = (int)threadIdx.x;
  for (int i = tid; i < half; i += 256) {
    // angle = position * base^(-2i/d), evaluated in binary64 then rounded.
    const double inv_freq = pow((double)base, -2.0 * (double)i / (double)d);
    const double angle = (double)(pos0 + t) * inv_freq;
    rope_cs[i] = make_float2((float)cos(angle), (float)sin(angle));
  }
  const float* row = P + (size_t)t * ldq;
  // V and the K pairs need no angle: load them before the barrier.
  for (int j = tid; j < d; j += 256) V[(size_t)t * d + j] = add_slices(row, (size_t)(Hq + 1) * d + j, slices, slab);
  __syncthreads();
  for (int i = tid; i < half; i += 256) {
    const float k1 = add_slices(row, (size_t)Hq * d + i, slices, slab);
    const float k2 = add_slices(row, (size_t)Hq * d + i + half, slices, slab);
    const float c = rope_cs[i].x, sn = rope_cs[i].y;
    Kt[(size_t)i * ldkt + t] = k1 * c - k2 * sn;
    Kt[(size_t)(i + half) * ldkt + t] = k2 * c + k1 * sn;
  }
  // Q: the pairs (i, i + half) of every head, four per thread per pass.
  const int qpairs = Hq * half;
  float* qrow = Q + (size_t)t * Hq * d;
  for (int e0 = tid; e0 < qpairs; e0 += 4 * 256) {
    float x1[4], x2[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = min(e0 + 256 * u, qpairs - 1);
      const int h = e / half;
      const size_t col = (size_t)h * d + (e - h * half);
      x1[u] = add_slices(row, col, slices, slab);
      x2[u] = add_slices(row, col + half, slices, slab);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = e0 + 256 * u;
      if (e >= qpairs) break;
      const int h = e / half;
      const int i = e - h * half;
      const float c = rope_cs[i].x, sn = rope_cs[i].y;
      qrow[h * d + i] = (x1[u] * c - x2[u] * sn) * q_scale;
      qrow[h * d + i + half] = (x2[u] * c + x1[u] * sn) * q_scale;
    }
  }
}

// Row r of S [rows, width] belongs to query token t = r / heads_per_token at
// position t; it keeps columns 0..t and zeroes the rest.  Stable softmax with
// expf and a binary64 row sum, as the fused softmax kernel.
__global__ __launch_bounds__(256) void causal_softmax_kernel(float* __restrict__ S, int rows, int width,
                                                             int heads_per_token) {
  const int wave = (int)(threadIdx.x >> 6);
  const int lane = (int)(threadIdx.x & 63);
  const int r = (int)blockIdx.x * 4 + wave;
  if (r >= rows) return;
  float* row = S + (size_t)r * width;
  const int valid = min(width, r / heads_per_token + 1);
  float m = row[0];
  for (int j = lane; j < valid; j += 64) m = row[j] > m ? row[j] : m;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(m, off, 64);
    m = o > m ? o : m;
  }
  double sum = 0.0;
  for (int j = lane; j < valid; j += 64) sum += (double)expf(row[j] - m);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  const float denom = (float)sum;
  for (int j = lane; j < width; j += 64) row[j] = j < valid ? expf(row[j] - m) / denom : 0.0f;
}

// G [T, 2F] (gate | up) -> A [T, F]
__global__ __launch_bounds__(256) void geglu_kernel(const float* __restrict__ G, float* __restrict__ A, int T, int F) {
  const size_t total = (size_t)T * F;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
    const size_t t = idx / F;
    const size_t i = idx - t * F;
    const float g = G[t * 2 * F + i];
    const float u = G[t * 2 * F + F + i];
    A[idx] = gelu_tanh(g) * u;
  }
}

// The same with 16-byte accesses (F % 4 == 0, G and A 16-byte aligned): row
// t = blockIdx.y, four columns per thread, no per-element index division.
__global__ __launch_bounds__(256) void geglu_vec_kernel(const float4* __restrict__ G, float4* __restrict__ A, int F4) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= F4) return;
  const size_t t = blockIdx.y;
  const float4 g = G[t * 2 * F4 + i];
  const float4 u = G[t * 2 * F4 + F4 + i];
  A[t * F4 + i] = make_float4(gelu_tanh(g.x) * u.x, gelu_tanh(g.y) * u.y, gelu_tanh(g.z) * u.z, gelu_tanh(g.w) * u.w);
}

struct LayerShape {
  int T, D, Hq, d, F, nqkv;
  int ldkt() const { return (T + 3) & ~3; }  // K^T row stride: 16-byte rows for the attention's tile transfers
};

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

// The RoPE split's LDS (one token's angles) fits.
bool rope_fused(const LayerShape& s) { return (size_t)s.d / 2 * sizeof(float2) <= 32768; }

// Workspace layout: n1 [T,D] | qkv [T,nqkv] | Q [T,Hq*d] | Kt [d,ldkt] | V [T,d]
// | attention partials (or S [T*Hq,T]) | O [T,Hq*d] | h [T,D] | n2 [T,D] | G [T,2F] | A [T,F]
size_t layer_workspace_bytes(const LayerShape& s, size_t offsets[11]) {
  // Slot 5: the key-split partials of the flash attention (often none), or
  // the [T*Hq, T] score matrix of the unfused path for other head dims.
  // The QKV projection's unreduced K-split slices live here first: the RoPE
  // split consumes them before the attention writes its partials.
  size_t attn_bytes = flash_attn_f32_supported(s.d) ? flash_attn_f32_partial_bytes(s.T, s.Hq, s.Hq, s.d, 1)
                                                    : (size_t)s.T * s.Hq * s.T * sizeof(float);
  if (rope_fused(s)) {
    const int slices = sgemm_f32_unreduced_slices(s.D, s.nqkv, s.T, s.nqkv, s.D, kRopeMaxSlices);
    if (slices > 1) attn_bytes = std::max(attn_bytes, (size_t)slices * s.T * s.nqkv * sizeof(float));
  }
  const size_t sizes[11] = {(size_t)s.T * s.D * 4,        (size_t)s.T * s.nqkv * 4, (size_t)s.T * s.Hq * s.d * 4,
                            (size_t)s.d * s.ldkt() * 4,   (size_t)s.T * s.d * 4,    attn_bytes,
                            (size_t)s.T * s.Hq * s.d * 4, (size_t)s.T * s.D * 4,    (size_t)s.T * s.D * 4,
                            (size_t)s.T * 2 * s.F * 4,    (size_t)s.T * s.F * 4};
  size_t off = 0;
  for (int i = 0; i < 11; ++i) {
    offsets[i] = off;
    off += align_up(sizes[i]);
  }
  return off;
}

int32_t validate_layer(const PrometheusDecoderLayerF32Request* r) {
  if (r == nullptr || r->struct_size < sizeof(*r)) return PROM_BLOCK_DETAIL_INVALID_REQUEST;
  if (!r->input || !r->attn_norm_weight || !r->w_qkv || !r->w_o || !r->ffn_norm_weight || !r->w_gate_up ||
      !r->w_down || !r->output)
    return PROM_BLOCK_DETAIL_INVALID_REQUEST;
  if (r->tokens == 0 || r->hidden == 0 || r->q_heads == 0 || r->head_dim == 0 || r->ffn_hidden == 0 ||
      (r->head_dim & 1u) != 0)
    return PROM_BLOCK_DETAIL_SHAPE;
  if (r->kv_heads != 1) return PROM_BLOCK_DETAIL_UNSUPPORTED;
  if (!isfinite(r->rms_epsilon) || r->rms_epsilon <= 0.f || !isfinite(r->rope_base) || r->rope_base <= 0.f)
    return PROM_BLOCK_DETAIL_INVALID_REQUEST;
  const uint64_t lim = 1ull << 31;
  if ((uint64_t)r->tokens * r->q_heads * r->tokens >= lim || (uint64_t)r->tokens * 2 * r->ffn_hidden >= lim ||
      (uint64_t)r->hidden * 2 * r->ffn_hidden >= lim || (uint64_t)r->tokens * r->hidden >= lim)
    return PROM_BLOCK_DETAIL_SHAPE;
  return 0;
}

// Enqueues the whole layer; all pointers are device pointers.
hipError_t enqueue_layer(const PrometheusDecoderLayerF32Request* r, char* ws, const size_t off[11], hipStream_t st,
                         uint32_t* launches) {
  const LayerShape s{(int)r->tokens, (int)r->hidden, (int)r->q_heads, (int)r->head_dim, (int)r->ffn_hidden,
                     (int)((r->q_heads + 2) * r->head_dim)};
  float* n1 = reinterpret_cast<float*>(ws + off[0]);
  float* qkv = reinterpret_cast<float*>(ws + off[1]);
  float* Q = reinterpret_cast<float*>(ws + off[2]);
  float* Kt = reinterpret_cast<float*>(ws + off[3]);
  float* V = reinterpret_cast<float*>(ws + off[4]);
  float* S = reinterpret_cast<float*>(ws + off[5]);
  float* O = reinterpret_cast<float*>(ws + off[6]);
  float* h = reinterpret_cast<float*>(ws + off[7]);
  float* n2 = reinterpret_cast<float*>(ws + off[8]);
  float* G = reinterpret_cast<float*>(ws + off[9]);
  float* A = reinterpret_cast<float*>(ws + off[10]);
  hipError_t e;
  uint32_t n = 0;
#define PROM_STEP(call)             \
  do {                              \
    e = (call);                     \
    if (e != hipSuccess) return e;  \
    ++n;                            \
  } while (0)
  PROM_STEP(launch_rmsnorm(r->input, r->attn_norm_weight, n1, nullptr, s.T, s.D, s.D, r->rms_epsilon, st));
  const float q_scale = 1.0f / sqrtf((float)s.d);
  if (rope_fused(s)) {
    // The QKV projection's K-split slices (if any) go to slot 5 unreduced and
    // the RoPE split adds them: one launch and one [T, nqkv] round trip fewer.
    int slices = 1;
    const size_t slot5 = off[6] - off[5];
    PROM_STEP(launch_sgemm_f32_unreduced(n1, s.D, r->w_qkv, s.nqkv, qkv, s.nqkv, s.T, s.nqkv, s.D, S,
                                         slot5 / sizeof(float), kRopeMaxSlices, st, &slices));
    const float* src = slices > 1 ? S : qkv;
    hipLaunchKernelGGL(qkv_rope_split_kernel, dim3(s.T), dim3(256), (size_t)s.d / 2 * sizeof(float2), st, src,
                       s.nqkv, slices, (size_t)s.T * s.nqkv, s.Hq, s.d, (int)r->position_offset, r->rope_base,
                       q_scale, Q, Kt, s.ldkt(), V);
    PROM_STEP(hipGetLastError());
  } else {
    PROM_STEP(launch_sgemm_f32_ex(n1, s.D, r->w_qkv, s.nqkv, qkv, s.nqkv, s.T, s.nqkv, s.D, nullptr, 0, st, nullptr));
    const int threads = s.T * s.d;  // covers T*d/2 rope pairs and T*d V elements
    hipLaunchKernelGGL(gemma_rope_split_kernel, dim3((threads + 255) / 256), dim3(256), 0, st, qkv, s.nqkv, s.T, s.Hq,
                       s.d, (int)r->position_offset, r->rope_base, q_scale, Q, Kt, s.ldkt(), V);
    PROM_STEP(hipGetLastError());
  }
  if (flash_attn_f32_supported(s.d)) {
    // Causal flash attention, every query head on the one K/V head; S holds
    // only the key-split partials (no score matrix).
    AttnF32Params ap{};
    ap.q = Q;
    ap.kt = Kt;
    ap.v = V;
    ap.o = O;
    ap.q_hs = s.d;
    ap.q_rs = s.Hq * s.d;
    ap.kt_hs = 0;
    ap.kt_rs = s.ldkt();
    ap.v_hs = 0;
    ap.v_rs = s.d;
    ap.o_rs = s.Hq * s.d;
    ap.T = s.T;
    ap.q_heads = s.Hq;
    ap.group = s.Hq;
    ap.causal = 1;
    flash_attn_f32_bind_partials(ap, s.d, S);
    PROM_STEP(launch_flash_attn_f32(ap, s.d, 1.0f, st));
  } else {
    PROM_STEP(launch_sgemm_f32_ex(Q, s.d, Kt, s.ldkt(), S, s.T, s.T * s.Hq, s.T, s.d, nullptr, 0, st, nullptr));
    hipLaunchKernelGGL(causal_softmax_kernel, dim3((s.T * s.Hq + 3) / 4), dim3(256), 0, st, S, s.T * s.Hq, s.T,
                       s.Hq);
    PROM_STEP(hipGetLastError());
    PROM_STEP(launch_sgemm_f32_ex(S, s.T, V, s.d, O, s.d, s.T * s.Hq, s.d, s.T, nullptr, 0, st, nullptr));
  }
  PROM_STEP(launch_sgemm_f32_ex(O, s.Hq * s.d, r->w_o, s.D, h, s.D, s.T, s.D, s.Hq * s.d, r->input, s.D, st, nullptr));
  PROM_STEP(launch_rmsnorm(h, r->ffn_norm_weight, n2, nullptr, s.T, s.D, s.D, r->rms_epsilon, st));
  // gate|up with GeGLU in the GEMM's epilogue (the [T, 2F] intermediate is
  // never written); shapes the fused kernel does not take run the GEMM and
  // the elementwise GeGLU.
  e = launch_sgemm_f32_geglu(n2, s.D, r->w_gate_up, A, s.F, s.T, s.F, s.D, st);
  const bool fused = e == hipSuccess;
  if (fused) {
    ++n;
  } else if (e != hipErrorNotSupported) {
    return e;
  } else {
    PROM_STEP(launch_sgemm_f32_ex(n2, s.D, r->w_gate_up, 2 * s.F, G, 2 * s.F, s.T, 2 * s.F, s.D, nullptr, 0, st,
                                  nullptr));
  }
  if (fused) {
    // the GeGLU ran in the GEMM's epilogue
  } else if (s.F % 4 == 0 && ((reinterpret_cast<uintptr_t>(G) | reinterpret_cast<uintptr_t>(A)) & 15) == 0 && s.T <= 65535) {
    const int f4 = s.F / 4;
    hipLaunchKernelGGL(geglu_vec_kernel, dim3((unsigned)((f4 + 255) / 256), (unsigned)s.T), dim3(256), 0, st,
                       reinterpret_cast<const float4*>(G), reinterpret_cast<float4*>(A), f4);
    PROM_STEP(hipGetLastError());
  } else {
    const size_t total = (size_t)s.T * s.F;
    const unsigned blocks = (unsigned)min((size_t)65536, (total + 255) / 256);
    hipLaunchKernelGGL(geglu_kernel, dim3(blocks), dim3(256), 0, st, G, A, s.T, s.F);
    PROM_STEP(hipGetLastError());
  }
  PROM_STEP(launch_sgemm_f32_ex(A, s.F, r->w_down, s.D, r->output, s.D, s.T, s.D, s.F, h, s.D, st, nullptr));
#undef PROM_STEP
  if (launches) *launches = n;
  return hipSuccess;
}

LayerShape shape_of(const PrometheusDecoderLayerF32Request* r) {
  return LayerShape{(int)r->tokens, (int)r->hidden, (int)r->q_heads, (int)r->head_dim, (int)r->ffn_hidden,
                    (int)((r->q_heads + 2) * r->head_dim)};
}

void result_init(PrometheusBlockResult* res) {
  memset(res, 0, sizeof(*res));
  res->struct_size = sizeof(*res);
}

}  // namespace
}  // namespace prom

using namespace prom;

extern "C" {

PROM_REACTOR_API int prometheus_reactor_runtime_decoder_layer_f32_device(
    void* handle, const PrometheusDecoderLayerF32Request* request, PrometheusBlockResult* out_result) {
  PrometheusBlockResult local;
  PrometheusBlockResult* res = out_result ? out_result : &local;
  result_init(res);
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    res->stage = PROM_STAGE_INIT;
    res->detail_code = PROM_INVALID_HANDLE;
    return PROM_INVALID_HANDLE;
  }
  const int32_t d = validate_layer(request);
  if (d != 0) {
    res->stage = PROM_STAGE_INIT;
    res->detail_code = d;
    return PROM_ERROR;
  }
  if (!rt->available) {
    res->stage = PROM_STAGE_INIT;
    res->detail_code = rt->init_detail;
    return PROM_ERROR;
  }
  size_t off[11];
  const size_t ws_bytes = layer_workspace_bytes(shape_of(request), off);
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  char* ws = static_cast<char*>(staging(4, ws_bytes));
  if (ws == nullptr) {
    res->stage = PROM_STAGE_INIT;
    res->detail_code = PROM_DETAIL_HIP_ALLOC_FAILED;
    return PROM_ERROR;
  }
  res->workspace_bytes = ws_bytes;
  uint32_t launches = 0;
  if (enqueue_layer(request, ws, off, cx.stream, &launches) != hipSuccess) {
    res->stage = PROM_STAGE_SUBMIT;
    res->detail_code = PROM_DETAIL_HIP_LAUNCH_FAILED;
    return PROM_ERROR;
  }
  res->kernel_launches = launches;
  res->stage = PROM_STAGE_SUBMIT;
  res->detail_code = PROM_DETAIL_PATH_HIP_MFMA_F32;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_decoder_layer_f32(void* handle,
                                                                  const PrometheusDecoderLayerF32Request* request,
                                                                  PrometheusBlockResult* out_result) {
  PrometheusBlockResult local;
  PrometheusBlockResult* res = out_result ? out_result : &local;
  result_init(res);
  const uint64_t t0 = wall_ns();
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    res->stage = PROM_STAGE_INIT;
    res->detail_code = PROM_INVALID_HANDLE;
    return PROM_INVALID_HANDLE;
  }
  const int32_t d = validate_layer(request);
  if (d != 0) {
    res->stage = PROM_STAGE_INIT;
    res->detail_code = d;
    return PROM_ERROR;
  }
  if (!rt->available) {
    res->stage = PROM_STAGE_INIT;
    res->detail_code = rt->init_detail;
    return PROM_ERROR;
  }
  const PrometheusDecoderLayerF32Request& r = *request;
  const LayerShape s = shape_of(request);
  // Device copies of every host array, packed into one staging buffer.
  const size_t sizes[8] = {(size_t)s.T * s.D, (size_t)s.D, (size_t)s.D * s.nqkv, (size_t)s.Hq * s.d * s.D,
                           (size_t)s.D,       (size_t)s.D * 2 * s.F, (size_t)s.F * s.D, (size_t)s.T * s.D};
  const float* srcs[7] = {r.input, r.attn_norm_weight, r.w_qkv, r.w_o, r.ffn_norm_weight, r.w_gate_up, r.w_down};
  size_t offs[8], total = 0;
  for (int i = 0; i < 8; ++i) {
    offs[i] = total;
    total += align_up(sizes[i] * sizeof(float));
  }
  size_t woff[11];
  const size_t ws_bytes = layer_workspace_bytes(s, woff);
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  char* dev = static_cast<char*>(staging(5, total));
  char* ws = static_cast<char*>(staging(4, ws_bytes));
  if (dev == nullptr || ws == nullptr) {
    res->stage = PROM_STAGE_TRANSFER_IN;
    res->detail_code = PROM_DETAIL_HIP_ALLOC_FAILED;
    return PROM_ERROR;
  }
  res->stage = PROM_STAGE_TRANSFER_IN;
  for (int i = 0; i < 7; ++i) {
    if (upload_host(dev + offs[i], srcs[i], sizes[i] * sizeof(float), cx.stream) != hipSuccess) {
      res->detail_code = PROM_DETAIL_HIP_COPY_FAILED;
      return PROM_ERROR;
    }
  }
  PrometheusDecoderLayerF32Request dr = r;
  dr.input = reinterpret_cast<const float*>(dev + offs[0]);
  dr.attn_norm_weight = reinterpret_cast<const float*>(dev + offs[1]);
  dr.w_qkv = reinterpret_cast<const float*>(dev + offs[2]);
  dr.w_o = reinterpret_cast<const float*>(dev + offs[3]);
  dr.ffn_norm_weight = reinterpret_cast<const float*>(dev + offs[4]);
  dr.w_gate_up = reinterpret_cast<const float*>(dev + offs[5]);
  dr.w_down = reinterpret_cast<const float*>(dev + offs[6]);
  dr.output = reinterpret_cast<float*>(dev + offs[7]);
  res->stage = PROM_STAGE_SUBMIT;
  uint32_t launches = 0;
  (void)hipEventRecord(cx.op_begin, cx.stream);
  if (enqueue_layer(&dr, ws, woff, cx.stream, &launches) != hipSuccess) {
    (void)hipStreamSynchronize(cx.stream);
    res->detail_code = PROM_DETAIL_HIP_LAUNCH_FAILED;
    return PROM_ERROR;
  }
  (void)hipEventRecord(cx.op_end, cx.stream);
  res->stage = PROM_STAGE_TRANSFER_OUT;
  if (download_host(r.output, dr.output, sizes[7] * sizeof(float), cx.stream) != hipSuccess ||
      hipStreamSynchronize(cx.stream) != hipSuccess) {
    res->detail_code = PROM_DETAIL_HIP_COPY_FAILED;
    return PROM_ERROR;
  }
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, cx.op_begin, cx.op_end) == hipSuccess) res->gpu_duration_ns = (uint64_t)(ms * 1.0e6);
  res->kernel_launches = launches;
  res->workspace_bytes = ws_bytes;
  res->detail_code = PROM_DETAIL_PATH_HIP_MFMA_F32;
  res->output_written = 1;
  res->end_to_end_ns = wall_ns() - t0;
  return PROM_OK;
}

}  // extern "C"
