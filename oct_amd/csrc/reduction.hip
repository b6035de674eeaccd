// Fused row reductions (sum, max, stable softmax) and RMSNorm on fp32 rows.
//
// Semantics follow the reference's CPU oracles:
//   sum      binary64 accumulation, rounded to float
//            (internal/prometheus/native/reactor_vulkan_fused_reduction.c:1011-1014)
//   max      float comparison `v > m` (same file :1015-1018)
//   softmax  float row max, sum of exp(x - max), out = exp(x - max) / sum (:1019-1028)
//   rmsnorm  inv = 1 / sqrt(sum(x^2)/W + eps), y = x * inv * w, no mean
//            subtraction (reactor_vulkan_gemma4e2b.c:286-319)
//
// MI355X design (the reference's Vulkan path splits a 4096-wide row into
// 1024-element partial workgroups and runs up to 5 dispatches per softmax,
// PrometheusReduction.concept:128-164; here every operation is ONE pass):
//   * one wave64 per row, 4 rows per 256-thread workgroup;
//   * rows up to 4096 floats with width % 4 == 0 stay in registers: each
//     lane holds up to 16 float4 (128-bit loads, fully coalesced), so x is
//     read from HBM exactly once and the output written once;
//   * cross-lane reductions use wave64 shuffles; sums accumulate in binary64
//     per lane (free on a bandwidth-bound kernel and closest to the oracle);
//   * wider or unaligned rows take a streaming variant that re-reads the row
//     (from L2 for rows that fit) with 32- or 128-bit loads.
#include "reactor_internal.h"

namespace prom {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kOpSum = 1, kOpMax = 2, kOpSoftmax = 3, kOpRms = 4;
constexpr float kLog2e = 1.4426950408889634f;

// Hardware base-2 exponential (v_exp_f32).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

// Register-resident path: width % 4 == 0, width <= 256 * kChunks.  kPreW
// (RMSNorm of few rows, where each wave's memory latency is the cost): the
// weight chunks load with the row, before the reduction, instead of after it.
template <uint32_t kOp, int kChunks, bool kPreW = false>
__global__ __launch_bounds__(256) void row_resident_kernel(const float* __restrict__ in, const float* __restrict__ w,
                                                           float* __restrict__ out, float* __restrict__ aux,
                                                           uint32_t rows, uint32_t width, float eps) {
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * 4u + wave;
  if (row >= rows) return;
  const uint32_t w4 = width >> 2;
  const floatx4* src = reinterpret_cast<const floatx4*>(in + (size_t)row * width);
  floatx4 v[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const uint32_t i = (uint32_t)c * 64u + lane;
    if (i < w4) v[c] = src[i];
  }
  if constexpr (kOp == kOpSum) {
    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint32_t i = (uint32_t)c * 64u + lane;
      if (i < w4) acc += ((double)v[c].x + (double)v[c].y) + ((double)v[c].z + (double)v[c].w);
    }
    acc = wave_sum_f64(acc);
    if (lane == 0) out[row] = (float)acc;
  } else if constexpr (kOp == kOpMax) {
    float m = src[0].x;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint32_t i = (uint32_t)c * 64u + lane;
      if (i < w4) {
        m = v[c].x > m ? v[c].x : m;
        m = v[c].y > m ? v[c].y : m;
        m = v[c].z > m ? v[c].z : m;
        m = v[c].w > m ? v[c].w : m;
      }
    }
    m = wave_max_f32(m);
    if (lane == 0) out[row] = m;
  } else if constexpr (kOp == kOpSoftmax) {
    float m = src[0].x;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint32_t i = (uint32_t)c * 64u + lane;
      if (i < w4) {
        m = v[c].x > m ? v[c].x : m;
        m = v[c].y > m ? v[c].y : m;
        m = v[c].z > m ? v[c].z : m;
        m = v[c].w > m ? v[c].w : m;
      }
    }
    m = wave_max_f32(m);
    // exp(x - m) = exp2((x - m) * log2 e) on the hardware exp2; the row sum
    // stays binary64; the normalisation multiplies by one correctly rounded
    // reciprocal.  Relative error per element is a few fp32 ulps.
    // (x - m) is formed first: it is exact when x and m are close, so rows of
    // large nearby values (e.g. 1e4 +- 8) keep full relative accuracy.
    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint32_t i = (uint32_t)c * 64u + lane;
      if (i < w4) {
        v[c].x = exp2_hw((v[c].x - m) * kLog2e);
        v[c].y = exp2_hw((v[c].y - m) * kLog2e);
        v[c].z = exp2_hw((v[c].z - m) * kLog2e);
        v[c].w = exp2_hw((v[c].w - m) * kLog2e);
        acc += ((double)v[c].x + (double)v[c].y) + ((double)v[c].z + (double)v[c].w);
      }
    }
    acc = wave_sum_f64(acc);
    const float rden = (float)(1.0 / acc);
    floatx4* dst = reinterpret_cast<floatx4*>(out + (size_t)row * width);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint32_t i = (uint32_t)c * 64u + lane;
      if (i < w4) {
        floatx4 o;
        o.x = v[c].x * rden;
        o.y = v[c].y * rden;
        o.z = v[c].z * rden;
        o.w = v[c].w * rden;
        dst[i] = o;
      }
    }
  } else {  // RMSNorm
    const floatx4* w4p = reinterpret_cast<const floatx4*>(w);
    floatx4 g[kPreW ? kChunks : 1];
    if constexpr (kPreW) {
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        const uint32_t i = (uint32_t)c * 64u + lane;
        if (i < w4) g[c] = w4p[i];
      }
    }
    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint32_t i = (uint32_t)c * 64u + lane;
      if (i < w4) {
        acc += ((double)(v[c].x * v[c].x) + (double)(v[c].y * v[c].y)) +
               ((double)(v[c].z * v[c].z) + (double)(v[c].w * v[c].w));
      }
    }
    acc = wave_sum_f64(acc);
    const float sumsq = (float)acc;
    const float inv = 1.0f / sqrtf(sumsq / (float)width + eps);
    floatx4* dst = reinterpret_cast<floatx4*>(out + (size_t)row * width);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const uint32_t i = (uint32_t)c * 64u + lane;
      if (i < w4) {
        const floatx4 gc = kPreW ? g[kPreW ? c : 0] : w4p[i];
        floatx4 o;
        o.x = v[c].x * inv * gc.x;
        o.y = v[c].y * inv * gc.y;
        o.z = v[c].z * inv * gc.z;
        o.w = v[c].w * inv * gc.w;
        dst[i] = o;
      }
    }
    if (aux != nullptr && lane == 0) aux[row] = inv;
  }
}

// Streaming path: any width, any alignment; `stride` is the input row pitch
// (elements).  Rows are re-read per phase.
template <uint32_t kOp>
__global__ __launch_bounds__(256) void row_stream_kernel(const float* __restrict__ in, const float* __restrict__ w,
                                                         float* __restrict__ out, float* __restrict__ aux,
                                                         uint32_t rows, uint32_t width, uint32_t stride, float eps) {
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * 4u + wave;
  if (row >= rows) return;
  const float* src = in + (size_t)row * stride;
  if constexpr (kOp == kOpSum) {
    double acc = 0.0;
    for (uint32_t i = lane; i < width; i += 64) acc += (double)src[i];
    acc = wave_sum_f64(acc);
    if (lane == 0) out[row] = (float)acc;
  } else if constexpr (kOp == kOpMax) {
    float m = src[0];
    for (uint32_t i = lane; i < width; i += 64) m = src[i] > m ? src[i] : m;
    m = wave_max_f32(m);
    if (lane == 0) out[row] = m;
  } else if constexpr (kOp == kOpSoftmax) {
    float m = src[0];
    for (uint32_t i = lane; i < width; i += 64) m = src[i] > m ? src[i] : m;
    m = wave_max_f32(m);
    double acc = 0.0;
    for (uint32_t i = lane; i < width; i += 64) acc += (double)expf(src[i] - m);
    acc = wave_sum_f64(acc);
    const float denom = (float)acc;
    float* dst = out + (size_t)row * width;
    for (uint32_t i = lane; i < width; i += 64) dst[i] = expf(src[i] - m) / denom;
  } else {
    double acc = 0.0;
    for (uint32_t i = lane; i < width; i += 64) acc += (double)(src[i] * src[i]);
    acc = wave_sum_f64(acc);
    const float sumsq = (float)acc;
    const float inv = 1.0f / sqrtf(sumsq / (float)width + eps);
    float* dst = out + (size_t)row * width;
    for (uint32_t i = lane; i < width; i += 64) dst[i] = src[i] * inv * w[i];
    if (aux != nullptr && lane == 0) aux[row] = inv;
  }
}

template <uint32_t kOp>
hipError_t dispatch(const float* in, const float* w, float* out, float* aux, uint32_t rows, uint32_t width,
                    uint32_t stride, float eps, hipStream_t stream) {
  const dim3 grid((rows + 3u) / 4u);
  const dim3 block(256);
  const bool resident = (width % 4u == 0u) && (stride == width) && ((reinterpret_cast<uintptr_t>(in) & 15u) == 0) &&
                        ((reinterpret_cast<uintptr_t>(out) & 15u) == 0) &&
                        (w == nullptr || (reinterpret_cast<uintptr_t>(w) & 15u) == 0);
  if (resident && width <= 256u * 4u) {
    hipLaunchKernelGGL((row_resident_kernel<kOp, 4>), grid, block, 0, stream, in, w, out, aux, rows, width, eps);
  } else if (resident && width <= 256u * 16u) {
    // Few rows (a transformer layer's tokens): one wave per row leaves the
    // chip mostly idle, so each wave's latency is the cost; preload the weights.
    if (kOp == kOpRms && rows <= 2048u && width <= 256u * 8u)
      hipLaunchKernelGGL((row_resident_kernel<kOp, 8, true>), grid, block, 0, stream, in, w, out, aux, rows, width,
                         eps);
    else
      hipLaunchKernelGGL((row_resident_kernel<kOp, 16>), grid, block, 0, stream, in, w, out, aux, rows, width, eps);
  } else {
    hipLaunchKernelGGL((row_stream_kernel<kOp>), grid, block, 0, stream, in, w, out, aux, rows, width, stride, eps);
  }
  return hipGetLastError();
}

// The benchmark entry's correctness reference: the same reduction with every
// sum, exponential and quotient in binary64 (one workgroup per row, a
// strided lane pass then an LDS tree), rounded to float at the end.  It shares
// no code with the fp32 kernels above.
__global__ __launch_bounds__(256) void row_reduction_check_kernel(const float* __restrict__ in,
                                                                  float* __restrict__ out, uint32_t width,
                                                                  uint32_t op) {
  __shared__ double part[256];
  const uint32_t lane = threadIdx.x;
  const float* x = in + (size_t)blockIdx.x * width;
  float m = -__builtin_inff();
  if (op != kOpSum) {
    for (uint32_t i = lane; i < width; i += 256) m = x[i] > m ? x[i] : m;
    part[lane] = (double)m;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
      if (lane < s && part[lane + s] > part[lane]) part[lane] = part[lane + s];
      __syncthreads();
    }
    m = (float)part[0];
    __syncthreads();
    if (op == kOpMax) {
      if (lane == 0) out[blockIdx.x] = m;
      return;
    }
  }
  double acc = 0.0;
  for (uint32_t i = lane; i < width; i += 256) acc += op == kOpSum ? (double)x[i] : exp((double)x[i] - (double)m);
  part[lane] = acc;
  __syncthreads();
  for (uint32_t s = 128; s > 0; s >>= 1) {
    if (lane < s) part[lane] += part[lane + s];
    __syncthreads();
  }
  const double total = part[0];
  if (op == kOpSum) {
    if (lane == 0) out[blockIdx.x] = (float)total;
    return;
  }
  for (uint32_t i = lane; i < width; i += 256)
    out[(size_t)blockIdx.x * width + i] = (float)(exp((double)x[i] - (double)m) / total);
}

}  // namespace

hipError_t launch_row_reduction_check(const float* in, float* out, uint32_t rows, uint32_t width, uint32_t op,
                                      hipStream_t stream) {
  if (rows == 0 || width == 0 || op < kOpSum || op > kOpSoftmax) return hipErrorInvalidValue;
  hipLaunchKernelGGL(row_reduction_check_kernel, dim3(rows), dim3(256), 0, stream, in, out, width, op);
  return hipGetLastError();
}

hipError_t launch_row_reduction(const float* in, float* out, uint32_t rows, uint32_t width, uint32_t op,
                                hipStream_t stream) {
  switch (op) {
    case kOpSum: return dispatch<kOpSum>(in, nullptr, out, nullptr, rows, width, width, 0.f, stream);
    case kOpMax: return dispatch<kOpMax>(in, nullptr, out, nullptr, rows, width, width, 0.f, stream);
    case kOpSoftmax: return dispatch<kOpSoftmax>(in, nullptr, out, nullptr, rows, width, width, 0.f, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rmsnorm(const float* in, const float* w, float* out, float* inv_rms, uint32_t tokens,
                          uint32_t width, uint32_t stride, float eps, hipStream_t stream) {
  return dispatch<kOpRms>(in, w, out, inv_rms, tokens, width, stride, eps, stream);
}

}  // namespace prom
