// Fused per-row kernels of the Z-Image transformer block, shared by the bf16
// DiT block (dit_block.hip) and the fp32 resident Z-Image blocks
// (zimage_f32.hip).  Stage definitions follow the reference's canonical block
// (internal/prometheus/zimage/canonical_reference.go:177-210, 373-480) and its
// unmodulated ContextRefiner (context_refiner_reference.go:230-311):
//   RMSNorm   y = x * (1 / sqrt(sum(x^2)/D + eps)) * w, no mean subtraction
//   modulate  y * scale          (scale = 1 + adaLN chunk; absent => 1)
//   gated add r + gate * y       (gate = tanh(adaLN chunk); absent => 1)
//
// One wave64 per row, 4 rows per 256-thread workgroup; rows up to
// 16 * 64 * 4 = 4096 floats (D % 4 == 0) stay in registers, so every input
// row is read from HBM once and every output written once with 128-bit
// accesses.  OutT selects the store format: float, or uint16_t for bf16
// (round to nearest even).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prom {
namespace {  // each translation unit gets its own copy of these kernels
namespace rows {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kRowChunks = 16;

__device__ __forceinline__ uint16_t f2bf(float v) {
  const uint32_t bits = __float_as_uint(v);
  return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ void store4(float* dst, floatx4 v) { *reinterpret_cast<floatx4*>(dst) = v; }

__device__ __forceinline__ void store4(uint16_t* dst, floatx4 v) {
  u32x2 w;
  w.x = (uint32_t)f2bf(v.x) | ((uint32_t)f2bf(v.y) << 16);
  w.y = (uint32_t)f2bf(v.z) | ((uint32_t)f2bf(v.w) << 16);
  *reinterpret_cast<u32x2*>(dst) = w;
}

__device__ __forceinline__ floatx4 load_or_one(const float* p, int i) {
  return p ? reinterpret_cast<const floatx4*>(p)[i] : floatx4{1.f, 1.f, 1.f, 1.f};
}

// Loads row t of src into v and returns the wave-wide sum of squares.
__device__ __forceinline__ float load_row(const float* __restrict__ src, int d4, int lane, floatx4 (&v)[kRowChunks]) {
  const floatx4* row = reinterpret_cast<const floatx4*>(src);
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = c * 64 + lane;
    if (i < d4) {
      v[c] = row[i];
      ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
    }
  }
  return wave_sum(ss);
}

// out = RMSNorm(x; w) * scale.
template <typename OutT>
__global__ __launch_bounds__(256) void norm_mod_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       const float* __restrict__ scale, OutT* __restrict__ out, int T,
                                                       int D, float eps) {
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int t = (int)blockIdx.x * 4 + wave;
  if (t >= T) return;
  const int d4 = D >> 2;
  floatx4 v[kRowChunks];
  const float ss = load_row(x + (size_t)t * D, d4, lane, v);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  const floatx4* w4 = reinterpret_cast<const floatx4*>(w);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = c * 64 + lane;
    if (i < d4) {
      const floatx4 g = w4[i], sc = load_or_one(scale, i);
      floatx4 o;
      o.x = v[c].x * inv * g.x * sc.x;
      o.y = v[c].y * inv * g.y * sc.y;
      o.z = v[c].z * inv * g.z * sc.z;
      o.w = v[c].w * inv * g.w * sc.w;
      store4(out + (size_t)t * D + 4 * i, o);
    }
  }
}

// r = x + gate * RMSNorm(proj; n2) (fp32 out), f = RMSNorm(r; n3) * scale (OutT).
template <typename OutT>
__global__ __launch_bounds__(256) void resid_norm_mod_kernel(const float* __restrict__ x, const float* __restrict__ proj,
                                                             const float* __restrict__ n2, const float* __restrict__ gate,
                                                             const float* __restrict__ n3, const float* __restrict__ scale,
                                                             float* __restrict__ r_out, OutT* __restrict__ f_out, int T,
                                                             int D, float eps) {
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int t = (int)blockIdx.x * 4 + wave;
  if (t >= T) return;
  const int d4 = D >> 2;
  floatx4 v[kRowChunks];
  const float ss = load_row(proj + (size_t)t * D, d4, lane, v);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  const floatx4* x4 = reinterpret_cast<const floatx4*>(x + (size_t)t * D);
  const floatx4* w4 = reinterpret_cast<const floatx4*>(n2);
  float ss2 = 0.0f;
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = c * 64 + lane;
    if (i < d4) {
      const floatx4 xv = x4[i], g = load_or_one(gate, i), w = w4[i];
      floatx4 r;
      r.x = xv.x + g.x * (v[c].x * inv * w.x);
      r.y = xv.y + g.y * (v[c].y * inv * w.y);
      r.z = xv.z + g.z * (v[c].z * inv * w.z);
      r.w = xv.w + g.w * (v[c].w * inv * w.w);
      v[c] = r;
      reinterpret_cast<floatx4*>(r_out + (size_t)t * D)[i] = r;
      ss2 += r.x * r.x + r.y * r.y + r.z * r.z + r.w * r.w;
    }
  }
  ss2 = wave_sum(ss2);
  const float inv2 = 1.0f / sqrtf(ss2 / (float)D + eps);
  const floatx4* w3 = reinterpret_cast<const floatx4*>(n3);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = c * 64 + lane;
    if (i < d4) {
      const floatx4 w = w3[i], sc = load_or_one(scale, i);
      floatx4 o;
      o.x = v[c].x * inv2 * w.x * sc.x;
      o.y = v[c].y * inv2 * w.y * sc.y;
      o.z = v[c].z * inv2 * w.z * sc.z;
      o.w = v[c].w * inv2 * w.w * sc.w;
      store4(f_out + (size_t)t * D + 4 * i, o);
    }
  }
}

// out = r + gate * RMSNorm(w2; n4)
__global__ __launch_bounds__(256) void final_resid_kernel(const float* __restrict__ r, const float* __restrict__ w2,
                                                          const float* __restrict__ n4, const float* __restrict__ gate,
                                                          float* __restrict__ out, int T, int D, float eps) {
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int t = (int)blockIdx.x * 4 + wave;
  if (t >= T) return;
  const int d4 = D >> 2;
  floatx4 v[kRowChunks];
  const float ss = load_row(w2 + (size_t)t * D, d4, lane, v);
  const float inv = 1.0f / sqrtf(ss / (float)D + eps);
  const floatx4* r4 = reinterpret_cast<const floatx4*>(r + (size_t)t * D);
  const floatx4* w4 = reinterpret_cast<const floatx4*>(n4);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = c * 64 + lane;
    if (i < d4) {
      const floatx4 rv = r4[i], w = w4[i], g = load_or_one(gate, i);
      floatx4 o;
      o.x = rv.x + g.x * (v[c].x * inv * w.x);
      o.y = rv.y + g.y * (v[c].y * inv * w.y);
      o.z = rv.z + g.z * (v[c].z * inv * w.z);
      o.w = rv.w + g.w * (v[c].w * inv * w.w);
      reinterpret_cast<floatx4*>(out + (size_t)t * D)[i] = o;
    }
  }
}

}  // namespace rows
}  // namespace
}  // namespace prom
