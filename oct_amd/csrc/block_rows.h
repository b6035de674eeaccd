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
// (round to nearest even).  Callers guarantee D % 4 == 0, D <= 4096 and
// 16-byte aligned rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prom {
namespace {  // each translation unit gets its own copy of these kernels
namespace rows {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

constexpr int kRowChunks = 16;

// Every access goes through a buffer resource spanning exactly one row (or
// one D-vector): chunks past D read zero and their stores are dropped by the
// hardware range check, so the 16 loads of a row are issued back to back with
// no per-chunk branch (and no wait between them).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

__device__ __forceinline__ floatx4 ld4(__amdgpu_buffer_rsrc_t r, int i) {
  return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(16 * i), 0, 0));
}

// Sum over the 64 lanes (every lane gets it; call with the whole wave
// active): four DPP steps within each row of 16 lanes (swap pairs, swap the
// halves of quads, mirror within 8, mirror within 16), then two lane permutes
// across the rows, in place of six permutes through the LDS unit (C5
// resid_norm_mod 47.5 -> 45.5 us).
template <int kCtrl>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF,
                                                                   false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// fp32 -> bf16 bits, hardware round-to-nearest-even (finite inputs).
__device__ __forceinline__ uint16_t f2bf(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }

// 4 values to dst with one 128-bit (fp32) or 64-bit (bf16) store.
__device__ __forceinline__ void store4(float* dst, floatx4 v) { *reinterpret_cast<floatx4*>(dst) = v; }

__device__ __forceinline__ void store4(uint16_t* dst, floatx4 v) {
  const bf16x4 h = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
  *reinterpret_cast<u32x2*>(dst) = __builtin_bit_cast(u32x2, h);
}

// Chunk i (4 values) of a row: fp32, or bf16 with the hardware
// round-to-nearest-even conversion.
__device__ __forceinline__ void st4(__amdgpu_buffer_rsrc_t r, int i, floatx4 v, float*) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (uint32_t)(16 * i), 0, 0);
}

__device__ __forceinline__ void st4(__amdgpu_buffer_rsrc_t r, int i, floatx4 v, uint16_t*) {
  const bf16x4 h = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, h), r, (uint32_t)(8 * i), 0, 0);
}

// Chunk i (4 values, bf16) of row t of a K-blocked matrix [D/32][slice][32]
// (the layout a following bf16 GEMM reads in whole 128-byte lines); chunks
// past D are dropped.
__device__ __forceinline__ void st4_blocked(uint16_t* base, int slice, int t, int i, int d4, floatx4 v) {
  if (i >= d4) return;
  const bf16x4 h = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
  *reinterpret_cast<u32x2*>(base + ((size_t)(i >> 3) * slice + t) * 32 + 4 * (i & 7)) = __builtin_bit_cast(u32x2, h);
}

__device__ __forceinline__ void st4_blocked(float*, int, int, int, int, floatx4) {}  // fp32 outputs stay row-major

// An fp32 chunk as a streaming store (cache-policy operand 2: nt), for fp32
// rows that no kernel reads soon: they leave no dirty L2 lines for the next
// kernels to wait on.
__device__ __forceinline__ void st4_stream(__amdgpu_buffer_rsrc_t r, int i, floatx4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (uint32_t)(16 * i), 0, 2);
}

// Issues the 16 chunk loads of a row (zero past D) into v.
__device__ __forceinline__ void load_row(const float* __restrict__ src, int D, int lane, floatx4 (&v)[kRowChunks]) {
  const __amdgpu_buffer_rsrc_t r = row_rsrc(src, 4 * D);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) v[c] = ld4(r, c * 64 + lane);
}

// The same from a bf16 row (64-bit loads, widened exactly).
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ src, int D, int lane,
                                         floatx4 (&v)[kRowChunks]) {
  const __amdgpu_buffer_rsrc_t r = row_rsrc(src, 2 * D);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (uint32_t)(8 * (c * 64 + lane)), 0, 0));
    v[c] = floatx4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                   __uint_as_float(w.y & 0xffff0000u)};
  }
}

__device__ __forceinline__ float sum_sq(const floatx4 (&v)[kRowChunks]) {
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
  return wave_sum(ss);
}

// The D-vectors (norm weights, adaLN scale and gate) are staged once per
// workgroup in LDS (absent vectors as ones) while the row loads are in
// flight; the per-chunk reads are then LDS reads, not dependent global loads.
__device__ __forceinline__ void stage_vec(floatx4* dst, const float* src, int d4) {
  for (int i = (int)threadIdx.x; i < d4; i += (int)blockDim.x)
    dst[i] = src ? reinterpret_cast<const floatx4*>(src)[i] : floatx4{1.f, 1.f, 1.f, 1.f};
}

// The norm kernels below run one row per wave, kRows rows per workgroup:
// the D-vectors (norm weights, adaLN scale and gate, up to 4 x 16 KiB) are
// staged in LDS once per workgroup.  resid_norm_mod, with four vectors, takes
// 8 rows by default (with 4 its vector reads from L2 matched the row data
// itself, 57 -> 53 us at C5; the bf16 block launches 12); the two-vector
// kernels keep 4, which lets more workgroups share a CU (final_resid: 36 us
// with 4 rows, 43 with 8).  Both hold two rows' worth of registers and run
// 3 waves per SIMD, so the row count sets how many rounds of workgroups a
// launch takes.
template <int kRows>
inline dim3 row_groups(int T) { return dim3((unsigned)((T + kRows - 1) / kRows)); }

// out = RMSNorm(x; w) * scale; out_slice > 0 (bf16 only): out is K-blocked
// with that many rows per slice.
template <typename OutT, int kRows = 4>
__global__ __launch_bounds__(64 * kRows) void norm_mod_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       const float* __restrict__ scale, OutT* __restrict__ out, int T,
                                                       int D, float eps, int out_slice) {
  __shared__ floatx4 sw[1024], ssc[1024];
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = (int)(threadIdx.x & 63);
  const int t = min((int)blockIdx.x * kRows + wave, T - 1);
  const int d4 = D >> 2;
  floatx4 v[kRowChunks];
  load_row(x + (size_t)t * D, D, lane, v);
  stage_vec(sw, w, d4);
  stage_vec(ssc, scale, d4);
  __syncthreads();
  if ((int)blockIdx.x * kRows + wave >= T) return;
  const float inv = 1.0f / sqrtf(sum_sq(v) / (float)D + eps);
  const __amdgpu_buffer_rsrc_t ro = row_rsrc(out + (size_t)t * D, (int)sizeof(OutT) * D);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = c * 64 + lane;
    const floatx4 g = sw[i], sc = ssc[i];
    floatx4 o;
    o.x = v[c].x * inv * g.x * sc.x;
    o.y = v[c].y * inv * g.y * sc.y;
    o.z = v[c].z * inv * g.z * sc.z;
    o.w = v[c].w * inv * g.w * sc.w;
    if (out_slice > 0)
      st4_blocked(out, out_slice, t, i, d4, o);
    else
      st4(ro, i, o, out);
  }
}

// r = x + gate * RMSNorm(proj; n2) (fp32 out), f = RMSNorm(r; n3) * scale (OutT); proj fp32 or bf16.
// kStream: r is written with streaming stores.  f_slice > 0 (bf16 only): f is
// K-blocked with that many rows per slice.
template <typename OutT, int kRows = 8, typename ProjT = float, bool kStream = false>
__global__ __launch_bounds__(64 * kRows) void resid_norm_mod_kernel(const float* __restrict__ x, const ProjT* __restrict__ proj,
                                                             const float* __restrict__ n2, const float* __restrict__ gate,
                                                             const float* __restrict__ n3, const float* __restrict__ scale,
                                                             float* __restrict__ r_out, OutT* __restrict__ f_out, int T,
                                                             int D, float eps, int f_slice) {
  __shared__ floatx4 s2[1024], sg[1024], s3[1024], ssc[1024];
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = (int)(threadIdx.x & 63);
  const int t = min((int)blockIdx.x * kRows + wave, T - 1);
  const int d4 = D >> 2;
  floatx4 v[kRowChunks], xv[kRowChunks];
  load_row(proj + (size_t)t * D, D, lane, v);
  load_row(x + (size_t)t * D, D, lane, xv);
  stage_vec(s2, n2, d4);
  stage_vec(sg, gate, d4);
  stage_vec(s3, n3, d4);
  stage_vec(ssc, scale, d4);
  __syncthreads();
  if ((int)blockIdx.x * kRows + wave >= T) return;
  const float inv = 1.0f / sqrtf(sum_sq(v) / (float)D + eps);
  const __amdgpu_buffer_rsrc_t rr = row_rsrc(r_out + (size_t)t * D, 4 * D);
  float ss2 = 0.0f;
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = c * 64 + lane;
    const floatx4 g = sg[i], w = s2[i];
    floatx4 r;
    r.x = xv[c].x + g.x * (v[c].x * inv * w.x);
    r.y = xv[c].y + g.y * (v[c].y * inv * w.y);
    r.z = xv[c].z + g.z * (v[c].z * inv * w.z);
    r.w = xv[c].w + g.w * (v[c].w * inv * w.w);
    // chunks past D hold garbage vector values: keep them out of the sum
    if (i >= d4) r = floatx4{0.f, 0.f, 0.f, 0.f};
    v[c] = r;
    if constexpr (kStream)
      st4_stream(rr, i, r);
    else
      st4(rr, i, r, r_out);
    ss2 += r.x * r.x + r.y * r.y + r.z * r.z + r.w * r.w;
  }
  ss2 = wave_sum(ss2);
  const float inv2 = 1.0f / sqrtf(ss2 / (float)D + eps);
  const __amdgpu_buffer_rsrc_t rf = row_rsrc(f_out + (size_t)t * D, (int)sizeof(OutT) * D);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = c * 64 + lane;
    const floatx4 w = s3[i], sc = ssc[i];
    floatx4 o;
    o.x = v[c].x * inv2 * w.x * sc.x;
    o.y = v[c].y * inv2 * w.y * sc.y;
    o.z = v[c].z * inv2 * w.z * sc.z;
    o.w = v[c].w * inv2 * w.w * sc.w;
    if (f_slice > 0)
      st4_blocked(f_out, f_slice, t, i, d4, o);
    else
      st4(rf, i, o, f_out);
  }
}

// out = r + gate * RMSNorm(w2; n4); w2 fp32 or bf16.
// kStream: out is written with streaming stores.
template <int kRows = 4, typename W2T = float, bool kStream = false>
__global__ __launch_bounds__(64 * kRows) void final_resid_kernel(const float* __restrict__ r, const W2T* __restrict__ w2,
                                                          const float* __restrict__ n4, const float* __restrict__ gate,
                                                          float* __restrict__ out, int T, int D, float eps) {
  __shared__ floatx4 s4[1024], sg[1024];
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = (int)(threadIdx.x & 63);
  const int t = min((int)blockIdx.x * kRows + wave, T - 1);
  const int d4 = D >> 2;
  floatx4 v[kRowChunks], rv[kRowChunks];
  load_row(w2 + (size_t)t * D, D, lane, v);
  load_row(r + (size_t)t * D, D, lane, rv);
  stage_vec(s4, n4, d4);
  stage_vec(sg, gate, d4);
  __syncthreads();
  if ((int)blockIdx.x * kRows + wave >= T) return;
  const float inv = 1.0f / sqrtf(sum_sq(v) / (float)D + eps);
  const __amdgpu_buffer_rsrc_t ro = row_rsrc(out + (size_t)t * D, 4 * D);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = c * 64 + lane;
    const floatx4 w = s4[i], g = sg[i];
    floatx4 o;
    o.x = rv[c].x + g.x * (v[c].x * inv * w.x);
    o.y = rv[c].y + g.y * (v[c].y * inv * w.y);
    o.z = rv[c].z + g.z * (v[c].z * inv * w.z);
    o.w = rv[c].w + g.w * (v[c].w * inv * w.w);
    if constexpr (kStream)
      st4_stream(ro, i, o);
    else
      st4(ro, i, o, out);
  }
}

}  // namespace rows
}  // namespace
}  // namespace prom
