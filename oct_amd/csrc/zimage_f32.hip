// fp32 Z-Image transformer block on resident weights: the compute behind the
// resident model-block ABI's NoiseRefiner, ContextRefiner and MainTransformer
// families (model_block.hip).
//
// Stage definitions are the reference's canonical blocks:
//   NoiseRefiner   internal/prometheus/zimage/canonical_reference.go:315-480
//   ContextRefiner internal/prometheus/zimage/context_refiner_reference.go:230-311
//                  (no adaLN: every scale and gate is 1)
//   MainTransformer tools/python/zimage/zimage_main_transformer_canonical.py:178-277
//                  (joint sequence, image tokens then context tokens)
// with weights cached row-major [input, output] (canonical_reference.go:153-175)
// and fp32 arithmetic throughout (FP16 weights are widened exactly once, at
// upload).
//
// MI355X design: the matrix work is the fp32 MFMA SGEMM (sgemm_f32.hip);
// attention is the fp32 flash kernel (attention_f32.hip: scores, online
// softmax and P.V per 32-key tile in registers and LDS, the 1/sqrt(128) scale
// folded into Q; no [H, T, T] score tensor).  Around them:
//   adaln         m = c @ Wada + b; raw and adjusted (1 + scale, tanh gate)
//   rope_table    (cos, sin) per token and pair, the reference's float32 angle
//   norm_mod      a = RMSNorm(x; n1) * scaleA                    (block_rows.h)
//   qkv_split     per (64 tokens, head): RMSNorm(q), RMSNorm(k), RoPE; writes
//                 Q [H, T, 128], K^T [H, 128, T] (transposed through LDS so the
//                 stores stay coalesced) and V [H, T, 128]
//   resid_norm_mod r = x + gateA * RMSNorm(proj; n2), f = RMSNorm(r; n3) * scaleM
//   swiglu        h = silu(w1) * w3
//   final_resid   out = r + gateM * RMSNorm(w2; n4)
// Every intermediate stays in its own workspace buffer, so any stage can be
// copied out for an audit after the chain completes.
#include <math.h>

#include "block_rows.h"
#include "reactor_internal.h"

namespace prom {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kHead = 128;
constexpr int kSplitTokens = 64;  // tokens per qkv_split workgroup

__global__ __launch_bounds__(256) void widen_f16_kernel(const uint16_t* __restrict__ src, float* __restrict__ dst,
                                                        size_t rows, size_t cols, size_t dst_ld) {
  const size_t total = rows * cols;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / cols, c = i - r * cols;
    dst[r * dst_ld + c] = (float)__builtin_bit_cast(_Float16, src[i]);
  }
}

__global__ __launch_bounds__(256) void widen_bf16_kernel(const uint16_t* __restrict__ src, float* __restrict__ dst,
                                                         size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = __uint_as_float((uint32_t)src[i] << 16);
}

// raw[j] = b[j] + sum_k c[k] * W[k][j]; adjusted: chunks 0 and 2 -> 1 + raw,
// chunks 1 and 3 -> tanh(raw) (canonical_reference.go:360-383).  A workgroup
// owns 64 columns; its 4 waves take every 4th k and combine through LDS.
__global__ __launch_bounds__(256) void adaln_f32_kernel(const float* __restrict__ cond, const float* __restrict__ W,
                                                        const float* __restrict__ b, float* __restrict__ raw,
                                                        float* __restrict__ mod, int C, int D) {
  __shared__ float part[4][64];
  const int lane = (int)(threadIdx.x & 63);
  const int kg = (int)(threadIdx.x >> 6);
  const int j = (int)blockIdx.x * 64 + lane;
  float acc = 0.0f;
  if (j < 4 * D) {
    for (int k = kg; k < C; k += 4) acc += cond[k] * W[(size_t)k * 4 * D + j];
  }
  part[kg][lane] = acc;
  __syncthreads();
  if (kg == 0 && j < 4 * D) {
    const float m = b[j] + ((part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]));
    const int chunk = j / D;
    raw[j] = m;
    mod[j] = (chunk == 0 || chunk == 2) ? 1.0f + m : (float)tanh((double)m);
  }
}

// The same product with 16-byte weight loads (W 16-byte aligned, 4D a
// multiple of 4): a workgroup owns 128 columns, lane c of each 32-lane group 4
// consecutive columns, and the 8 groups take every 8th k; every load of a
// thread is independent, so they are all in flight together (the loop above
// waits on one load per step: 30 us for the 15.7 MB of the MainTransformer's
// adaLN weight).  The 8 partial sums are added in a fixed order.
__global__ __launch_bounds__(256) void adaln_f32_vec_kernel(const float* __restrict__ cond,
                                                            const float* __restrict__ W, const float* __restrict__ b,
                                                            float* __restrict__ raw, float* __restrict__ mod, int C,
                                                            int D) {
  typedef float floatx4 __attribute__((ext_vector_type(4)));
  __shared__ float part[8][129];
  const int cg = (int)(threadIdx.x & 31);
  const int kg = (int)(threadIdx.x >> 5);
  const int j0 = (int)blockIdx.x * 128 + cg * 4;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  if (j0 < 4 * D) {
#pragma unroll 8
    for (int k = kg; k < C; k += 8) acc += cond[k] * *reinterpret_cast<const floatx4*>(W + (size_t)k * 4 * D + j0);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) part[kg][cg * 4 + i] = acc[i];
  __syncthreads();
  if (threadIdx.x < 128) {
    const int j = (int)blockIdx.x * 128 + (int)threadIdx.x;
    if (j < 4 * D) {
      float m = 0.0f;
#pragma unroll
      for (int g = 0; g < 8; ++g) m += part[g][threadIdx.x];
      m += b[j];
      const int chunk = j / D;
      raw[j] = m;
      mod[j] = (chunk == 0 || chunk == 2) ? 1.0f + m : (float)tanh((double)m);
    }
  }
}

// tab[t][p] = (cos, sin) of angle = coord(float32) * freq(float32), with
// freq = float32(1 / 256^(2*pair/width)) and cos/sin evaluated in binary64 on
// the float32 angle: CanonicalRopeFrequency/CanonicalRopeRotate
// (zimage/canonical_contract.go:66-87), axes [32, 48, 48].
__global__ __launch_bounds__(256) void rope_table_f32_kernel(const float* __restrict__ coords, float2* __restrict__ tab,
                                                             int T) {
  const int idx = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (idx >= T * 64) return;
  const int t = idx >> 6;
  const int p = idx & 63;
  int axis, width, pair;
  if (p < 16) {
    axis = 0; width = 32; pair = p;
  } else if (p < 40) {
    axis = 1; width = 48; pair = p - 16;
  } else {
    axis = 2; width = 48; pair = p - 40;
  }
  const float freq = (float)(1.0 / pow(256.0, (double)(2 * pair) / (double)width));
  const float angle = coords[(size_t)t * 3 + axis] * freq;
  tab[idx] = make_float2((float)cos((double)angle), (float)sin((double)angle));
}

// Workgroup (token tile of 64, head h).  Wave w handles tokens t0 + w + 4i;
// lane l owns the rotary pair (2l, 2l+1) of the 128-wide head.  q and k are
// RMSNormed over the head (eps), rotated with the token's table entry; q is
// scaled by q_scale.  K is staged in LDS and written transposed.
__global__ __launch_bounds__(256) void qkv_split_kernel(const float* __restrict__ qkv, const float2* __restrict__ tab,
                                                        const float* __restrict__ qn, const float* __restrict__ kn,
                                                        float* __restrict__ Q, float* __restrict__ Kt,
                                                        float* __restrict__ V, int T, int H, float eps, float q_scale) {
  __shared__ float ks[kHead][kSplitTokens + 1];
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int t0 = (int)blockIdx.x * kSplitTokens;
  const int h = (int)blockIdx.y;
  const int D = H * kHead;
  const float qw0 = qn[2 * lane], qw1 = qn[2 * lane + 1];
  const float kw0 = kn[2 * lane], kw1 = kn[2 * lane + 1];
  for (int j = wave; j < kSplitTokens; j += 4) {
    const int t = t0 + j;
    if (t >= T) break;
    const float* row = qkv + (size_t)t * 3 * D + h * kHead + 2 * lane;
    const float2 cs = tab[(size_t)t * 64 + lane];
    {
      const float e = row[0], o = row[1];
      const float inv = 1.0f / sqrtf(rows::wave_sum(e * e + o * o) / (float)kHead + eps);
      const float ne = e * inv * qw0, no = o * inv * qw1;
      float2 out;
      out.x = (ne * cs.x - no * cs.y) * q_scale;
      out.y = (ne * cs.y + no * cs.x) * q_scale;
      *reinterpret_cast<float2*>(Q + ((size_t)h * T + t) * kHead + 2 * lane) = out;
    }
    {
      const float e = row[D], o = row[D + 1];
      const float inv = 1.0f / sqrtf(rows::wave_sum(e * e + o * o) / (float)kHead + eps);
      const float ne = e * inv * kw0, no = o * inv * kw1;
      ks[2 * lane][j] = ne * cs.x - no * cs.y;
      ks[2 * lane + 1][j] = ne * cs.y + no * cs.x;
    }
    *reinterpret_cast<float2*>(V + ((size_t)h * T + t) * kHead + 2 * lane) =
        *reinterpret_cast<const float2*>(row + 2 * D);
  }
  __syncthreads();
  const int n = min(kSplitTokens, T - t0);
  for (int i = (int)threadIdx.x; i < kHead * kSplitTokens; i += 256) {
    const int c = i / kSplitTokens, j = i - c * kSplitTokens;
    if (j < n) Kt[((size_t)h * kHead + c) * T + t0 + j] = ks[c][j];
  }
}

// Audit recomputation of q or k (which = 0 / 1) after the head RMSNorm and,
// when rope is set, the rotation, in the canonical [T, H*128] layout without
// the attention scale (the "q_norm" / "q_rope" stages of canonical_reference.go:412-426).
__global__ __launch_bounds__(256) void qk_audit_kernel(const float* __restrict__ qkv, const float2* __restrict__ tab,
                                                       const float* __restrict__ nw, float* __restrict__ out, int T,
                                                       int H, float eps, int which, int rope) {
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int unit = (int)blockIdx.x * 4 + wave;
  if (unit >= T * H) return;
  const int t = unit / H, h = unit - t * H;
  const int D = H * kHead;
  const float* row = qkv + (size_t)t * 3 * D + (size_t)which * D + h * kHead + 2 * lane;
  const float e = row[0], o = row[1];
  const float inv = 1.0f / sqrtf(rows::wave_sum(e * e + o * o) / (float)kHead + eps);
  float ne = e * inv * nw[2 * lane], no = o * inv * nw[2 * lane + 1];
  if (rope) {
    const float2 cs = tab[(size_t)t * 64 + lane];
    const float re = ne * cs.x - no * cs.y, ro = ne * cs.y + no * cs.x;
    ne = re;
    no = ro;
  }
  *reinterpret_cast<float2*>(out + (size_t)t * D + h * kHead + 2 * lane) = make_float2(ne, no);
}

// G [T, 2F] (w1 | w3) -> h [T, F] = silu(w1) * w3 (canonical_reference.go:457-460).
__global__ __launch_bounds__(256) void swiglu_f32_kernel(const float* __restrict__ G, float* __restrict__ Hd, int T,
                                                         int F) {
  const size_t total = (size_t)T * F;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
    const size_t t = idx / F, i = idx - t * F;
    const float g = G[t * 2 * F + i], u = G[t * 2 * F + F + i];
    Hd[idx] = g / (1.0f + expf(-g)) * u;
  }
}

// The same with 16-byte accesses (F % 4 == 0, G and Hd 16-byte aligned): row
// t = blockIdx.y, four columns per thread, no per-element index division.
__device__ __forceinline__ float silu_mul_f32(float g, float u) { return g / (1.0f + expf(-g)) * u; }

__global__ __launch_bounds__(256) void swiglu_f32_vec_kernel(const float4* __restrict__ G, float4* __restrict__ Hd,
                                                             int F4) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= F4) return;
  const size_t t = blockIdx.y;
  const float4 g = G[t * 2 * F4 + i];
  const float4 u = G[t * 2 * F4 + F4 + i];
  Hd[t * F4 + i] = make_float4(silu_mul_f32(g.x, u.x), silu_mul_f32(g.y, u.y), silu_mul_f32(g.z, u.z),
                               silu_mul_f32(g.w, u.w));
}

// One audit summary record per workgroup.  Lane l reduces the elements
// l, l + 256, ... in increasing order; the lanes then combine in a fixed
// binary tree (strides 128 .. 1), the reference's order.
__global__ __launch_bounds__(256) void audit_summary_kernel(const ZImageAuditJob* __restrict__ jobs,
                                                            uint32_t* __restrict__ arena) {
  __shared__ float ss[256], lo[256], hi[256];
  __shared__ uint32_t nfin[256], nnan[256], ninf[256];
  const ZImageAuditJob& j = jobs[blockIdx.x];
  const uint32_t lane = threadIdx.x;
  const float* src = j.src;
  const uint32_t count = j.count, cols = j.cols, ld = j.ld;
  float sum = 0.0f, mn = __uint_as_float(0x7f800000u), mx = __uint_as_float(0xff800000u);
  uint32_t nf = 0, nn = 0, ni = 0;
#pragma unroll 4
  for (uint32_t e = lane; e < count; e += 256u) {
    const uint32_t r = e / cols;
    const float v = src[(size_t)r * ld + (e - r * cols)];
    if (v != v) {
      ++nn;
    } else if (v - v != 0.0f) {
      ++ni;
    } else {
      ++nf;
      sum += v * v;
      mn = v < mn ? v : mn;
      mx = v > mx ? v : mx;
    }
  }
  ss[lane] = sum;
  lo[lane] = mn;
  hi[lane] = mx;
  nfin[lane] = nf;
  nnan[lane] = nn;
  ninf[lane] = ni;
  __syncthreads();
  for (uint32_t stride = 128u; stride > 0u; stride >>= 1) {
    if (lane < stride) {
      const uint32_t o = lane + stride;
      ss[lane] = ss[lane] + ss[o];
      nfin[lane] += nfin[o];
      nnan[lane] += nnan[o];
      ninf[lane] += ninf[o];
      if (lo[o] < lo[lane]) lo[lane] = lo[o];
      if (hi[o] > hi[lane]) hi[lane] = hi[o];
    }
    __syncthreads();
  }
  if (lane != 0) return;
  const uint32_t qnan = 0x7fc00000u;
  uint32_t* rec = arena + j.dest_word;
  for (int i = 0; i < 64; ++i) rec[i] = 0u;
  const uint32_t finite = nfin[0];
  rec[0] = j.stage_id;
  rec[1] = j.generation;
  rec[2] = count;
  rec[3] = finite == count ? 1u : 0u;
  rec[4] = nnan[0];
  rec[5] = ninf[0];
  rec[6] = finite;
  rec[7] = j.key_count;
  rec[8] = finite ? __float_as_uint(lo[0]) : qnan;
  rec[9] = finite ? __float_as_uint(hi[0]) : qnan;
  rec[10] = __float_as_uint(ss[0]);
  rec[11] = finite ? __float_as_uint(sqrtf(ss[0] / (float)finite)) : qnan;
  rec[12] = 1u;
  for (uint32_t k = 0; k < j.key_count && k < kZImageAuditMaxKeys; ++k) {
    const uint32_t e = j.keys[k];
    rec[16 + 2 * k] = e;
    if (e < count) {
      const uint32_t r = e / cols;
      rec[17 + 2 * k] = __float_as_uint(src[(size_t)r * ld + (e - r * cols)]);
    } else {
      rec[17 + 2 * k] = qnan;
      rec[13] = 1u;
    }
  }
}

// The streaming-attention witness: workgroup 0 takes (token 0, head 0),
// workgroup 1 (token T-1, head H-1).  The scores come from the split Q and
// K^T (Q carries the 1/sqrt(128) scale, so s is the scaled score); lane 0
// then makes the reference's serial passes over the keys: the maximum, the
// exponentials and their sum, the normalisation and the row sum.
__global__ __launch_bounds__(256) void attention_witness_kernel(const float* __restrict__ Q,
                                                                const float* __restrict__ Kt,
                                                                const float* __restrict__ V,
                                                                const float* __restrict__ O, int T, int H,
                                                                float q_scale, int image_format,
                                                                float* __restrict__ out) {
  __shared__ float s[kZImageWitnessMaxTokens], p[kZImageWitnessMaxTokens];
  const int row = (int)blockIdx.x;
  const int t = row ? T - 1 : 0, h = row ? H - 1 : 0;
  const float* q = Q + ((size_t)h * T + t) * kHead;
  const float* kt = Kt + (size_t)h * kHead * T;
  for (int k = (int)threadIdx.x; k < T; k += 256) {
    float d = 0.0f;
    for (int c = 0; c < kHead; ++c) d += q[c] * kt[(size_t)c * T + k];
    s[k] = d;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  float w[32] = {};
  float mx = s[0];
  for (int k = 1; k < T; ++k) mx = s[k] > mx ? s[k] : mx;
  float sum = 0.0f;
  for (int k = 0; k < T; ++k) {
    p[k] = expf(s[k] - mx);
    sum += p[k];
  }
  const bool valid = sum == sum && sum > 0.0f && sum - sum == 0.0f;
  const int keys[4] = {0, 1, T / 2, T - 1};
  if (image_format) {
    for (int i = 0; i < 4; ++i) {
      const int k = keys[i];
      w[5 * i] = s[k] / q_scale;
      w[5 * i + 1] = s[k];
      w[5 * i + 2] = s[k] - mx;
      w[5 * i + 3] = p[k];
    }
    w[20] = mx;
    w[21] = sum;
  }
  float row_sum = 0.0f;
  for (int k = 0; k < T; ++k) {
    p[k] = valid ? p[k] / sum : 0.0f;
    row_sum += p[k];
  }
  if (image_format) {
    for (int i = 0; i < 4; ++i) w[5 * i + 4] = p[keys[i]];
    w[22] = row_sum;
    w[23] = p[0] * V[(size_t)h * T * kHead];
    w[24] = O[(size_t)t * H * kHead + (size_t)h * kHead];
  } else {
    w[0] = s[0] / q_scale;
    w[1] = s[0];
    w[2] = s[0] - mx;
    w[3] = p[0];
    w[4] = row_sum;
  }
  w[30] = valid ? 1.0f : 0.0f;
  for (int i = 0; i < 32; ++i) out[32 * row + i] = w[i];
}

inline unsigned grid_for(size_t n) { return (unsigned)std::min<size_t>(65536, (n + 255) / 256); }

}  // namespace

size_t zimage_workspace_layout(int T, int D, int H, int F, size_t off[kZCount]) {
  const size_t t = (size_t)T, d = (size_t)D, f = (size_t)F;
  size_t sizes[kZCount] = {};
  sizes[kZModRaw] = 4 * d * 4;
  sizes[kZMod] = 4 * d * 4;
  sizes[kZA] = t * d * 4;
  sizes[kZQkv] = t * 3 * d * 4;
  sizes[kZQ] = t * d * 4;
  sizes[kZKt] = t * d * 4;
  sizes[kZV] = t * d * 4;
  sizes[kZS] = flash_attn_f32_partial_bytes(T, H, 1, kHead, 0);  // attention key-split partials (usually none)
  sizes[kZO] = t * d * 4;
  sizes[kZProj] = t * d * 4;
  sizes[kZR] = t * d * 4;
  sizes[kZF] = t * d * 4;
  sizes[kZG] = t * 2 * f * 4;
  sizes[kZH] = t * f * 4;
  sizes[kZW2] = t * d * 4;
  sizes[kZRope] = t * 64 * 8;
  size_t o = 0;
  for (int i = 0; i < kZCount; ++i) {
    off[i] = o;
    o += (sizes[i] + 255) & ~(size_t)255;
  }
  return o;
}

hipError_t launch_widen_f16(const uint16_t* src, float* dst, size_t rows_n, size_t cols, size_t dst_ld,
                            hipStream_t stream) {
  if (rows_n * cols == 0) return hipSuccess;
  hipLaunchKernelGGL(widen_f16_kernel, dim3(grid_for(rows_n * cols)), dim3(256), 0, stream, src, dst, rows_n, cols,
                     dst_ld);
  return hipGetLastError();
}

hipError_t launch_widen_bf16(const uint16_t* src, float* dst, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(widen_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, stream, src, dst, n);
  return hipGetLastError();
}

hipError_t launch_zimage_rope_table(const float* coords, float2* tab, int T, hipStream_t stream) {
  hipLaunchKernelGGL(rope_table_f32_kernel, dim3((T * 64 + 255) / 256), dim3(256), 0, stream, coords, tab, T);
  return hipGetLastError();
}

hipError_t launch_zimage_norm(const float* x, const float* w, float* out, int T, int D, float eps, hipStream_t stream) {
  hipLaunchKernelGGL(rows::norm_mod_kernel<float>, rows::row_groups<4>(T), dim3(256), 0, stream, x, w, (const float*)nullptr,
                     out, T, D, eps, 0);
  return hipGetLastError();
}

hipError_t launch_zimage_qk_audit(const float* qkv, const float2* tab, const float* norm_w, float* out, int T, int H,
                                  float eps, int which, bool rope, hipStream_t stream) {
  hipLaunchKernelGGL(qk_audit_kernel, dim3((T * H + 3) / 4), dim3(256), 0, stream, qkv, tab, norm_w, out, T, H, eps,
                     which, rope ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_zimage_audit_summary(const ZImageAuditJob* jobs, uint32_t job_count, uint32_t* arena,
                                       hipStream_t stream) {
  if (job_count == 0) return hipSuccess;
  hipLaunchKernelGGL(audit_summary_kernel, dim3(job_count), dim3(256), 0, stream, jobs, arena);
  return hipGetLastError();
}

hipError_t launch_zimage_attention_witness(const float* Q, const float* Kt, const float* V, const float* O, int T,
                                           int H, float q_scale, bool image_format, float* out, hipStream_t stream) {
  if (T < 1 || T > kZImageWitnessMaxTokens || H < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_witness_kernel, dim3(2), dim3(256), 0, stream, Q, Kt, V, O, T, H, q_scale,
                     image_format ? 1 : 0, out);
  return hipGetLastError();
}

hipError_t enqueue_zimage_block_f32(const ZImageBlockWeights& w, const float* x, const float* cond, float* out,
                                    char* ws, const size_t off[kZCount], int T, int D, int F, float eps,
                                    hipStream_t st, uint32_t* launches, int first_phase, int last_phase,
                                    const hipEvent_t* stage_events) {
  const int H = D / kHead;
  float* raw = reinterpret_cast<float*>(ws + off[kZModRaw]);
  float* mod = reinterpret_cast<float*>(ws + off[kZMod]);
  float* A = reinterpret_cast<float*>(ws + off[kZA]);
  float* qkv = reinterpret_cast<float*>(ws + off[kZQkv]);
  float* Q = reinterpret_cast<float*>(ws + off[kZQ]);
  float* Kt = reinterpret_cast<float*>(ws + off[kZKt]);
  float* V = reinterpret_cast<float*>(ws + off[kZV]);
  float* S = reinterpret_cast<float*>(ws + off[kZS]);
  float* O = reinterpret_cast<float*>(ws + off[kZO]);
  float* proj = reinterpret_cast<float*>(ws + off[kZProj]);
  float* R = reinterpret_cast<float*>(ws + off[kZR]);
  float* Fm = reinterpret_cast<float*>(ws + off[kZF]);
  float* G = reinterpret_cast<float*>(ws + off[kZG]);
  float* Hd = reinterpret_cast<float*>(ws + off[kZH]);
  float* W2 = reinterpret_cast<float*>(ws + off[kZW2]);
  const float2* rope = reinterpret_cast<const float2*>(ws + off[kZRope]);
  const bool modulated = w.adaln_w != nullptr;
  const float* scaleA = modulated ? mod : nullptr;
  const float* gateA = modulated ? mod + D : nullptr;
  const float* scaleM = modulated ? mod + 2 * D : nullptr;
  const float* gateM = modulated ? mod + 3 * D : nullptr;
  hipError_t e;
  uint32_t n = 0;
#define PROM_STEP(call)            \
  do {                             \
    e = (call);                    \
    if (e != hipSuccess) return e; \
    ++n;                           \
  } while (0)
  // stage_events[0] before the first stage, stage_events[i] after stage i (1..13)
  auto mark = [&](int i) { return stage_events ? hipEventRecord(stage_events[i], st) : hipSuccess; };
  const dim3 blk(256);
  if (first_phase > last_phase || first_phase < 1 || last_phase > 3) return hipErrorInvalidValue;
  if (launches) *launches = 0;
  if (first_phase == 1) {  // adaLN, attention norm, QKV, head norms and RoPE
    if ((e = mark(0)) != hipSuccess) return e;
    if (modulated) {
      if ((reinterpret_cast<uintptr_t>(w.adaln_w) & 15u) == 0 && D % 4 == 0)
        hipLaunchKernelGGL(adaln_f32_vec_kernel, dim3((4 * D + 127) / 128), blk, 0, st, cond, w.adaln_w, w.adaln_b, raw,
                           mod, kZImageConditionWidth, D);
      else
        hipLaunchKernelGGL(adaln_f32_kernel, dim3((4 * D + 63) / 64), blk, 0, st, cond, w.adaln_w, w.adaln_b, raw, mod,
                           kZImageConditionWidth, D);
      PROM_STEP(hipGetLastError());
    }
    if ((e = mark(1)) != hipSuccess) return e;
    hipLaunchKernelGGL(rows::norm_mod_kernel<float>, rows::row_groups<4>(T), dim3(256), 0, st, x, w.attn_norm1, scaleA, A, T, D, eps, 0);
    PROM_STEP(hipGetLastError());
    if ((e = mark(2)) != hipSuccess) return e;
    PROM_STEP(launch_sgemm_f32_ex(A, D, w.w_qkv, 3 * D, qkv, 3 * D, T, 3 * D, D, nullptr, 0, st, nullptr));
    if ((e = mark(3)) != hipSuccess) return e;
    hipLaunchKernelGGL(qkv_split_kernel, dim3((T + kSplitTokens - 1) / kSplitTokens, H), blk, 0, st, qkv, rope,
                       w.q_norm, w.k_norm, Q, Kt, V, T, H, eps, 1.0f / sqrtf((float)kHead));
    PROM_STEP(hipGetLastError());
    if ((e = mark(4)) != hipSuccess) return e;
  }
  if (first_phase <= 2 && last_phase >= 2) {  // attention, projection, gated residual, FFN norm
    {
      // Scores, softmax and P.V in one flash kernel (Q is already scaled by
      // 1/sqrt(128)); stages 6 and 7 close immediately after stage 5.
      AttnF32Params ap{};
      ap.q = Q;
      ap.kt = Kt;
      ap.v = V;
      ap.o = O;
      ap.q_hs = (long long)T * kHead;
      ap.q_rs = kHead;
      ap.kt_hs = (long long)kHead * T;
      ap.kt_rs = T;
      ap.v_hs = (long long)T * kHead;
      ap.v_rs = kHead;
      ap.o_rs = D;
      ap.T = T;
      ap.q_heads = H;
      ap.group = 1;
      ap.causal = 0;
      flash_attn_f32_bind_partials(ap, kHead, S);
      PROM_STEP(launch_flash_attn_f32(ap, kHead, 1.0f, st));
    }
    if ((e = mark(5)) != hipSuccess) return e;
    if ((e = mark(6)) != hipSuccess) return e;
    if ((e = mark(7)) != hipSuccess) return e;
    PROM_STEP(launch_sgemm_f32_ex(O, D, w.w_out, D, proj, D, T, D, D, nullptr, 0, st, nullptr));
    if ((e = mark(8)) != hipSuccess) return e;
    hipLaunchKernelGGL(rows::resid_norm_mod_kernel<float>, rows::row_groups<8>(T), dim3(512), 0, st, x, proj, w.attn_norm2, gateA,
                       w.ffn_norm1, scaleM, R, Fm, T, D, eps, 0);
    PROM_STEP(hipGetLastError());
    if ((e = mark(9)) != hipSuccess) return e;
  }
  if (last_phase == 3) {  // W1/W3, SwiGLU, W2, gated final residual
    PROM_STEP(launch_sgemm_f32_ex(Fm, D, w.w_13, 2 * F, G, 2 * F, T, 2 * F, D, nullptr, 0, st, nullptr));
    if ((e = mark(10)) != hipSuccess) return e;
    if (F % 4 == 0 && ((reinterpret_cast<uintptr_t>(G) | reinterpret_cast<uintptr_t>(Hd)) & 15) == 0 && T <= 65535)
      hipLaunchKernelGGL(swiglu_f32_vec_kernel, dim3((unsigned)((F / 4 + 255) / 256), (unsigned)T), blk, 0, st,
                         reinterpret_cast<const float4*>(G), reinterpret_cast<float4*>(Hd), F / 4);
    else
      hipLaunchKernelGGL(swiglu_f32_kernel, dim3(grid_for((size_t)T * F)), blk, 0, st, G, Hd, T, F);
    PROM_STEP(hipGetLastError());
    if ((e = mark(11)) != hipSuccess) return e;
    PROM_STEP(launch_sgemm_f32_ex(Hd, F, w.w_2, D, W2, D, T, D, F, nullptr, 0, st, nullptr));
    if ((e = mark(12)) != hipSuccess) return e;
    hipLaunchKernelGGL(rows::final_resid_kernel<4>, rows::row_groups<4>(T), dim3(256), 0, st, R, W2, w.ffn_norm2, gateM, out, T, D, eps);
    PROM_STEP(hipGetLastError());
    if ((e = mark(13)) != hipSuccess) return e;
  }
#undef PROM_STEP
  if (launches) *launches = n;
  return hipSuccess;
}

}  // namespace prom
