// Z-Image-style single-stream DiT block in bf16.
//
// Stage definitions follow the reference's canonical block
// (internal/prometheus/zimage/canonical_reference.go:315-480) and its joint
// main-transformer variant (tools/python/zimage/zimage_main_transformer_canonical.py:178-277):
// adaLN chunks (scaleA, gateA, scaleM, gateM) with 1+scale and tanh(gate),
// RMSNorm without mean subtraction, fused QKV with [Q|K|V] column order, per-head
// Q/K RMSNorm, 3-axis interleaved-pair RoPE, full softmax attention, gated
// residuals with a second RMSNorm, SwiGLU FFN.
//
// MI355X design: the four projections are bf16 MFMA GEMMs (gemm_bf16.hip) with
// fp32 accumulation; attention is the flash kernel (attention_bf16.hip); the
// per-row work between them is fused into four one-pass row kernels (one wave
// per row, the row held in registers, 128-bit loads):
//   adaln          m = c @ Wada + b -> modulation vectors       (16-byte weight loads, k split 16 ways)
//   rope_table     (cos, sin) per token and pair, binary64 angles (one launch with adaln)
//   norm_mod       a = RMSNorm(x; n1) * scaleA                   -> bf16
//   (QKV GEMM      -> bf16 [T, 3D])
//   k_norm_rope    per token and head, in place: RMSNorm(k), RoPE; the
//                  attention applies RMSNorm(q) and RoPE to Q as it loads it
//                  and reads Q, K, V from the [T, 3D] rows
//   (out-projection GEMM -> bf16 proj)
//   resid_norm_mod r = x + gateA * RMSNorm(proj; n2)             -> fp32
//                  f = RMSNorm(r; n3) * scaleM                   -> bf16
//   swiglu         h = silu(g) * u -> bf16, fused into the W1|W3 GEMM epilogue
//                  (gemm_bf16.hip) when F % 128 == 0 and D % 64 == 0
//   (W2 GEMM       -> bf16 w2)
//   final_resid    out = r + gateM * RMSNorm(w2; n4)              -> fp32
// The bf16 intermediates (qkv, proj, w2) are each normalised before they
// meet the fp32 residual stream.
#include <math.h>
#include <string.h>

#include "block_rows.h"
#include "reactor_internal.h"

namespace prom {

namespace {

using rows::f2bf;
using rows::floatx4;
using rows::wave_sum;

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// mod[j] = b[j] + sum_k c[k] * W[k][j]; chunk 0 and 2 -> 1 + m, chunk 1 and 3 -> tanh(m)
// (canonical_reference.go:373-383).  A workgroup owns 64 columns; its 4 waves
// take every 4th k (coalesced 128-byte row segments) and combine through LDS.
__global__ __launch_bounds__(256) void adaln_kernel(const float* __restrict__ cond, const uint16_t* __restrict__ W,
                                                    const float* __restrict__ b, float* __restrict__ mod, int C,
                                                    int D) {
  __shared__ float part[4][64];
  const int lane = (int)(threadIdx.x & 63);
  const int kg = (int)(threadIdx.x >> 6);
  const int j = (int)blockIdx.x * 64 + lane;
  float acc = 0.0f;
  if (j < 4 * D) {
    for (int k = kg; k < C; k += 4) acc += cond[k] * bf2f(W[(size_t)k * 4 * D + j]);
  }
  part[kg][lane] = acc;
  __syncthreads();
  if (kg == 0 && j < 4 * D) {
    const float m = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]) + b[j];
    const int chunk = j / D;
    mod[j] = (chunk == 0 || chunk == 2) ? 1.0f + m : tanhf(m);
  }
}

// The same product with 16-byte weight loads (W 16-byte aligned, 4D a
// multiple of 8): a workgroup owns 128 columns, lane c of each 16-lane group
// 8 consecutive columns, and the 16 groups take every 16th k; every load of a
// thread is independent, so they are all in flight together.  The 16 partial
// sums are added in a fixed order.
__device__ __forceinline__ void adaln_vec_block(int blk, const float* __restrict__ cond,
                                                const uint16_t* __restrict__ W, const float* __restrict__ b,
                                                float* __restrict__ mod, int C, int D, float (*part)[129]) {
  const int cg = (int)(threadIdx.x & 15);
  const int kg = (int)(threadIdx.x >> 4);
  const int j0 = blk * 128 + cg * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (j0 < 4 * D) {
#pragma unroll 4
    for (int k = kg; k < C; k += 16) {
      const uint4 w = *reinterpret_cast<const uint4*>(W + (size_t)k * 4 * D + j0);
      const float c = cond[k];
      const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += c * __uint_as_float(wv[i] << 16);
        acc[2 * i + 1] += c * __uint_as_float(wv[i] & 0xffff0000u);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) part[kg][cg * 8 + i] = acc[i];
  __syncthreads();
  if (threadIdx.x < 128) {
    const int j = blk * 128 + (int)threadIdx.x;
    if (j < 4 * D) {
      float m = b[j];
#pragma unroll
      for (int g = 0; g < 16; ++g) m += part[g][threadIdx.x];
      const int chunk = j / D;
      mod[j] = (chunk == 0 || chunk == 2) ? 1.0f + m : tanhf(m);
    }
  }
}

// RoPE table: tab[t][p] = (cos, sin) of coord[t][axis(p)] * theta^(-2*pair/width)
// for the 64 pairs of a 128-wide head; angles in binary64 (once per token,
// shared by every head).
__device__ __forceinline__ void rope_table_entry(int idx, const float* __restrict__ coords,
                                                 float2* __restrict__ tab, int T, float theta, int ax0, int ax1) {
  if (idx >= T * 64) return;
  const int t = idx >> 6;
  const int p = idx & 63;
  int axis, width, pair;
  if (p < ax0 / 2) {
    axis = 0; width = ax0; pair = p;
  } else if (p < (ax0 + ax1) / 2) {
    axis = 1; width = ax1; pair = p - ax0 / 2;
  } else {
    axis = 2; width = 128 - ax0 - ax1; pair = p - (ax0 + ax1) / 2;
  }
  const double freq = pow((double)theta, -2.0 * (double)pair / (double)width);
  const double angle = (double)coords[(size_t)t * 3 + axis] * freq;
  tab[idx] = make_float2((float)cos(angle), (float)sin(angle));
}

__global__ __launch_bounds__(256) void rope_table_kernel(const float* __restrict__ coords, float2* __restrict__ tab,
                                                         int T, float theta, int ax0, int ax1) {
  rope_table_entry((int)(blockIdx.x * blockDim.x + threadIdx.x), coords, tab, T, theta, ax0, ax1);
}

// The block's two independent set-up products in one launch (16-byte-aligned
// adaLN weights): workgroups below n_adaln take 128 adaLN columns each
// (adaln_vec_block), the rest 256 RoPE-table entries each.  Apart, the two
// took about 6 us each at C5, one after the other.
__global__ __launch_bounds__(256) void adaln_rope_kernel(const float* __restrict__ cond,
                                                         const uint16_t* __restrict__ W, const float* __restrict__ b,
                                                         float* __restrict__ mod, int C, int D, int n_adaln,
                                                         const float* __restrict__ coords, float2* __restrict__ tab,
                                                         int T, float theta, int ax0, int ax1) {
  __shared__ float part[16][129];
  const int blk = (int)blockIdx.x;
  if (blk < n_adaln)
    adaln_vec_block(blk, cond, W, b, mod, C, D, part);
  else
    rope_table_entry((blk - n_adaln) * 256 + (int)threadIdx.x, coords, tab, T, theta, ax0, ax1);
}

// Per (token, head): k RMSNorm over 128 channels, then RoPE on the
// interleaved pairs (2p, 2p+1) with the token's (cos, sin) table entry for
// pair p (zimage/canonical_contract.go:66-87, zimage_main_transformer_canonical.py:124-140).
// In place on the K part of the QKV projection, bf16 [T, 3D] (Q | K | V per
// token); the attention kernel applies the same norm (q_norm) and RoPE to Q as
// it loads it (launch_flash_attn_bf16_qnorm_rope), and V is left as it is.
// One wave per token: lane l takes the 16-byte chunks c = l + 64 j of the
// token's K row (c < 16 H): head c / 16, channels 8 (c % 16) .. +7, i.e. pairs
// 4 (l % 16) .. +3 of the head, so the lane's (cos, sin) entries and norm
// weights are the same for every chunk and are loaded once.  A head's sum of
// squares is reduced over its 16-lane group.  Up to 8 chunks (32 heads) are
// loaded before any arithmetic.
__global__ __launch_bounds__(256) void k_norm_rope_kernel(uint16_t* __restrict__ qkv, const float2* __restrict__ tab,
                                                          const float* __restrict__ kn, int T, int H, float eps) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  constexpr int kBatch = 8;
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int t = (int)blockIdx.x * 4 + wave;
  if (t >= T) return;  // the whole wave
  const int D = H * 128;
  const int nc = H * 16;
  const int sub = lane & 15;
  uint16_t* row = qkv + (size_t)t * 3 * D + D;
  float cs[4], sn[4], wk[8];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float2 e = tab[(size_t)t * 64 + 4 * sub + p];
    cs[p] = e.x;
    sn[p] = e.y;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) wk[i] = kn[8 * sub + i];
  auto norm_rope = [&](u32x4 v, const float* w) __attribute__((always_inline)) {
    float e[4], o[4];
    float ss = 0.0f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      e[p] = __uint_as_float(v[p] << 16);
      o[p] = __uint_as_float(v[p] & 0xffff0000u);
      ss += e[p] * e[p] + o[p] * o[p];
    }
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
    u32x4 r;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float ne = e[p] * inv * w[2 * p], no = o[p] * inv * w[2 * p + 1];
      r[p] = (uint32_t)f2bf(ne * cs[p] - no * sn[p]) | ((uint32_t)f2bf(ne * sn[p] + no * cs[p]) << 16);
    }
    return r;
  };
  for (int c0 = 0; c0 < nc; c0 += 64 * kBatch) {
    u32x4 kv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int c = c0 + lane + 64 * j;
      kv[j] = u32x4{0u, 0u, 0u, 0u};
      if (c < nc) kv[j] = *reinterpret_cast<const u32x4*>(row + 8 * c);
    }
    // c < nc holds for whole 16-lane groups (nc is a multiple of 16), so
    // every group's reduction sees only its own head
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int c = c0 + lane + 64 * j;
      const u32x4 kr = norm_rope(kv[j], wk);
      if (c < nc) *reinterpret_cast<u32x4*>(row + 8 * c) = kr;
    }
  }
}

// G [T, 2F] (w1 | w3) -> h [T, F] bf16: silu(g) * u (canonical_reference.go:457-460)
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ G, uint16_t* __restrict__ Hb, int T,
                                                     int F) {
  const int f4 = F >> 2;
  const size_t total = (size_t)T * f4;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
    const size_t t = idx / f4;
    const size_t i = idx - t * f4;
    const floatx4 g = reinterpret_cast<const floatx4*>(G + t * 2 * F)[i];
    const floatx4 u = reinterpret_cast<const floatx4*>(G + t * 2 * F + F)[i];
    floatx4 o;
    o.x = silu_mul(g.x, u.x);
    o.y = silu_mul(g.y, u.y);
    o.z = silu_mul(g.z, u.z);
    o.w = silu_mul(g.w, u.w);
    rows::store4(Hb + t * F + 4 * i, o);
  }
}

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

enum { kWsMod, kWsA, kWsQkv, kWsQ, kWsK, kWsV, kWsO, kWsProj, kWsR, kWsF, kWsG, kWsH, kWsW2, kWsRope, kWsCount };

// Rows of a K-blocked GEMM operand: every slice covers the GEMM's last tile row.
size_t blocked_rows(size_t T) { return (T + 255) & ~(size_t)255; }

size_t dit_workspace(const PrometheusDitBlockBf16Request* r, size_t off[kWsCount]) {
  const size_t T = r->tokens, D = r->hidden, F = r->ffn_hidden, Tb = blocked_rows(T);
  // A, O, F and H (the bf16 GEMMs' left operands) hold Tb rows so that they
  // can be K-blocked.
  const size_t sizes[kWsCount] = {4 * D * 4,  Tb * D * 2, T * 3 * D * 2, 0,             0,          0,
                                  Tb * D * 2, T * D * 4,  T * D * 4,     Tb * D * 2,    T * 2 * F * 4, Tb * F * 2,
                                  T * D * 4,  T * 64 * 8};
  size_t o = 0;
  for (int i = 0; i < kWsCount; ++i) {
    off[i] = o;
    o += align_up(sizes[i]);
  }
  return o;
}

int32_t validate_dit(const PrometheusDitBlockBf16Request* r) {
  if (r == nullptr || r->struct_size < sizeof(*r)) return PROM_BLOCK_DETAIL_INVALID_REQUEST;
  if (!r->input || !r->coordinates || !r->condition || !r->w_adaln || !r->b_adaln || !r->attn_norm1 ||
      !r->attn_norm2 || !r->ffn_norm1 || !r->ffn_norm2 || !r->q_norm || !r->k_norm || !r->w_qkv || !r->w_out ||
      !r->w_13 || !r->w_2 || !r->output)
    return PROM_BLOCK_DETAIL_INVALID_REQUEST;
  if (r->tokens == 0 || r->heads == 0 || r->cond_dim == 0 || r->ffn_hidden == 0) return PROM_BLOCK_DETAIL_SHAPE;
  if (r->head_dim != 128 || r->hidden != r->heads * 128 || r->hidden > 4096 || (r->ffn_hidden % 8) != 0)
    return PROM_BLOCK_DETAIL_UNSUPPORTED;
  if (r->rope_axes[0] + r->rope_axes[1] + r->rope_axes[2] != r->head_dim || (r->rope_axes[0] & 1) ||
      (r->rope_axes[1] & 1) || (r->rope_axes[2] & 1) || r->rope_axes[0] == 0 || r->rope_axes[1] == 0 ||
      r->rope_axes[2] == 0)
    return PROM_BLOCK_DETAIL_SHAPE;
  if (!isfinite(r->rms_epsilon) || r->rms_epsilon <= 0.f || !isfinite(r->rope_theta) || r->rope_theta <= 0.f)
    return PROM_BLOCK_DETAIL_INVALID_REQUEST;
  const uint64_t lim = 1ull << 31;
  if ((uint64_t)r->tokens * 2 * r->ffn_hidden >= lim || (uint64_t)r->tokens * 3 * r->hidden >= lim)
    return PROM_BLOCK_DETAIL_SHAPE;
  return 0;
}

hipError_t enqueue_dit(const PrometheusDitBlockBf16Request* r, char* ws, const size_t off[kWsCount], hipStream_t st,
                       uint32_t* launches) {
  const int T = (int)r->tokens, D = (int)r->hidden, H = (int)r->heads, F = (int)r->ffn_hidden, C = (int)r->cond_dim;
  const float eps = r->rms_epsilon;
  float* mod = reinterpret_cast<float*>(ws + off[kWsMod]);
  uint16_t* A = reinterpret_cast<uint16_t*>(ws + off[kWsA]);
  uint16_t* qkv = reinterpret_cast<uint16_t*>(ws + off[kWsQkv]);  // bf16 [T, 3D]
  uint16_t* O = reinterpret_cast<uint16_t*>(ws + off[kWsO]);
  uint16_t* projb = reinterpret_cast<uint16_t*>(ws + off[kWsProj]);
  float* R = reinterpret_cast<float*>(ws + off[kWsR]);
  uint16_t* Fb = reinterpret_cast<uint16_t*>(ws + off[kWsF]);
  float* G = reinterpret_cast<float*>(ws + off[kWsG]);
  uint16_t* Hb = reinterpret_cast<uint16_t*>(ws + off[kWsH]);
  uint16_t* w2b = reinterpret_cast<uint16_t*>(ws + off[kWsW2]);
  float2* rope = reinterpret_cast<float2*>(ws + off[kWsRope]);
  const float* scaleA = mod;
  const float* gateA = mod + D;
  const float* scaleM = mod + 2 * D;
  const float* gateM = mod + 3 * D;
  hipError_t e;
  uint32_t n = 0;
#define PROM_STEP(call)            \
  do {                             \
    e = (call);                    \
    if (e != hipSuccess) return e; \
    ++n;                           \
  } while (0)
  const dim3 blk(256);
  if ((reinterpret_cast<uintptr_t>(r->w_adaln) & 15u) == 0 && (4 * D) % 8 == 0) {
    const int n_adaln = (4 * D + 127) / 128;
    hipLaunchKernelGGL(adaln_rope_kernel, dim3((unsigned)(n_adaln + (T * 64 + 255) / 256)), blk, 0, st, r->condition,
                       r->w_adaln, r->b_adaln, mod, C, D, n_adaln, r->coordinates, rope, T, r->rope_theta,
                       (int)r->rope_axes[0], (int)r->rope_axes[1]);
    PROM_STEP(hipGetLastError());
  } else {
    hipLaunchKernelGGL(adaln_kernel, dim3((4 * D + 63) / 64), blk, 0, st, r->condition, r->w_adaln, r->b_adaln, mod, C,
                       D);
    PROM_STEP(hipGetLastError());
    hipLaunchKernelGGL(rope_table_kernel, dim3((T * 64 + 255) / 256), blk, 0, st, r->coordinates, rope, T,
                       r->rope_theta, (int)r->rope_axes[0], (int)r->rope_axes[1]);
    PROM_STEP(hipGetLastError());
  }
  // Each GEMM that runs on the four-stage kernel reads its left operand
  // K-blocked ([K/32][Tb][32]: whole 128-byte lines per transfer, 4096^3
  // 109 -> 105.5 us), written so by the kernel that produces it; the others
  // read rows.  The values and their order are the same either way.
  const int Tb = (int)blocked_rows((size_t)T);
  const int qkv_slice = gemm_bf16_takes_blocked_a(A, D, r->w_qkv, 3 * D, T, 3 * D, D) ? Tb : 0;
  const int o_slice = gemm_bf16_takes_blocked_a(O, D, r->w_out, D, T, D, D) ? Tb : 0;
  const int f_slice = gemm_bf16_swiglu_takes_blocked_a(Fb, D, r->w_13, T, F, D) ? Tb : 0;
  const int h_slice = f_slice > 0 && gemm_bf16_takes_blocked_a(Hb, F, r->w_2, D, T, D, F) ? Tb : 0;
  hipLaunchKernelGGL(rows::norm_mod_kernel<uint16_t>, rows::row_groups<4>(T), dim3(256), 0, st, r->input,
                     r->attn_norm1, scaleA, A, T, D, eps, qkv_slice);
  PROM_STEP(hipGetLastError());
  // QKV in bf16 (one rounding before the per-head norms), K's norm and RoPE in
  // place, Q's inside the attention, which reads Q, K, V from the [T, 3D] rows.
  PROM_STEP(launch_gemm_bf16_ex(A, D, r->w_qkv, 3 * D, nullptr, qkv, 3 * D, T, 3 * D, D, nullptr, 0, st, nullptr,
                                qkv_slice));
  hipLaunchKernelGGL(k_norm_rope_kernel, dim3((T + 3) / 4), blk, 0, st, qkv, rope, r->k_norm, T, H, eps);
  PROM_STEP(hipGetLastError());
  PROM_STEP(launch_flash_attn_bf16_qnorm_rope(qkv, 3 * D, qkv + D, 3 * D, qkv + 2 * D, 3 * D, O, D, T, H,
                                              1.0f / sqrtf(128.0f), rope, r->q_norm, r->k_norm, eps, st, o_slice));
  // The out- and down-projections go to bf16: both are RMS-normalised before
  // they join the fp32 residual stream.
  PROM_STEP(launch_gemm_bf16_ex(O, D, r->w_out, D, nullptr, projb, D, T, D, D, nullptr, 0, st, nullptr, o_slice));
  // 149 VGPRs allow 3 waves per SIMD, so one 12-wave workgroup per CU: 352
  // workgroups at T = 4224 run in two rounds, where 8-row workgroups (one per
  // CU as well) took three, the last with 16 (45 -> 37.5 us).  R is next read
  // after the FFN GEMMs and the block output by the next block's first
  // kernel: both go out as streaming stores (W1|W3 -4 us, the first row
  // kernel -1.3, this one -1.2).
  hipLaunchKernelGGL((rows::resid_norm_mod_kernel<uint16_t, 12, uint16_t, true>), rows::row_groups<12>(T), dim3(768), 0, st, r->input, projb, r->attn_norm2, gateA, r->ffn_norm1, scaleM,
                     R, Fb, T, D, eps, f_slice);
  PROM_STEP(hipGetLastError());
  // FFN up-projection with SwiGLU fused into the GEMM epilogue when the shape
  // allows (F a multiple of 128, D of 64); otherwise GEMM to fp32, then SwiGLU.
  // (G, unused on the fused path, takes the K-slice sums of a final partial wave.)
  uint32_t k13 = 1;
  const hipError_t fused =
      launch_gemm_bf16_swiglu(Fb, D, r->w_13, Hb, F, T, F, D, st, G, (size_t)T * 2 * F * sizeof(float), &k13,
                              f_slice, h_slice);
  if (fused == hipErrorNotSupported) {
    PROM_STEP(launch_gemm_bf16_ex(Fb, D, r->w_13, 2 * F, G, nullptr, 2 * F, T, 2 * F, D, nullptr, 0, st, nullptr));
    const size_t total = (size_t)T * (F / 4);
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)std::min((size_t)65536, (total + 255) / 256)), blk, 0, st, G, Hb,
                       T, F);
    PROM_STEP(hipGetLastError());
  } else {
    PROM_STEP(fused);
    n += k13 - 1;
  }
  PROM_STEP(launch_gemm_bf16_ex(Hb, F, r->w_2, D, nullptr, w2b, D, T, D, F, nullptr, 0, st, nullptr, h_slice));
  hipLaunchKernelGGL((rows::final_resid_kernel<4, uint16_t, true>), rows::row_groups<4>(T), dim3(256), 0, st, R, w2b, r->ffn_norm2, gateM, r->output, T, D, eps);
  PROM_STEP(hipGetLastError());
#undef PROM_STEP
  if (launches) *launches = n;
  return hipSuccess;
}

void result_init(PrometheusBlockResult* res) {
  memset(res, 0, sizeof(*res));
  res->struct_size = sizeof(*res);
}

}  // namespace
}  // namespace prom

using namespace prom;

extern "C" {

PROM_REACTOR_API int prometheus_reactor_runtime_dit_block_bf16_device(void* handle,
                                                                      const PrometheusDitBlockBf16Request* request,
                                                                      PrometheusBlockResult* out_result) {
  PrometheusBlockResult local;
  PrometheusBlockResult* res = out_result ? out_result : &local;
  result_init(res);
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    res->stage = PROM_STAGE_INIT;
    res->detail_code = PROM_INVALID_HANDLE;
    return PROM_INVALID_HANDLE;
  }
  const int32_t d = validate_dit(request);
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
  size_t off[kWsCount];
  const size_t ws_bytes = dit_workspace(request, off);
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
  if (enqueue_dit(request, ws, off, cx.stream, &launches) != hipSuccess) {
    res->stage = PROM_STAGE_SUBMIT;
    res->detail_code = PROM_DETAIL_HIP_LAUNCH_FAILED;
    return PROM_ERROR;
  }
  res->kernel_launches = launches;
  res->stage = PROM_STAGE_SUBMIT;
  res->detail_code = PROM_DETAIL_PATH_HIP_MFMA_BF16;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_dit_block_bf16(void* handle, const PrometheusDitBlockBf16Request* request,
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
  const int32_t d = validate_dit(request);
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
  const PrometheusDitBlockBf16Request& r = *request;
  const size_t T = r.tokens, D = r.hidden, F = r.ffn_hidden, C = r.cond_dim;
  // Host arrays: byte sizes in request order.
  const void* srcs[16] = {r.input,     r.coordinates, r.condition, r.w_adaln, r.b_adaln, r.attn_norm1,
                          r.attn_norm2, r.ffn_norm1,  r.ffn_norm2, r.q_norm,  r.k_norm,  r.w_qkv,
                          r.w_out,     r.w_13,        r.w_2,       nullptr};
  const size_t bytes[16] = {T * D * 4, T * 3 * 4, C * 4, C * 4 * D * 2, 4 * D * 4, D * 4, D * 4, D * 4, D * 4,
                            128 * 4,   128 * 4,   D * 3 * D * 2, D * D * 2, D * 2 * F * 2, F * D * 2, T * D * 4};
  size_t offs[16], total = 0;
  for (int i = 0; i < 16; ++i) {
    offs[i] = total;
    total += align_up(bytes[i]);
  }
  size_t woff[kWsCount];
  const size_t ws_bytes = dit_workspace(request, woff);
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
  for (int i = 0; i < 15; ++i) {
    if (upload_host(dev + offs[i], srcs[i], bytes[i], cx.stream) != hipSuccess) {
      res->detail_code = PROM_DETAIL_HIP_COPY_FAILED;
      return PROM_ERROR;
    }
  }
  PrometheusDitBlockBf16Request dr = r;
  dr.input = reinterpret_cast<const float*>(dev + offs[0]);
  dr.coordinates = reinterpret_cast<const float*>(dev + offs[1]);
  dr.condition = reinterpret_cast<const float*>(dev + offs[2]);
  dr.w_adaln = reinterpret_cast<const uint16_t*>(dev + offs[3]);
  dr.b_adaln = reinterpret_cast<const float*>(dev + offs[4]);
  dr.attn_norm1 = reinterpret_cast<const float*>(dev + offs[5]);
  dr.attn_norm2 = reinterpret_cast<const float*>(dev + offs[6]);
  dr.ffn_norm1 = reinterpret_cast<const float*>(dev + offs[7]);
  dr.ffn_norm2 = reinterpret_cast<const float*>(dev + offs[8]);
  dr.q_norm = reinterpret_cast<const float*>(dev + offs[9]);
  dr.k_norm = reinterpret_cast<const float*>(dev + offs[10]);
  dr.w_qkv = reinterpret_cast<const uint16_t*>(dev + offs[11]);
  dr.w_out = reinterpret_cast<const uint16_t*>(dev + offs[12]);
  dr.w_13 = reinterpret_cast<const uint16_t*>(dev + offs[13]);
  dr.w_2 = reinterpret_cast<const uint16_t*>(dev + offs[14]);
  dr.output = reinterpret_cast<float*>(dev + offs[15]);
  res->stage = PROM_STAGE_SUBMIT;
  uint32_t launches = 0;
  (void)hipEventRecord(cx.op_begin, cx.stream);
  if (enqueue_dit(&dr, ws, woff, cx.stream, &launches) != hipSuccess) {
    (void)hipStreamSynchronize(cx.stream);
    res->detail_code = PROM_DETAIL_HIP_LAUNCH_FAILED;
    return PROM_ERROR;
  }
  (void)hipEventRecord(cx.op_end, cx.stream);
  res->stage = PROM_STAGE_TRANSFER_OUT;
  if (download_host(r.output, dr.output, bytes[15], cx.stream) != hipSuccess ||
      hipStreamSynchronize(cx.stream) != hipSuccess) {
    res->detail_code = PROM_DETAIL_HIP_COPY_FAILED;
    return PROM_ERROR;
  }
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, cx.op_begin, cx.op_end) == hipSuccess) res->gpu_duration_ns = (uint64_t)(ms * 1.0e6);
  res->kernel_launches = launches;
  res->workspace_bytes = ws_bytes;
  res->detail_code = PROM_DETAIL_PATH_HIP_MFMA_BF16;
  res->output_written = 1;
  res->end_to_end_ns = wall_ns() - t0;
  return PROM_OK;
}

}  // extern "C"
