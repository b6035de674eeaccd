// FP32 SGEMM on CDNA4 MFMA (v_mfma_f32_32x32x2_f32) and the HBM-bound GEMV.
//
// Computes C[m,n] = A[m,k] @ B[k,n], row-major fp32: the arithmetic of Oct's
// `@` inside PROMETHEUS { } (internal/prometheus/runtime.go:298-331, C ABI
// internal/prometheus/native/reactor_api.h:2587-2595).  The reference's
// Vulkan kernels (e.g. sgemm_reg2x2_tile16x16_exacttail_fp32.sdslv:49-190)
// are FMA loops on 8x8 threads; this is a different design built for the
// matrix cores:
//
//   * workgroup = 256 threads = 4 wave64, macro tile 128x256, K tile 16;
//     each wave owns a 64x128 sub-tile = 2x4 MFMA 32x32 blocks (128 fp32
//     accumulators per lane; 6 LDS reads per 8 MFMAs);
//   * A and B are staged through LDS, double-buffered: the next K tile is
//     fetched into registers while the current one feeds the MFMAs, then
//     written to the other LDS buffer; one barrier per K tile;
//   * A is transposed on its way into LDS (k-major) so that every MFMA
//     operand read is 32 consecutive floats per half-wave;
//   * exact tails: out-of-range rows/columns/k are zero-filled on load and
//     masked on store, no host padding.  Shapes whose k and n are multiples
//     of 4 use 128-bit global loads; others use predicated 32-bit loads;
//   * workgroup -> tile mapping is XCD-aware: hardware deals workgroups to
//     the 8 XCDs round-robin, so consecutive ids are remapped to contiguous
//     chunks of a grouped (GROUP_M) tile order, keeping each XCD's L2 on a
//     compact block of A rows and B columns.
#include <algorithm>

#include "reactor_internal.h"

namespace prom {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 256;
constexpr int kBK = 16;
constexpr int kLdsA = kBM + 2;  // k-major A rows; +2 keeps the transposing stores conflict-free
constexpr int kLdsB = kBN + 4;  // k-major B rows; multiple of 4 for 128-bit stores
constexpr int kGroupM = 8;

__device__ __forceinline__ void map_tile(int tiles_m, int tiles_n, int* tm, int* tn) {
  const int num_tiles = tiles_m * tiles_n;
  int pid = (int)blockIdx.x;
  if ((num_tiles & 7) == 0) pid = (pid & 7) * (num_tiles >> 3) + (pid >> 3);
  const int per_group = kGroupM * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroupM;
  const int group_m = min(tiles_m - first_m, kGroupM);
  const int in_group = pid - group * per_group;
  *tm = first_m + in_group % group_m;
  *tn = in_group / group_m;
}

// Strides are leading dimensions in elements.  R (may be null) is added in the
// epilogue: C = A @ B + R; R may alias C (each element is read, then written,
// by the same lane).
template <bool kVec, bool kBuf>
__global__ __launch_bounds__(256, 2) void sgemm_f32_mfma_kernel(const float* __restrict__ A,
                                                                const float* __restrict__ B, float* C, int M,
                                                                int N, int K, int tiles_m, int tiles_n, int lda,
                                                                int ldb, int ldc, const float* R, int ldr,
                                                                int k_len, long long sa, long long sb, long long sc) {
  __shared__ float As[2][kBK][kLdsA];
  __shared__ float Bs[2][kBK][kLdsB];

  // Batched launches (gridDim.z > 1, never split-K): matrix z of A, B and C
  // starts sa, sb and sc elements after the previous one.
  if (gridDim.z > 1) {
    A += (size_t)blockIdx.z * sa;
    B += (size_t)blockIdx.z * sb;
    C += (size_t)blockIdx.z * sc;
  }
  int tm, tn;
  map_tile(tiles_m, tiles_n, &tm, &tn);
  const int row0 = tm * kBM;
  const int col0 = tn * kBN;
  // Split-K: slice blockIdx.y covers k in [y*k_len, y*k_len + k_len) and writes
  // its partial product to slab y of C (slabs M*ldc apart); R is then null.
  if (gridDim.y > 1) {
    const int kb = (int)blockIdx.y * k_len;
    A += kb;
    B += (size_t)kb * ldb;
    C += (size_t)blockIdx.y * M * ldc;
    K = min(k_len, K - kb);
  }

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;

  // Global->register assignment: A: one row, 8 consecutive k;
  // B: k rows tid/64 + {0,4,8,12}, 4 consecutive n at (tid%64)*4.
  const int a_row = tid >> 1;
  const int a_k = (tid & 1) * 8;
  const int b_k = tid >> 6;
  const int b_n = (tid & 63) * 4;

  float ra[8];
  float rb[16];
  // Branch-free loads (kBuf: K of this slice is a multiple of the K tile): buffer
  // loads return zero for rows of A at or past M and past the end of B; columns of
  // B at or past N only feed output columns that are never stored.
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      (void*)A, (short)0, kBuf ? (int)(((size_t)M * lda - (gridDim.y > 1 ? (size_t)blockIdx.y * k_len : 0)) * 4) : 0,
      0x00020000);
  const __amdgpu_buffer_rsrc_t rsb =
      __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, kBuf ? (int)((size_t)K * ldb * 4) : 0, 0x00020000);

  auto load_tile = [&](int k0) {
    const int gr = row0 + a_row;
    const int gn = col0 + b_n;
    if constexpr (kBuf) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int gk = k0 + a_k + 4 * h;
        const floatx4 v =
            __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rsa, (uint32_t)((gr * lda + gk) * 4), 0, 0));
        ra[4 * h + 0] = v.x;
        ra[4 * h + 1] = v.y;
        ra[4 * h + 2] = v.z;
        ra[4 * h + 3] = v.w;
      }
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int gk = k0 + b_k + 4 * h;
        const floatx4 v =
            __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rsb, (uint32_t)((gk * ldb + gn) * 4), 0, 0));
        rb[4 * h + 0] = v.x;
        rb[4 * h + 1] = v.y;
        rb[4 * h + 2] = v.z;
        rb[4 * h + 3] = v.w;
      }
    } else if constexpr (kVec) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int gk = k0 + a_k + 4 * h;
        floatx4 v = {0.f, 0.f, 0.f, 0.f};
        if (gr < M && gk < K) v = *reinterpret_cast<const floatx4*>(A + (size_t)gr * lda + gk);
        ra[4 * h + 0] = v.x;
        ra[4 * h + 1] = v.y;
        ra[4 * h + 2] = v.z;
        ra[4 * h + 3] = v.w;
      }
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int gk = k0 + b_k + 4 * h;
        floatx4 v = {0.f, 0.f, 0.f, 0.f};
        if (gk < K && gn < N) v = *reinterpret_cast<const floatx4*>(B + (size_t)gk * ldb + gn);
        rb[4 * h + 0] = v.x;
        rb[4 * h + 1] = v.y;
        rb[4 * h + 2] = v.z;
        rb[4 * h + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int gk = k0 + a_k + j;
        ra[j] = (gr < M && gk < K) ? A[(size_t)gr * lda + gk] : 0.f;
      }
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int gk = k0 + b_k + 4 * h;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          rb[4 * h + j] = (gk < K && gn + j < N) ? B[(size_t)gk * ldb + gn + j] : 0.f;
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 8; ++j) As[buf][a_k + j][a_row] = ra[j];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      floatx4 v = {rb[4 * h + 0], rb[4 * h + 1], rb[4 * h + 2], rb[4 * h + 3]};
      *reinterpret_cast<floatx4*>(&Bs[buf][b_k + 4 * h][b_n]) = v;
    }
  };

  floatx16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx16{};

  const int k_tiles = (K + kBK - 1) / kBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int lrow = lane & 31;
  const int lk = lane >> 5;
  const int am = wm * 64 + lrow;
  const int bn = wn * 128 + lrow;

  for (int kt = 0; kt < k_tiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < k_tiles;
    if (more) load_tile((kt + 1) * kBK);
#pragma unroll
    for (int s = 0; s < kBK / 2; ++s) {
      const int kr = 2 * s + lk;
      float a[2], b[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[cur][kr][am + 32 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[cur][kr][bn + 32 * j];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Accumulator layout of a 32x32 MFMA block: lane l, register r holds
  // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  auto store_block = [&](const floatx16& acc, int mi, int ni) {
    const int col = col0 + wn * 128 + ni * 32 + lrow;
    if (col >= N) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + wm * 64 + mi * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
      if (row < M) {
        float v = acc[r];
        if (R != nullptr) v += R[(size_t)row * ldr + col];
        C[(size_t)row * ldc + col] = v;
      }
    }
  };
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) store_block(acc[i][j], i, j);
}

// y[m] = A[m,:] . x : one wave per row, 4 rows per workgroup.  HBM-bound:
// every byte of A is read once with 128-bit loads, x stays in L2.
template <bool kVec>
__global__ __launch_bounds__(256) void gemv_f32_kernel(const float* __restrict__ A, const float* __restrict__ x,
                                                       float* __restrict__ y, int M, int K) {
  const int wave = (int)(threadIdx.x >> 6);
  const int lane = (int)(threadIdx.x & 63);
  const int row = (int)blockIdx.x * 4 + wave;
  if (row >= M) return;
  const float* a = A + (size_t)row * K;
  float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
  if constexpr (kVec) {
    const int k4 = K >> 2;
    const floatx4* a4 = reinterpret_cast<const floatx4*>(a);
    const floatx4* x4 = reinterpret_cast<const floatx4*>(x);
    int i = lane;
    for (; i + 192 < k4; i += 256) {
      const floatx4 p0 = a4[i], p1 = a4[i + 64], p2 = a4[i + 128], p3 = a4[i + 192];
      const floatx4 q0 = x4[i], q1 = x4[i + 64], q2 = x4[i + 128], q3 = x4[i + 192];
      acc0 += p0.x * q0.x + p0.y * q0.y + p0.z * q0.z + p0.w * q0.w;
      acc1 += p1.x * q1.x + p1.y * q1.y + p1.z * q1.z + p1.w * q1.w;
      acc2 += p2.x * q2.x + p2.y * q2.y + p2.z * q2.z + p2.w * q2.w;
      acc3 += p3.x * q3.x + p3.y * q3.y + p3.z * q3.z + p3.w * q3.w;
    }
    for (; i < k4; i += 64) {
      const floatx4 p = a4[i], q = x4[i];
      acc0 += p.x * q.x + p.y * q.y + p.z * q.z + p.w * q.w;
    }
  } else {
    for (int i = lane; i < K; i += 64) acc0 += a[i] * x[i];
  }
  float acc = (acc0 + acc1) + (acc2 + acc3);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) y[row] = acc;
}

// C = sum over `splits` slabs of P (fixed order: deterministic) + R.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ P, float* C, int M, int N,
                                                            int ldc, int splits, const float* R, int ldr) {
  const size_t total = (size_t)M * N;
  const size_t slab = (size_t)M * N;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
    const size_t row = idx / N;
    const size_t col = idx - row * N;
    float v = P[idx];
    for (int s = 1; s < splits; ++s) v += P[(size_t)s * slab + idx];
    if (R != nullptr) v += R[row * ldr + col];
    C[row * ldc + col] = v;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Number of K slices.  2 workgroups per CU make 512 concurrent slots; a grid
// of w workgroups runs in ceil(w / 512) rounds, each as long as one slice's
// K tiles (~4 us per 128x256x16 tile step at full rate, plus ~2 us of
// prologue and epilogue).  Slicing adds the reduce launch (~8 us) and
// (2s + 1) M N floats of partial-sum traffic (~3 TB/s effective).  The count
// minimising this estimate is chosen, with slices at least 128 deep and at
// most 16 of them.
int choose_splits(int tiles, uint32_t m, uint32_t n, uint32_t k) {
  const int k_tiles = (int)((k + kBK - 1) / kBK);
  auto cost = [&](int s) {
    const int per = (k_tiles + s - 1) / s;
    const double rounds = (double)(((size_t)tiles * s + 511) / 512);
    const double reduce = s == 1 ? 0.0 : 8.0 + (double)(2 * s + 1) * m * n * 4.0 / 3.0e6;
    return rounds * (per * 4.0 + 2.0) + reduce;
  };
  int best = 1;
  double best_cost = cost(1);
  for (int s = 2; s <= 16 && k / (uint32_t)s >= 128; ++s) {
    const double c = cost(s);
    if (c < best_cost) {
      best_cost = c;
      best = s;
    }
  }
  return best;
}

}  // namespace

hipError_t launch_sgemm_f32_ex(const float* a, int lda, const float* b, int ldb, float* c, int ldc, uint32_t m,
                               uint32_t n, uint32_t k, const float* residual, int ldr, hipStream_t stream,
                               int* path_detail) {
  if (n == 1 && residual == nullptr && ldb == 1 && lda == (int)k) {
    const bool vec = (k % 4 == 0) && aligned16(a) && aligned16(b);
    const dim3 grid((m + 3) / 4);
    if (vec)
      hipLaunchKernelGGL(gemv_f32_kernel<true>, grid, dim3(256), 0, stream, a, b, c, (int)m, (int)k);
    else
      hipLaunchKernelGGL(gemv_f32_kernel<false>, grid, dim3(256), 0, stream, a, b, c, (int)m, (int)k);
    if (path_detail) *path_detail = PROM_DETAIL_PATH_HIP_GEMV_F32;
    return hipGetLastError();
  }
  const int tiles_m = (int)((m + kBM - 1) / kBM);
  const int tiles_n = (int)((n + kBN - 1) / kBN);
  const bool vec = (k % 4 == 0) && (n % 4 == 0) && (lda % 4 == 0) && (ldb % 4 == 0) && aligned16(a) && aligned16(b);
  int splits = choose_splits(tiles_m * tiles_n, m, n, k);
  int k_len = (int)k;
  float* partial = nullptr;
  if (splits > 1) {
    // slices are whole K tiles (multiples of 16 keep 128-bit loads aligned)
    k_len = (int)((((k + splits - 1) / splits) + kBK - 1) / kBK * kBK);
    splits = (int)((k + k_len - 1) / k_len);
    partial = splits > 1 ? static_cast<float*>(staging(6, (size_t)splits * m * n * sizeof(float))) : nullptr;
    if (partial == nullptr) {
      splits = 1;
      k_len = (int)k;
    }
  }
  const dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)splits);
  float* out = splits > 1 ? partial : c;
  const int ldo = splits > 1 ? (int)n : ldc;
  const float* res = splits > 1 ? nullptr : residual;
  // Buffer-load path: every slice length a multiple of the K tile and every
  // 32-bit byte offset (rows up to M + kBM, all of B plus a tile row) in range.
  const bool buf = vec && (k % kBK == 0) && (k_len % kBK == 0) &&
                   (size_t)(m + kBM) * lda * 4 < (1ull << 31) && ((size_t)k * ldb + n + kBN) * 4 < (1ull << 31);
  if (buf)
    hipLaunchKernelGGL((sgemm_f32_mfma_kernel<true, true>), grid, dim3(256), 0, stream, a, b, out, (int)m, (int)n,
                       (int)k, tiles_m, tiles_n, lda, ldb, ldo, res, ldr, k_len, 0ll, 0ll, 0ll);
  else if (vec)
    hipLaunchKernelGGL((sgemm_f32_mfma_kernel<true, false>), grid, dim3(256), 0, stream, a, b, out, (int)m, (int)n,
                       (int)k, tiles_m, tiles_n, lda, ldb, ldo, res, ldr, k_len, 0ll, 0ll, 0ll);
  else
    hipLaunchKernelGGL((sgemm_f32_mfma_kernel<false, false>), grid, dim3(256), 0, stream, a, b, out, (int)m, (int)n,
                       (int)k, tiles_m, tiles_n, lda, ldb, ldo, res, ldr, k_len, 0ll, 0ll, 0ll);
  if (splits > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t total = (size_t)m * n;
    const unsigned blocks = (unsigned)std::min((size_t)8192, (total + 255) / 256);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, partial, c, (int)m, (int)n, ldc,
                       splits, residual, ldr);
  }
  if (path_detail) *path_detail = PROM_DETAIL_PATH_HIP_MFMA_F32;
  return hipGetLastError();
}

hipError_t launch_sgemm_f32_batched(const float* a, int lda, long long sa, const float* b, int ldb, long long sb,
                                    float* c, int ldc, long long sc, uint32_t m, uint32_t n, uint32_t k,
                                    uint32_t batch, hipStream_t stream) {
  if (batch == 0 || m == 0 || n == 0) return hipSuccess;
  if (batch == 1) return launch_sgemm_f32_ex(a, lda, b, ldb, c, ldc, m, n, k, nullptr, 0, stream, nullptr);
  const int tiles_m = (int)((m + kBM - 1) / kBM);
  const int tiles_n = (int)((n + kBN - 1) / kBN);
  const bool vec = (k % 4 == 0) && (n % 4 == 0) && (lda % 4 == 0) && (ldb % 4 == 0) && (sa % 4 == 0) &&
                   (sb % 4 == 0) && aligned16(a) && aligned16(b);
  // Per-matrix extents bound every buffer offset, as in the single launch.
  const bool buf = vec && (k % kBK == 0) && (size_t)(m + kBM) * lda * 4 < (1ull << 31) &&
                   ((size_t)k * ldb + n + kBN) * 4 < (1ull << 31);
  const dim3 grid((unsigned)(tiles_m * tiles_n), 1u, batch);
  if (buf)
    hipLaunchKernelGGL((sgemm_f32_mfma_kernel<true, true>), grid, dim3(256), 0, stream, a, b, c, (int)m, (int)n,
                       (int)k, tiles_m, tiles_n, lda, ldb, ldc, (const float*)nullptr, 0, (int)k, sa, sb, sc);
  else if (vec)
    hipLaunchKernelGGL((sgemm_f32_mfma_kernel<true, false>), grid, dim3(256), 0, stream, a, b, c, (int)m, (int)n,
                       (int)k, tiles_m, tiles_n, lda, ldb, ldc, (const float*)nullptr, 0, (int)k, sa, sb, sc);
  else
    hipLaunchKernelGGL((sgemm_f32_mfma_kernel<false, false>), grid, dim3(256), 0, stream, a, b, c, (int)m, (int)n,
                       (int)k, tiles_m, tiles_n, lda, ldb, ldc, (const float*)nullptr, 0, (int)k, sa, sb, sc);
  return hipGetLastError();
}

hipError_t launch_sgemm_f32(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                            hipStream_t stream, int* path_detail) {
  return launch_sgemm_f32_ex(a, (int)k, b, (int)n, c, (int)n, m, n, k, nullptr, 0, stream, path_detail);
}

}  // namespace prom
