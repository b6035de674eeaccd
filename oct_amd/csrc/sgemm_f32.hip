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
#include <cmath>
#include <cstddef>
#include <cstring>
#include <type_traits>

#include "reactor_internal.h"

namespace prom {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 16;
constexpr int kGroupM = 8;

// xcd_pid gives each XCD a contiguous range of tile ids, so the tiles an XCD
// runs together are neighbours in the grouped order and share their A and B
// panels in its L2.
__device__ __forceinline__ void map_tile(int tiles_m, int tiles_n, int* tm, int* tn) {
  const int num_tiles = tiles_m * tiles_n;
  const int pid = xcd_pid((int)blockIdx.x, num_tiles);
  const int per_group = kGroupM * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroupM;
  const int group_m = min(tiles_m - first_m, kGroupM);
  const int in_group = pid - group * per_group;
  *tm = first_m + in_group % group_m;
  *tn = in_group / group_m;
}

// Macro tile kBM x kBN (kBM in {64, 128}, kBN in {128, 256}); the four waves
// form a 2x2 grid, each owning (kBM/2) x (kBN/2) = kMI x kNI MFMA 32x32 blocks.
// Occupancy: 2 workgroups per CU for 128x256 (198 VGPRs), more for the
// smaller tiles.
template <int kBM, int kBN>
struct TileCfg {
  static constexpr int kMI = kBM / 64;
  static constexpr int kNI = kBN / 64;
  static constexpr int kLdsA = kBM + 2;  // k-major A rows; +2 keeps the transposing stores conflict-free
  static constexpr int kLdsB = kBN + 4;  // k-major B rows; multiple of 4 for 128-bit stores
  static constexpr int kAPer = kBM / 16;            // A floats per thread per K tile (one row, consecutive k)
  static constexpr int kAThreadsPerRow = 16 / kAPer;
  static constexpr int kBVec = kBN / 64;            // B float4s per thread per K tile
  static constexpr int kBRowStep = 1024 / kBN;      // K rows between a thread's float4s
};

// Strides are leading dimensions in elements.  R (may be null) is added in the
// epilogue: C = A @ B + R; R may alias C (each element is read, then written,
// by the same lane).
template <bool kVec, bool kBuf, int kBM, int kBN>
__global__ __launch_bounds__(256, (kBM * kBN >= 128 * 256 ? 2 : 3)) void sgemm_f32_mfma_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* C, int M, int N, int K, int tiles_m,
    int tiles_n, int lda, int ldb, int ldc, const float* R, int ldr, int k_len, long long sa, long long sb,
    long long sc) {
  using T = TileCfg<kBM, kBN>;
  __shared__ float As[2][kBK][T::kLdsA];
  __shared__ float Bs[2][kBK][T::kLdsB];

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

  // Global->register assignment: A: one row, kAPer consecutive k;
  // B: k rows b_k + kBRowStep*h, 4 consecutive n at b_n.
  const int a_row = tid / T::kAThreadsPerRow;
  const int a_k = (tid % T::kAThreadsPerRow) * T::kAPer;
  const int b_k = tid / (kBN / 4);
  const int b_n = (tid % (kBN / 4)) * 4;

  float ra[T::kAPer];
  float rb[4 * T::kBVec];
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
      for (int h = 0; h < T::kAPer / 4; ++h) {
        const int gk = k0 + a_k + 4 * h;
        const floatx4 v =
            __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rsa, (uint32_t)((gr * lda + gk) * 4), 0, 0));
        ra[4 * h + 0] = v.x;
        ra[4 * h + 1] = v.y;
        ra[4 * h + 2] = v.z;
        ra[4 * h + 3] = v.w;
      }
#pragma unroll
      for (int h = 0; h < T::kBVec; ++h) {
        const int gk = k0 + b_k + T::kBRowStep * h;
        const floatx4 v =
            __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rsb, (uint32_t)((gk * ldb + gn) * 4), 0, 0));
        rb[4 * h + 0] = v.x;
        rb[4 * h + 1] = v.y;
        rb[4 * h + 2] = v.z;
        rb[4 * h + 3] = v.w;
      }
    } else if constexpr (kVec) {
#pragma unroll
      for (int h = 0; h < T::kAPer / 4; ++h) {
        const int gk = k0 + a_k + 4 * h;
        floatx4 v = {0.f, 0.f, 0.f, 0.f};
        if (gr < M && gk < K) v = *reinterpret_cast<const floatx4*>(A + (size_t)gr * lda + gk);
        ra[4 * h + 0] = v.x;
        ra[4 * h + 1] = v.y;
        ra[4 * h + 2] = v.z;
        ra[4 * h + 3] = v.w;
      }
#pragma unroll
      for (int h = 0; h < T::kBVec; ++h) {
        const int gk = k0 + b_k + T::kBRowStep * h;
        floatx4 v = {0.f, 0.f, 0.f, 0.f};
        if (gk < K && gn < N) v = *reinterpret_cast<const floatx4*>(B + (size_t)gk * ldb + gn);
        rb[4 * h + 0] = v.x;
        rb[4 * h + 1] = v.y;
        rb[4 * h + 2] = v.z;
        rb[4 * h + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < T::kAPer; ++j) {
        const int gk = k0 + a_k + j;
        ra[j] = (gr < M && gk < K) ? A[(size_t)gr * lda + gk] : 0.f;
      }
#pragma unroll
      for (int h = 0; h < T::kBVec; ++h) {
        const int gk = k0 + b_k + T::kBRowStep * h;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          rb[4 * h + j] = (gk < K && gn + j < N) ? B[(size_t)gk * ldb + gn + j] : 0.f;
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int j = 0; j < T::kAPer; ++j) As[buf][a_k + j][a_row] = ra[j];
#pragma unroll
    for (int h = 0; h < T::kBVec; ++h) {
      floatx4 v = {rb[4 * h + 0], rb[4 * h + 1], rb[4 * h + 2], rb[4 * h + 3]};
      *reinterpret_cast<floatx4*>(&Bs[buf][b_k + T::kBRowStep * h][b_n]) = v;
    }
  };

  floatx16 acc[T::kMI][T::kNI];
#pragma unroll
  for (int i = 0; i < T::kMI; ++i)
#pragma unroll
    for (int j = 0; j < T::kNI; ++j) acc[i][j] = floatx16{};

  const int k_tiles = (K + kBK - 1) / kBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int lrow = lane & 31;
  const int lk = lane >> 5;
  const int am = wm * (kBM / 2) + lrow;
  const int bn = wn * (kBN / 2) + lrow;

  // MFMA operands of one k step (k = 2s + lane/32): register double buffering
  // reads step s+1 from LDS while step s's MFMAs run.
  float a_op[2][T::kMI], b_op[2][T::kNI];
  auto read_step = [&](int buf, int s, int slot) {
    const int kr = 2 * s + lk;
#pragma unroll
    for (int i = 0; i < T::kMI; ++i) a_op[slot][i] = As[buf][kr][am + 32 * i];
#pragma unroll
    for (int j = 0; j < T::kNI; ++j) b_op[slot][j] = Bs[buf][kr][bn + 32 * j];
  };

  for (int kt = 0; kt < k_tiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < k_tiles;
    if (more) load_tile((kt + 1) * kBK);
    read_step(cur, 0, 0);
#pragma unroll
    for (int s = 0; s < kBK / 2; ++s) {
      if (s + 1 < kBK / 2) read_step(cur, s + 1, (s + 1) & 1);
#pragma unroll
      for (int i = 0; i < T::kMI; ++i)
#pragma unroll
        for (int j = 0; j < T::kNI; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a_op[s & 1][i], b_op[s & 1][j], acc[i][j], 0, 0, 0);
    }
    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Accumulator layout of a 32x32 MFMA block: lane l, register r holds
  // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  auto store_block = [&](const floatx16& acc, int mi, int ni) {
    const int col = col0 + wn * (kBN / 2) + ni * 32 + lrow;
    if (col >= N) return;
    const int rb = row0 + wm * (kBM / 2) + mi * 32 + 4 * lk;
    float* cp = C + (size_t)rb * ldc + col;
    const float* rp = R != nullptr ? R + (size_t)rb * ldr + col : nullptr;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int dr = 8 * (r >> 2) + (r & 3);
      if (rb + dr < M) {
        float v = acc[r];
        if (rp != nullptr) v += rp[(size_t)dr * ldr];
        cp[(size_t)dr * ldc] = v;
      }
    }
  };
#pragma unroll
  for (int i = 0; i < T::kMI; ++i)
#pragma unroll
    for (int j = 0; j < T::kNI; ++j) store_block(acc[i][j], i, j);
}

// Direct-to-LDS variant for the branch-free shapes (k, n, lda, ldb multiples
// of 4, every slice a multiple of the K tile): A and B tiles go from HBM to LDS
// with buffer_load ... lds (16 bytes per lane, no register staging), which
// frees the staging registers for a third workgroup per CU (128x256) and
// removes the transposing LDS stores.
//
// LDS stage (kBM = 128, K tile 16): A is row-major, 8 blocks of 16 rows x 64 B,
// and chunk kc (4 floats) of block row r sits at position kc ^ ((r >> 2) & 3);
// B is k-major: 256-wide rows at a 1056-byte pitch, or 128-wide rows at 512
// bytes with chunk c of row k at c ^ (8 * ((k >> 2) & 1)).  Both choices make
// the MFMA operand reads bank-conflict free.
//
// K order: an MFMA 32x32x2 takes k index 0 from lanes 0-31 and k index 1 from
// lanes 32-63.  Lane half h reads the 4-float chunk 2p + h of its A row with
// one 128-bit read, so step (p, j) pairs k = 8p + j (lanes 0-31) with
// k = 8p + 4 + j (lanes 32-63); the B operand reads the same two k rows.
// Every k of the tile enters each accumulator exactly once.
template <int kBN>
struct DlCfg {
  static constexpr int kNI = kBN / 64;
  static constexpr int kABytes = 128 * kBK * 4;
  static constexpr int kBPitch = kBN == 256 ? 1056 : 512;
  static constexpr int kStage = kABytes + kBK * kBPitch;
};

// kGeGLU (128-wide tiles, eight waves only): B is [gate | up] with N gate
// columns, the tile of column block tn takes gate columns 64 tn .. +63 and the
// matching up columns, placed so that each wave's two 32-column MFMA blocks
// are a gate block and its up block (tile columns 0-31 gate, 32-63 up, 64-95
// gate + 32, 96-127 up + 32); the epilogue stores gelu_tanh(gate) * up, N
// columns in all.
template <int kBN, int kWaves, bool kGeGLU = false>
__device__ __forceinline__ void sgemm_f32_dl_body(const float* __restrict__ A, const float* __restrict__ B, float* C,
                                                  int M, int N, int K, int tiles_m, int tiles_n, int lda, int ldb,
                                                  int ldc, const float* R, int ldr, int k_len, long long sa,
                                                  long long sb, long long sc, char* S0, char* S1) {
  static_assert(!kGeGLU || (kBN == 128 && kWaves == 8), "the GeGLU tile is the eight-wave 128x128 one");
  using D = DlCfg<kBN>;
  constexpr int kNI = D::kNI;
  constexpr int kRW = 256 / kWaves;                  // rows per wave (waves: kWaves/2 along M, 2 along N)
  constexpr int kMI = kRW / 32;
  constexpr int kAI = 8 / kWaves;                    // A transfers (16-row blocks) per wave
  constexpr int kBI = (kBN == 256 ? 16 : 8) / kWaves;  // B transfers per wave
  typedef __attribute__((address_space(3))) void lds_void;

  if (gridDim.z > 1) {
    A += (size_t)blockIdx.z * sa;
    B += (size_t)blockIdx.z * sb;
    C += (size_t)blockIdx.z * sc;
  }
  int tm, tn;
  map_tile(tiles_m, tiles_n, &tm, &tn);
  const int row0 = tm * 128;
  const int col0 = kGeGLU ? tn * (kBN / 2) : tn * kBN;
  size_t a_extent = (size_t)M * lda;
  if (gridDim.y > 1) {
    const int kb = (int)blockIdx.y * k_len;
    A += kb;
    a_extent -= (size_t)kb;
    B += (size_t)kb * ldb;
    C += (size_t)blockIdx.y * M * ldc;
    K = min(k_len, K - kb);
  }
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1;
  const int wn = wave & 1;

  const __amdgpu_buffer_rsrc_t rsa =
      __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)(a_extent * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb =
      __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, (int)((size_t)K * ldb * 4), 0x00020000);

  // Per-lane source offsets (bytes, k0 = 0) of this wave's kAI A and kBI B
  // instructions; the tile's k offset travels in the scalar soffset.
  uint32_t a_off[kAI], b_off[kBI];
#pragma unroll
  for (int i = 0; i < kAI; ++i) {
    const int q = kAI * wave + i;  // A block: rows 16q..16q+15
    const int r = lane >> 2;
    const int kc = (lane & 3) ^ ((r >> 2) & 3);
    a_off[i] = (uint32_t)(((row0 + 16 * q + r) * lda + 4 * kc) * 4);
  }
#pragma unroll
  for (int i = 0; i < kBI; ++i) {
    if constexpr (kBN == 256) {
      const int kr = kBI * wave + i;  // one 256-wide row per instruction
      b_off[i] = (uint32_t)((kr * ldb + col0 + 4 * lane) * 4);
    } else {
      const int q = kBI * wave + i;  // rows 2q, 2q+1
      const int kr = 2 * q + (lane >> 5);
      const int c = (lane & 31) ^ (((kr >> 2) & 1) << 3);
      int gcol = col0 + 4 * c;
      if constexpr (kGeGLU) {
        const int seg = c >> 3;  // tile columns 32 seg .. +31
        gcol = col0 + (seg >> 1) * 32 + 4 * (c & 7) + ((seg & 1) ? N : 0);
      }
      b_off[i] = (uint32_t)((kr * ldb + gcol) * 4);
    }
  }
  auto issue = [&](char* stage, int k0) {
    const int sa_k = __builtin_amdgcn_readfirstlane(k0 * 4);
    const int sb_k = __builtin_amdgcn_readfirstlane(k0 * ldb * 4);
#pragma unroll
    for (int i = 0; i < kAI; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_void*)(stage + (kAI * wave + i) * 1024), 16, a_off[i], sa_k,
                                               0, 0);
#pragma unroll
    for (int i = 0; i < kBI; ++i) {
      char* dst = kBN == 256 ? stage + D::kABytes + (kBI * wave + i) * D::kBPitch
                             : stage + D::kABytes + (kBI * wave + i) * 1024;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_void*)dst, 16, b_off[i], sb_k, 0, 0);
    }
  };

  // Operand addresses (bytes within a stage).
  const int lrow = lane & 31;
  const int h = lane >> 5;
  const int am = wm * kRW + lrow;  // + 32 mi: two blocks further, same swizzle
  const int ar = am & 15;
  const uint32_t a_base = (uint32_t)((am >> 4) * 1024 + ar * 64 + ((h ^ ((ar >> 2) & 3)) << 4));
  uint32_t b_base[kBN == 256 ? 1 : 2];
  if constexpr (kBN == 256) {
    b_base[0] = (uint32_t)(D::kABytes + 4 * h * D::kBPitch + (wn * 128 + lrow) * 4);
  } else {
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
      b_base[ni] = (uint32_t)(D::kABytes + 4 * h * D::kBPitch + (wn * 16 + ((ni ^ h) << 3) + (lrow >> 2)) * 16 +
                              (lrow & 3) * 4);
  }

  floatx16 acc[kMI][kNI];
#pragma unroll
  for (int i = 0; i < kMI; ++i)
#pragma unroll
    for (int j = 0; j < kNI; ++j) acc[i][j] = floatx16{};

  auto compute = [&](const char* st) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      floatx4 a[kMI];
#pragma unroll
      for (int mi = 0; mi < kMI; ++mi)
        a[mi] = *reinterpret_cast<const floatx4*>(st + ((a_base ^ (uint32_t)(32 * p)) + mi * 2048));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float b[kNI];
        const int row_off = (8 * p + j) * D::kBPitch;
#pragma unroll
        for (int ni = 0; ni < kNI; ++ni) {
          if constexpr (kBN == 256)
            b[ni] = *reinterpret_cast<const float*>(st + b_base[0] + row_off + ni * 128);
          else
            b[ni] = *reinterpret_cast<const float*>(st + b_base[ni] + row_off);
        }
#pragma unroll
        for (int mi = 0; mi < kMI; ++mi)
#pragma unroll
          for (int ni = 0; ni < kNI; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[mi][j], b[ni], acc[mi][ni], 0, 0, 0);
      }
      // Keep each half's operand reads within the half: bounds register pressure.
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  const int k_tiles = K / kBK;
  issue(S0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // Unrolled by two so that the reads of one stage are visibly independent of
  // the transfers into the other (separate arrays).
  int kt = 0;
  for (; kt + 1 < k_tiles; kt += 2) {
    issue(S1, (kt + 1) * kBK);
    compute(S0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (kt + 2 < k_tiles) issue(S0, (kt + 2) * kBK);
    compute(S1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (kt < k_tiles) compute(S0);  // odd count: the last tile was issued into S0

  if constexpr (kGeGLU) {
    // acc[0][0]: gate columns col0 + 32 wn + lrow, acc[0][1]: the same up columns
    const int col = col0 + wn * 32 + lrow;
    if (col >= N) return;
    const int rb = row0 + wm * kRW + 4 * h;
    float* cp = C + (size_t)rb * ldc + col;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int dr = 8 * (r >> 2) + (r & 3);
      if (rb + dr < M) cp[(size_t)dr * ldc] = gelu_tanh(acc[0][0][r]) * acc[0][1][r];
    }
    return;
  }
  // Row offsets from the block's first row are wave-uniform (scalar), so only
  // one 64-bit address per block lives in vector registers.
  auto store_block = [&](const floatx16& acc, int mi, int ni) {
    const int col = col0 + wn * (kBN / 2) + ni * 32 + lrow;
    if (col >= N) return;
    const int rb = row0 + wm * kRW + mi * 32 + 4 * h;
    float* cp = C + (size_t)rb * ldc + col;
    const float* rp = R != nullptr ? R + (size_t)rb * ldr + col : nullptr;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int dr = 8 * (r >> 2) + (r & 3);
      if (rb + dr < M) {
        float v = acc[r];
        if (rp != nullptr) v += rp[(size_t)dr * ldr];
        cp[(size_t)dr * ldc] = v;
      }
    }
  };
#pragma unroll
  for (int i = 0; i < kMI; ++i)
#pragma unroll
    for (int j = 0; j < kNI; ++j) store_block(acc[i][j], i, j);
}

// Two stages of LDS; the kernels differ in tile width and occupancy target.
__global__ __launch_bounds__(256, 3) void sgemm_f32_dl256_kernel(const float* __restrict__ A,
                                                                 const float* __restrict__ B, float* C, int M, int N,
                                                                 int K, int tiles_m, int tiles_n, int lda, int ldb,
                                                                 int ldc, const float* R, int ldr, int k_len,
                                                                 long long sa, long long sb, long long sc) {
  __shared__ __attribute__((aligned(1024))) char S0[DlCfg<256>::kStage];
  __shared__ __attribute__((aligned(1024))) char S1[DlCfg<256>::kStage];
  sgemm_f32_dl_body<256, 4>(A, B, C, M, N, K, tiles_m, tiles_n, lda, ldb, ldc, R, ldr, k_len, sa, sb, sc, S0, S1);
}

// 128x128 with eight waves (each 32x64, 50 VGPRs): two waves per SIMD even
// when the grid gives one workgroup per CU (small and split-K products), and
// three workgroups per CU on large grids (106 SGPRs, the residual epilogue's
// row offsets among them, allow seven waves per SIMD).  Two or four
// workgroups per CU measured the same at 4096^3 (921 us), four 4 % slower
// at 8192 x 8192 x 2048.
__global__ __launch_bounds__(512, 1) void sgemm_f32_dl128w8_kernel(const float* __restrict__ A,
                                                                   const float* __restrict__ B, float* C, int M,
                                                                   int N, int K, int tiles_m, int tiles_n, int lda,
                                                                   int ldb, int ldc, const float* R, int ldr,
                                                                   int k_len, long long sa, long long sb,
                                                                   long long sc) {
  __shared__ __attribute__((aligned(1024))) char S0[DlCfg<128>::kStage];
  __shared__ __attribute__((aligned(1024))) char S1[DlCfg<128>::kStage];
  sgemm_f32_dl_body<128, 8>(A, B, C, M, N, K, tiles_m, tiles_n, lda, ldb, ldc, R, ldr, k_len, sa, sb, sc, S0, S1);
}

// The gate|up product of the Gemma-style layer with GeGLU in the epilogue
// (sgemm_f32_dl_body's kGeGLU): C is the [M, N] GeGLU output.
__global__ __launch_bounds__(512, 1) void sgemm_f32_dl128w8_geglu_kernel(const float* __restrict__ A,
                                                                         const float* __restrict__ B, float* C,
                                                                         int M, int N, int K, int tiles_m,
                                                                         int tiles_n, int lda, int ldb, int ldc) {
  __shared__ __attribute__((aligned(1024))) char S0[DlCfg<128>::kStage];
  __shared__ __attribute__((aligned(1024))) char S1[DlCfg<128>::kStage];
  sgemm_f32_dl_body<128, 8, true>(A, B, C, M, N, K, tiles_m, tiles_n, lda, ldb, ldc, nullptr, 0, K, 0, 0, 0, S0,
                                  S1);
}

// 64x64 tile for grids that would otherwise leave CUs idle or need a
// split-K launch (C1's 1024^3 is 256 such tiles: one per CU, no K split
// across workgroups).  Eight waves: wave (kh, wm, wn) owns the 32x32 quadrant
// (wm, wn) for the kh-th 16-wide half of every 32-wide K tile, so each SIMD
// runs two independent accumulation chains; at the end the kh = 1 waves hand
// their accumulators to the kh = 0 waves through LDS, which add them in a
// fixed order (deterministic) and store.
//
// LDS stage (K tile 32): A is row-major, 64 rows of 128 bytes, chunk c
// (4 floats) of row r at position c ^ ((r >> 1) & 7): the 16 lanes of a
// 128-bit read group hit 16 distinct 16-byte bank groups.  B is row-major, 32
// k-rows of 256 bytes, with the 128-byte halves of rows with (k >> 2) & 1
// exchanged, so the two lane halves of a B read (rows k and k + 4) use
// opposite halves of the banks.  Both placements are set by each lane's
// source address in the HBM -> LDS transfers (one 1 KB transfer of A and one
// of B per wave per tile).  K order: MFMA step (p, j) of half kh pairs
// k = 16kh + 8p + j (lanes 0-31) with k = 16kh + 8p + 4 + j (lanes 32-63).
template <int kBKs>
struct Dl64Cfg {
  static constexpr int kRowBytes = kBKs * 4;            // A row (kBKs floats)
  static constexpr int kChunks = kBKs / 4;              // 16-byte chunks per A row
  static constexpr int kABytes = 64 * kRowBytes;
  static constexpr int kStage = 2 * kABytes;            // A then B [kBKs][64]
  static constexpr int kXfer = kABytes / 1024 / 8;      // 1 KB transfers of A (and of B) per wave
};
// A chunk c of row r sits at position c ^ swz: for 32-wide K tiles (128-byte
// rows) swz = (r >> 1) & 7, for 64-wide tiles (256-byte rows) swz = r & 15.
template <int kBKs>
__device__ __forceinline__ int dl64_swz(int r) {
  return kBKs == 32 ? ((r >> 1) & 7) : (r & 15);
}

// kSt LDS stages in a ring: the transfers of tile t + kSt - 1 are issued while
// tile t is computed.  With two stages a tile's transfers are waited for one
// tile (about 0.8 us of MFMA work at one workgroup per CU) after they are
// issued, less than the memory latency; the four-stage form, launched when a
// grid has at most one workgroup per CU and K slices of 2048 or more, keeps
// three tiles in flight.  The
// transfers are inline assembly (the compiler then adds no waits of its own
// before the LDS reads of other stages); explicit vmcnt waits and barriers
// order each tile.
template <int kBKs, int kSt>
__device__ __forceinline__ void sgemm_f32_dl64_body(const float* __restrict__ A, const float* __restrict__ B,
                                                    float* C, int M, int N, int K, int tiles_m, int tiles_n, int lda,
                                                    int ldb, int ldc, const float* R, int ldr, int k_len,
                                                    long long sa, long long sb, long long sc,
                                                    char* const (&S)[kSt]) {
  static_assert(kSt >= 2 && kSt <= 4, "two to four stages");
  using Cfg = Dl64Cfg<kBKs>;
  if (gridDim.z > 1) {
    A += (size_t)blockIdx.z * sa;
    B += (size_t)blockIdx.z * sb;
    C += (size_t)blockIdx.z * sc;
  }
  int tm, tn;
  map_tile(tiles_m, tiles_n, &tm, &tn);
  const int row0 = tm * 64;
  const int col0 = tn * 64;
  size_t a_extent = (size_t)M * lda;
  if (gridDim.y > 1) {
    const int kb = (int)blockIdx.y * k_len;
    A += kb;
    a_extent -= (size_t)kb;
    B += (size_t)kb * ldb;
    C += (size_t)blockIdx.y * M * ldc;
    K = min(k_len, K - kb);
  }
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kh = wave >> 2;
  const int wm = (wave >> 1) & 1;
  const int wn = wave & 1;

  typedef int int4v __attribute__((ext_vector_type(4)));
  auto desc = [](const void* ptr, uint32_t bytes) {
    const unsigned long long addr = (unsigned long long)ptr;
    int4v d;
    d.x = __builtin_amdgcn_readfirstlane((int)(addr & 0xffffffffu));
    d.y = __builtin_amdgcn_readfirstlane((int)(addr >> 32));
    d.z = __builtin_amdgcn_readfirstlane((int)bytes);
    d.w = 0x00020000;
    return d;
  };
  const int4v rsa = desc(A, (uint32_t)(a_extent * 4));
  const int4v rsb = desc(B, (uint32_t)((size_t)K * ldb * 4));
  // Transfer q (1 KB) of A covers rows 1024q/kRowBytes.., of B k-rows 4q..4q+3;
  // wave w issues q = kXfer*w + i.
  uint32_t a_off[Cfg::kXfer], b_off[Cfg::kXfer];
#pragma unroll
  for (int i = 0; i < Cfg::kXfer; ++i) {
    const int q = Cfg::kXfer * wave + i;
    const int e = 64 * q + lane;  // 16-byte chunk index of the A tile
    const int r = e / Cfg::kChunks;
    const int c = (e % Cfg::kChunks) ^ dl64_swz<kBKs>(r);
    a_off[i] = (uint32_t)(((row0 + r) * lda + 4 * c) * 4);
    const int kr = 4 * q + (lane >> 4);
    const int cb = (lane & 15) ^ (8 * ((kr >> 2) & 1));
    b_off[i] = (uint32_t)((kr * ldb + col0 + 4 * cb) * 4);
  }
  auto issue = [&](char* stage, int k0) {
    const int sa_k = __builtin_amdgcn_readfirstlane(k0 * 4);
    const int sb_k = __builtin_amdgcn_readfirstlane(k0 * ldb * 4);
    const uint32_t base = (uint32_t)(size_t)(__attribute__((address_space(3))) char*)stage;
#pragma unroll
    for (int i = 0; i < Cfg::kXfer; ++i) {
      const int q = Cfg::kXfer * wave + i;
      const uint32_t la = __builtin_amdgcn_readfirstlane(base + q * 1024);
      const uint32_t lb = __builtin_amdgcn_readfirstlane(base + Cfg::kABytes + q * 1024);
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(la), "v"(a_off[i]), "s"(rsa),
                   "s"(sa_k)
                   : "memory", "m0");
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lb), "v"(b_off[i]), "s"(rsb),
                   "s"(sb_k)
                   : "memory", "m0");
    }
  };
  // This wave's transfers of a tile: kPerTile; at most `in_flight` later
  // tiles may stay outstanding.
  constexpr int kPerTile = 2 * Cfg::kXfer;
  auto wait_tiles = [&](int in_flight) {
    if (in_flight >= 2)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kPerTile) : "memory");
    else if (in_flight == 1)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kPerTile) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  auto barrier = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // Operand addresses (bytes within a stage).  Half kh covers k in
  // [kh*kBKs/2, (kh+1)*kBKs/2): logical A chunk kh*kChunks/2 + 2p + h.  B row
  // k = kh*kBKs/2 + 8p + 4h + j holds column c at c ^ (32 h).
  const int lrow = lane & 31;
  const int h = lane >> 5;
  const int ar = 32 * wm + lrow;
  const uint32_t a_row = (uint32_t)(ar * Cfg::kRowBytes);
  const int a_sw = dl64_swz<kBKs>(ar);
  const uint32_t b_base =
      (uint32_t)(Cfg::kABytes + (kh * kBKs / 2 + 4 * h) * 256 + ((((32 * wn) ^ (32 * h)) + lrow) * 4));

  floatx16 acc = {};
  auto compute = [&](const char* st) {
#pragma unroll
    for (int p = 0; p < kBKs / 16; ++p) {
      const floatx4 a =
          *reinterpret_cast<const floatx4*>(st + a_row + (((kh * Cfg::kChunks / 2 + 2 * p + h) ^ a_sw) << 4));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float b = *reinterpret_cast<const float*>(st + b_base + (8 * p + j) * 256);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b, acc, 0, 0, 0);
      }
    }
  };

  // K need not be a multiple of the K tile (only of 4): the last tile's B
  // rows past K read zero (outside the buffer range), and its A columns past
  // K, which the transfers fill from the next row, are cleared in LDS before
  // that tile is used, so they add exact zeros whatever they held.
  const int k_tiles = (K + kBKs - 1) / kBKs;
  const int krem = K - (k_tiles - 1) * kBKs;
  auto settle_last = [&](char* st, int t) {
    if (t != k_tiles - 1 || krem == kBKs) return;
    const int c0 = krem / 4;
    const int nc = Cfg::kChunks - c0;
    for (int e = tid; e < 64 * nc; e += 512) {
      const int r = e / nc;
      const int c = c0 + e % nc;
      *reinterpret_cast<floatx4*>(st + r * Cfg::kRowBytes + ((c ^ dl64_swz<kBKs>(r)) << 4)) = floatx4{};
    }
    __syncthreads();
  };
  // Step t: tile t has landed for this wave (later tiles may stay in flight),
  // the barrier makes it complete for all waves and frees tile t-1's stage,
  // which takes tile t + kSt - 1; then tile t is computed.  u = t % kSt is a
  // compile-time constant (the loop is unrolled by kSt).
  auto step = [&](int t, auto u_c) {
    constexpr int u = decltype(u_c)::value;
    wait_tiles(min(kSt - 2, k_tiles - 1 - t));
    barrier();
    if (t + kSt - 1 < k_tiles) issue(S[(u + kSt - 1) % kSt], (t + kSt - 1) * kBKs);
    settle_last(S[u], t);
    compute(S[u]);
  };
#pragma unroll
  for (int j = 0; j < kSt - 1; ++j)
    if (j < k_tiles) issue(S[j], j * kBKs);
  const std::integral_constant<int, 0> u0{};
  const std::integral_constant<int, 1> u1{};
  const std::integral_constant<int, (kSt > 2 ? 2 : 0)> u2{};
  const std::integral_constant<int, (kSt > 3 ? 3 : 0)> u3{};
  int t = 0;
  for (; t + kSt <= k_tiles; t += kSt) {
    step(t, u0);
    step(t + 1, u1);
    if constexpr (kSt > 2) step(t + 2, u2);
    if constexpr (kSt > 3) step(t + 3, u3);
  }
  if (t < k_tiles) step(t, u0);
  if constexpr (kSt > 2)
    if (t + 1 < k_tiles) step(t + 1, u1);
  if constexpr (kSt > 3)
    if (t + 2 < k_tiles) step(t + 2, u2);
  __syncthreads();  // every wave is done with the stages

  // The kh = 1 waves pass their quadrant's accumulators to the kh = 0 waves
  // (stage 0 is free after the last barrier): 64 lanes x 16 floats per quadrant.
  float* xchg = reinterpret_cast<float*>(S[0]) + (wave & 3) * 1024;
  if (kh == 1) {
#pragma unroll
    for (int r = 0; r < 16; r += 4)
      *reinterpret_cast<floatx4*>(xchg + lane * 16 + r) = floatx4{acc[r], acc[r + 1], acc[r + 2], acc[r + 3]};
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int r = 0; r < 16; r += 4) {
    const floatx4 o = *reinterpret_cast<const floatx4*>(xchg + lane * 16 + r);
    acc[r] += o.x;
    acc[r + 1] += o.y;
    acc[r + 2] += o.z;
    acc[r + 3] += o.w;
  }
  const int col = col0 + 32 * wn + lrow;
  if (col >= N) return;
  const int rb = row0 + 32 * wm + 4 * h;
  float* cp = C + (size_t)rb * ldc + col;
  const float* rp = R != nullptr ? R + (size_t)rb * ldr + col : nullptr;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int dr = 8 * (r >> 2) + (r & 3);
    if (rb + dr < M) {
      float v = acc[r];
      if (rp != nullptr) v += rp[(size_t)dr * ldr];
      cp[(size_t)dr * ldc] = v;
    }
  }
}

__global__ __launch_bounds__(512, 2) void sgemm_f32_dl64_kernel(const float* __restrict__ A,
                                                                const float* __restrict__ B, float* C, int M, int N,
                                                                int K, int tiles_m, int tiles_n, int lda, int ldb,
                                                                int ldc, const float* R, int ldr, int k_len,
                                                                long long sa, long long sb, long long sc) {
  __shared__ __attribute__((aligned(1024))) char S0[Dl64Cfg<32>::kStage];
  __shared__ __attribute__((aligned(1024))) char S1[Dl64Cfg<32>::kStage];
  char* const st[2] = {S0, S1};
  sgemm_f32_dl64_body<32, 2>(A, B, C, M, N, K, tiles_m, tiles_n, lda, ldb, ldc, R, ldr, k_len, sa, sb, sc, st);
}

// 64-wide K tiles: twice the MFMA work between barriers and per LDS stage,
// for operands that stream from the Infinity Cache (long K) rather than L2.
__global__ __launch_bounds__(512, 2) void sgemm_f32_dl64k64_kernel(const float* __restrict__ A,
                                                                   const float* __restrict__ B, float* C, int M,
                                                                   int N, int K, int tiles_m, int tiles_n, int lda,
                                                                   int ldb, int ldc, const float* R, int ldr,
                                                                   int k_len, long long sa, long long sb,
                                                                   long long sc) {
  __shared__ __attribute__((aligned(1024))) char S0[Dl64Cfg<64>::kStage];
  __shared__ __attribute__((aligned(1024))) char S1[Dl64Cfg<64>::kStage];
  char* const st[2] = {S0, S1};
  sgemm_f32_dl64_body<64, 2>(A, B, C, M, N, K, tiles_m, tiles_n, lda, ldb, ldc, R, ldr, k_len, sa, sb, sc, st);
}

// The four-stage forms, for grids of at most one workgroup per CU (the LDS
// ring takes 64 and 128 KB).
template <int kBKs>
__global__ __launch_bounds__(512, 1) void sgemm_f32_dl64_ring_kernel(const float* __restrict__ A,
                                                                     const float* __restrict__ B, float* C, int M,
                                                                     int N, int K, int tiles_m, int tiles_n, int lda,
                                                                     int ldb, int ldc, const float* R, int ldr,
                                                                     int k_len, long long sa, long long sb,
                                                                     long long sc) {
  __shared__ __attribute__((aligned(1024))) char S0[Dl64Cfg<kBKs>::kStage];
  __shared__ __attribute__((aligned(1024))) char S1[Dl64Cfg<kBKs>::kStage];
  __shared__ __attribute__((aligned(1024))) char S2[Dl64Cfg<kBKs>::kStage];
  __shared__ __attribute__((aligned(1024))) char S3[Dl64Cfg<kBKs>::kStage];
  char* const st[4] = {S0, S1, S2, S3};
  sgemm_f32_dl64_body<kBKs, 4>(A, B, C, M, N, K, tiles_m, tiles_n, lda, ldb, ldc, R, ldr, k_len, sa, sb, sc, st);
}

// dst [rows_d][ld_d] (16-byte rows) = src [rows_s][cols_s] (row stride ld_s,
// any alignment), zero outside: the padded copies through which operands the
// direct-to-LDS kernels cannot read (ragged k or n, unaligned rows) reach them.
// One launch pads both operands: the first blocks_a workgroups copy A, the
// rest B.  A workgroup's four waves take four consecutive rows and one
// 256-float chunk of them (pad_blocks per job); lane l moves floats l, l + 64,
// l + 128 and l + 192 of the chunk, so each load and store instruction covers
// 256 contiguous bytes of its row on either side (rows_d * ld_d < 2^32 and
// the block count < 2^22: the GEMM admission bounds m*k and k*n below 2^32).
struct PadJob {
  const float* src;
  float* dst;
  int rows_s, cols_s, ld_s, rows_d, ld_d;
};

constexpr uint32_t kPadChunk = 256;

uint32_t pad_blocks(uint32_t rows_d, uint32_t ld_d) {
  return ((rows_d + 3u) / 4u) * ((ld_d + kPadChunk - 1u) / kPadChunk);
}

__global__ __launch_bounds__(256) void pack_pad_kernel(PadJob ja, PadJob jb, uint32_t blocks_a) {
  const bool first = blockIdx.x < blocks_a;
  const PadJob j = first ? ja : jb;
  const uint32_t blk = first ? blockIdx.x : blockIdx.x - blocks_a;
  const uint32_t chunks = ((uint32_t)j.ld_d + kPadChunk - 1u) / kPadChunk;
  const uint32_t group = blk / chunks;
  const int r = (int)(group * 4u + (threadIdx.x >> 6));
  if (r >= j.rows_d) return;
  const int c0 = (int)((blk - group * chunks) * kPadChunk + (threadIdx.x & 63u));
  const bool row_in = r < j.rows_s;
  const float* sp = j.src + (row_in ? (size_t)r * j.ld_s : 0);
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = c0 + 64 * q;
    v[q] = (row_in && c < j.cols_s) ? sp[c] : 0.0f;
  }
  float* dp = j.dst + (size_t)r * j.ld_d;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = c0 + 64 * q;
    if (c < j.ld_d) dp[c] = v[q];
  }
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

// Same sum, 4 columns per thread (N, ldc, ldr multiples of 4, 16-byte aligned
// C and R): one workgroup row-slice per (blockIdx.x, row), no per-element
// 64-bit division; the slabs are read with 128-bit loads, all issued before
// the adds (same order of additions as the scalar kernel).
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(const float* __restrict__ P, float* C, int M, int N,
                                                             int ldc, int splits, const float* R, int ldr) {
  const int n4 = N >> 2;
  const int c4 = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (c4 >= n4) return;
  const size_t slab4 = (size_t)M * n4;
  const floatx4* P4 = reinterpret_cast<const floatx4*>(P);
  for (int row = (int)blockIdx.y; row < M; row += (int)gridDim.y) {
    const size_t i = (size_t)row * n4 + c4;
    floatx4 part[16];
#pragma unroll
    for (int s = 0; s < 16; ++s)
      if (s < splits) part[s] = P4[(size_t)s * slab4 + i];
    floatx4 v = part[0];
#pragma unroll
    for (int s = 1; s < 16; ++s)
      if (s < splits) {
        v.x += part[s].x;
        v.y += part[s].y;
        v.z += part[s].z;
        v.w += part[s].w;
      }
    if (R != nullptr) {
      const floatx4 r = reinterpret_cast<const floatx4*>(R + (size_t)row * ldr)[c4];
      v.x += r.x;
      v.y += r.y;
      v.z += r.z;
      v.w += r.w;
    }
    reinterpret_cast<floatx4*>(C + (size_t)row * ldc)[c4] = v;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Tile shapes: 0 = 128x256, 1 = 128x128, 2 = 64x128 (register-staged loads);
// 5 / 6 = 64x64 direct-to-LDS with each K tile (32 / 64 wide) split between
// two wave groups (branch-free shapes whose K slices are whole K tiles only);
// 3 = 128x256 (four waves), 4 = 128x128 (eight waves) direct-to-LDS, for
// branch-free shapes only (otherwise the staged shape of the same size runs).
constexpr int kTileShapes = 7;
constexpr int kTileM[kTileShapes] = {128, 128, 64, 128, 128, 64, 64};
constexpr int kTileN[kTileShapes] = {256, 128, 128, 256, 128, 64, 64};
constexpr int kStagedFallback[kTileShapes] = {0, 1, 2, 0, 1, 2, 2};
constexpr int kTileK[kTileShapes] = {16, 16, 16, 16, 16, 32, 64};  // K granule of a slice

struct SgemmPlan {
  int tile;    // index into kTileM / kTileN
  int splits;  // K slices (1: no split)
  int k_len;   // K elements per slice (a multiple of the K tile when split)
};

// Rounds a requested slice count to whole K tiles per slice.
SgemmPlan make_plan(int tile, int splits, uint32_t k) {
  SgemmPlan p{tile, 1, (int)k};
  if (splits > 1) {
    const int g = kTileK[tile];
    p.k_len = (int)((((k + splits - 1) / splits) + g - 1) / g * g);
    p.splits = (int)((k + p.k_len - 1) / p.k_len);
    if (p.splits <= 1) {
      p.splits = 1;
      p.k_len = (int)k;
    }
  }
  return p;
}

// True when the buffer-load kernels apply: 128-bit aligned operands, every
// slice length a multiple of the K tile and every 32-bit byte offset (rows up
// to M + 128, all of B plus a tile row) in range.
// `aligned`: both operand base addresses are 16-byte aligned.  The 128-wide
// direct kernels need every slice to be whole K tiles of 16; the 64x64 ones
// (tiles 5 and 6) take a K tail (k % 4 == 0) in the last tile of each product.
bool buffer_path(bool aligned, int lda, long long sa, int ldb, long long sb, uint32_t m, uint32_t n, uint32_t k,
                 int k_len, int tile = 4) {
  // B chunks past column n lie in B's padding or next row and only feed
  // output columns that are never stored, so n itself may be ragged.
  const bool vec = (k % 4 == 0) && (lda % 4 == 0) && (ldb % 4 == 0) && (sa % 4 == 0) && (sb % 4 == 0) && aligned;
  const bool k_ok = tile >= 5 ? true : (k % kBK == 0) && (k_len % kBK == 0);
  return vec && k_ok && (size_t)(m + 128) * lda * 4 < (1ull << 31) && ((size_t)k * ldb + n + 256) * 4 < (1ull << 31);
}

// Plan choice: the (tile shape, K slices) pair with the least estimated time.
// A grid of W workgroups fills the CUs in rounds of occ*256 (occ = resident
// workgroups per CU for the tile); a CU holding w workgroups of tile t runs
// them at efficiency kTileEffW[t][w-1] of its MFMA rate (256 flop/clk at 2.38
// GHz), so a K step of 16 of a BMxBN workgroup costs w * BM*BN*32/609280 us /
// eff.  Each round adds ~1.7 us of prologue/epilogue, a launch ~3.5 us, and a
// split adds the reduce (~1.5 us + (s+1) M N floats at ~3.5 TB/s).  The
// efficiencies and overheads are a least-squares fit (log time) to every
// valid (tile, K slices) variant timed at 28 shapes on MI355X (the benchmark
// shapes, the C4 and Z-Image block products, their 32-row tails, tall and
// wide panels); the chosen plan is within 1 % of the measured best on
// average and within 5 % at all but one shape.
constexpr int kTileOcc[kTileShapes] = {2, 3, 4, 3, 5, 4, 2};
constexpr double kTileEffW[kTileShapes][5] = {
    {0.776, 0.883},                       // 128x256 staged
    {0.726, 0.837, 0.913},                // 128x128 staged
    {0.555, 0.740, 0.774, 0.894},         // 64x128 staged
    {0.900, 0.975, 0.948},                // 128x256 direct
    {0.935, 0.971, 0.976, 0.967, 0.967},  // 128x128 direct, eight waves
    {0.606, 0.766, 0.846, 0.931},         // 64x64 direct, K tile 32
    {0.772, 0.911}};                      // 64x64 direct, K tile 64

// scalar_loads: the register-staged kernels read the operands with predicated
// 32-bit loads (k or n not a multiple of 4, unaligned rows), about 1.5x slower
// per K step than with 128-bit loads (measured at 4097x3001x513).
double plan_cost(const SgemmPlan& p, uint32_t m, uint32_t n, uint32_t batch, bool scalar_loads = false) {
  const int t = p.tile;
  const double w_total = (double)((m + kTileM[t] - 1) / kTileM[t]) * ((n + kTileN[t] - 1) / kTileN[t]) * p.splits *
                         batch;
  const double k_tiles = (double)((p.k_len + kBK - 1) / kBK);
  const double t16 = (double)kTileM[t] * kTileN[t] * 32.0 / 609280.0;
  const double slots = 256.0 * kTileOcc[t];
  const double full = std::floor(w_total / slots);
  const double rest = w_total - full * slots;
  auto eff = [&](int w) { return kTileEffW[t][std::min(w, kTileOcc[t]) - 1]; };
  double us = full * kTileOcc[t] * k_tiles * t16 / eff(kTileOcc[t]);
  if (rest > 0) {
    const int w = (int)std::ceil(rest / 256.0);
    us += w * k_tiles * t16 / eff(w);
  }
  if (scalar_loads && t < 3) us *= 1.5;
  us += 3.45 + 1.72 * (full + (rest > 0 ? 1.0 : 0.0));
  if (p.splits > 1) us += 1.46 + (double)(p.splits + 1) * m * n * 4.0 / 3.5e6;
  return us;
}

// max_partial_floats bounds the split-K partial buffer (splits * m * n floats)
// a plan may use; a plan without a split needs none, so one always exists.
SgemmPlan plan_sgemm(bool aligned, int lda, long long sa, int ldb, long long sb, uint32_t m, uint32_t n, uint32_t k,
                     uint32_t batch, uint64_t max_partial_floats = ~0ull) {
  static const int kSplitChoices[] = {1, 2, 3, 4, 6, 8, 12, 16};
  // The eight-wave 128x128 kernel is tried first and is only replaced by a
  // plan more than 1 % cheaper (near ties keep the established kernel; the
  // model is accurate to a few per cent).
  static const int kTileOrder[kTileShapes] = {4, 3, 0, 1, 2, 5, 6};
  const bool scalar = !((k % 4 == 0) && (n % 4 == 0) && (lda % 4 == 0) && (ldb % 4 == 0) && (sa % 4 == 0) &&
                        (sb % 4 == 0) && aligned);
  SgemmPlan best = make_plan(0, 1, k);
  double best_cost = 1e300;
  for (int t : kTileOrder) {
    for (int s : kSplitChoices) {
      if (s > 1 && (batch > 1 || k / (uint32_t)s < 64)) break;
      const SgemmPlan p = make_plan(t, s, k);
      if (p.splits != s) continue;
      if (p.splits > 1 && (uint64_t)p.splits * m * n > max_partial_floats) continue;
      if (t >= 3 && !buffer_path(aligned, lda, sa, ldb, sb, m, n, k, p.k_len, t)) continue;
      const double c = plan_cost(p, m, n, batch, scalar);
      if (c < best_cost * 0.99) {
        best_cost = c;
        best = p;
      }
    }
  }
  return best;
}

template <int kBM, int kBN>
void launch_tile(bool buf, bool vec, dim3 grid, hipStream_t stream, const float* a, const float* b, float* c, int m,
                 int n, int k, int tiles_m, int tiles_n, int lda, int ldb, int ldc, const float* r, int ldr, int k_len,
                 long long sa, long long sb, long long sc) {
  if (buf)
    hipLaunchKernelGGL((sgemm_f32_mfma_kernel<true, true, kBM, kBN>), grid, dim3(256), 0, stream, a, b, c, m, n, k,
                       tiles_m, tiles_n, lda, ldb, ldc, r, ldr, k_len, sa, sb, sc);
  else if (vec)
    hipLaunchKernelGGL((sgemm_f32_mfma_kernel<true, false, kBM, kBN>), grid, dim3(256), 0, stream, a, b, c, m, n, k,
                       tiles_m, tiles_n, lda, ldb, ldc, r, ldr, k_len, sa, sb, sc);
  else
    hipLaunchKernelGGL((sgemm_f32_mfma_kernel<false, false, kBM, kBN>), grid, dim3(256), 0, stream, a, b, c, m, n, k,
                       tiles_m, tiles_n, lda, ldb, ldc, r, ldr, k_len, sa, sb, sc);
}

// Launches the MFMA kernel of plan p over `batch` matrices (batch > 1 only
// without split) and, when split, the reduce into c (partial: splits*m*n floats).
hipError_t run_sgemm_plan(const SgemmPlan& p, const float* a, int lda, long long sa, const float* b, int ldb,
                          long long sb, float* c, int ldc, long long sc, uint32_t m, uint32_t n, uint32_t k,
                          uint32_t batch, const float* residual, int ldr, float* partial, hipStream_t stream,
                          bool reduce = true) {
  const bool split = p.splits > 1;
  const bool vec = (k % 4 == 0) && (n % 4 == 0) && (lda % 4 == 0) && (ldb % 4 == 0) && (sa % 4 == 0) &&
                   (sb % 4 == 0) && aligned16(a) && aligned16(b);
  const bool buf = buffer_path(aligned16(a) && aligned16(b), lda, sa, ldb, sb, m, n, k, p.k_len, p.tile);
  const int tile = (p.tile >= 3 && !buf) ? kStagedFallback[p.tile] : p.tile;
  const int bm = kTileM[tile], bn = kTileN[tile];
  const int tiles_m = (int)((m + bm - 1) / bm);
  const int tiles_n = (int)((n + bn - 1) / bn);
  const dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)p.splits, batch);
  float* out = split ? partial : c;
  // A grid that gives every CU at most one workgroup, with a long K loop:
  // the 64x64 kernels take their four-stage form (C4's 512x2048x2048 output
  // projection 38.8 -> 36.8 us; at K = 1024, C1, the deeper ring measured
  // 0.4 us slower, so shorter slices keep two stages).
  const int cus = ctx().props.multiProcessorCount > 0 ? ctx().props.multiProcessorCount : 256;
  const bool one_per_cu = (long long)grid.x * grid.y * grid.z <= cus && p.k_len >= 2048;
  const int ldo = split ? (int)n : ldc;
  const float* res = split ? nullptr : residual;
  switch (tile) {
    case 5:
      if (one_per_cu)
        hipLaunchKernelGGL(sgemm_f32_dl64_ring_kernel<32>, grid, dim3(512), 0, stream, a, b, out, (int)m, (int)n,
                           (int)k, tiles_m, tiles_n, lda, ldb, ldo, res, ldr, p.k_len, sa, sb, sc);
      else
        hipLaunchKernelGGL(sgemm_f32_dl64_kernel, grid, dim3(512), 0, stream, a, b, out, (int)m, (int)n, (int)k,
                           tiles_m, tiles_n, lda, ldb, ldo, res, ldr, p.k_len, sa, sb, sc);
      break;
    case 6:
      if (one_per_cu)
        hipLaunchKernelGGL(sgemm_f32_dl64_ring_kernel<64>, grid, dim3(512), 0, stream, a, b, out, (int)m, (int)n,
                           (int)k, tiles_m, tiles_n, lda, ldb, ldo, res, ldr, p.k_len, sa, sb, sc);
      else
        hipLaunchKernelGGL(sgemm_f32_dl64k64_kernel, grid, dim3(512), 0, stream, a, b, out, (int)m, (int)n, (int)k,
                           tiles_m, tiles_n, lda, ldb, ldo, res, ldr, p.k_len, sa, sb, sc);
      break;
    case 3:
      hipLaunchKernelGGL(sgemm_f32_dl256_kernel, grid, dim3(256), 0, stream, a, b, out, (int)m, (int)n, (int)k,
                         tiles_m, tiles_n, lda, ldb, ldo, res, ldr, p.k_len, sa, sb, sc);
      break;
    case 4:
      hipLaunchKernelGGL(sgemm_f32_dl128w8_kernel, grid, dim3(512), 0, stream, a, b, out, (int)m, (int)n, (int)k,
                         tiles_m, tiles_n, lda, ldb, ldo, res, ldr, p.k_len, sa, sb, sc);
      break;
    case 0:
      launch_tile<128, 256>(buf, vec, grid, stream, a, b, out, (int)m, (int)n, (int)k, tiles_m, tiles_n, lda, ldb,
                            ldo, res, ldr, p.k_len, sa, sb, sc);
      break;
    case 1:
      launch_tile<128, 128>(buf, vec, grid, stream, a, b, out, (int)m, (int)n, (int)k, tiles_m, tiles_n, lda, ldb,
                            ldo, res, ldr, p.k_len, sa, sb, sc);
      break;
    default:
      launch_tile<64, 128>(buf, vec, grid, stream, a, b, out, (int)m, (int)n, (int)k, tiles_m, tiles_n, lda, ldb,
                           ldo, res, ldr, p.k_len, sa, sb, sc);
      break;
  }
  if (split && reduce) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const bool vec4 = n % 4 == 0 && ldc % 4 == 0 && aligned16(c) && (residual == nullptr || (ldr % 4 == 0 && aligned16(residual)));
    if (vec4 && p.splits <= 16) {
      const unsigned bx = (unsigned)((n / 4 + 255) / 256);
      const unsigned by = (unsigned)std::min<uint32_t>(m, std::max(1u, 8192u / bx));
      hipLaunchKernelGGL(splitk_reduce4_kernel, dim3(bx, by), dim3(256), 0, stream, partial, c, (int)m, (int)n, ldc,
                         p.splits, residual, ldr);
    } else {
      const size_t total = (size_t)m * n;
      const unsigned blocks = (unsigned)std::min((size_t)8192, (total + 255) / 256);
      hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, partial, c, (int)m, (int)n, ldc,
                         p.splits, residual, ldr);
    }
  }
  return hipGetLastError();
}

// What launch_sgemm_f32_ex queues for one product: the GEMV, or one or two
// MFMA products (rows [0, head_rows) and, after a tail split, the rest),
// optionally on padded copies of A and B.  A pure function of the shape,
// strides and operand alignment.
struct SgemmSchedule {
  bool gemv;
  bool tail_split;
  bool repack;         // A, B copied first to [m][k4] and [k4][n4], 16-byte rows, zero padding
  uint32_t k4, n4;     // padded K and B row stride when repacking
  uint32_t head_rows;  // rows of the first product (m without a tail split)
  SgemmPlan plan[2];
  double cost_us;      // plan-model estimate of the queued work
};

// One or two products (tail split) of an m x n x k problem with the given
// operand description.
SgemmSchedule schedule_products(bool aligned, int lda, int ldb, uint32_t m, uint32_t n, uint32_t k,
                                uint64_t max_partial_floats) {
  SgemmSchedule s{};
  s.head_rows = m;
  const bool scalar = !((k % 4 == 0) && (n % 4 == 0) && (lda % 4 == 0) && (ldb % 4 == 0) && aligned);
  s.plan[0] = plan_sgemm(aligned, lda, 0, ldb, 0, m, n, k, 1, max_partial_floats);
  s.cost_us = plan_cost(s.plan[0], m, n, 1, scalar);
  // A partial last row of 128-row tiles runs nearly empty for the whole K depth
  // (M = 1056: a 32-row tail in 9 tile rows).  When the estimate favours it, the
  // rows past the last full tile row run as a second product (usually K-split)
  // after the rest, on the same stream.  The tail starts 128 rows in, so its A
  // keeps the alignment of a when lda is a multiple of 4.
  const uint32_t tail = m % 128u;
  if (tail != 0 && m > 128u) {
    const uint32_t head = m - tail;
    const bool tail_aligned = aligned && (lda % 4 == 0);
    const SgemmPlan ph = plan_sgemm(aligned, lda, 0, ldb, 0, head, n, k, 1, max_partial_floats);
    const SgemmPlan pt = plan_sgemm(tail_aligned, lda, 0, ldb, 0, tail, n, k, 1, max_partial_floats);
    const double split_cost = plan_cost(ph, head, n, 1, scalar) + plan_cost(pt, tail, n, 1, scalar);
    if (split_cost < s.cost_us) {
      s.tail_split = true;
      s.head_rows = head;
      s.plan[0] = ph;
      s.plan[1] = pt;
      s.cost_us = split_cost;
    }
  }
  return s;
}

SgemmSchedule schedule_sgemm(bool aligned, int lda, int ldb, uint32_t m, uint32_t n, uint32_t k, bool has_residual,
                             uint64_t max_partial_floats) {
  SgemmSchedule s{};
  s.head_rows = m;
  if (n == 1 && !has_residual && ldb == 1 && lda == (int)k) {
    s.gemv = true;
    return s;
  }
  s = schedule_products(aligned, lda, ldb, m, n, k, max_partial_floats);
  // Operands the direct-to-LDS kernels cannot read (rows not 16-byte aligned,
  // k not a multiple of 4) otherwise run on the register-staged kernels; when
  // the estimate favours it they are first copied to padded buffers (two
  // launches, the copy at ~3 TB/s) and the fast kernels run on the copies.
  const bool direct = aligned && k % 4 == 0 && lda % 4 == 0 && ldb % 4 == 0;
  if (!direct) {
    const uint32_t k4 = (k + 3u) & ~3u, n4 = (n + 3u) & ~3u;
    if ((size_t)(m + 128) * k4 * 4 < (1ull << 31) && ((size_t)k4 * n4 + 256) * 4 < (1ull << 31)) {
      SgemmSchedule r = schedule_products(true, (int)k4, (int)n4, m, n, k4, max_partial_floats);
      const double bytes = 4.0 * ((double)m * k + (double)k * n + (double)m * k4 + (double)k4 * n4);
      r.cost_us += 4.0 + bytes / 3.0e6;
      if (r.cost_us < s.cost_us) {
        r.repack = true;
        r.k4 = k4;
        r.n4 = n4;
        return r;
      }
    }
  }
  return s;
}

uint64_t schedule_repack_floats(const SgemmSchedule& s, uint32_t m) {
  return s.repack ? (uint64_t)m * s.k4 + (uint64_t)s.k4 * s.n4 : 0;
}

// Queues schedule s; partial (null: runtime staging slot 6) receives the
// split-K slices and must hold partial_floats; packed (null: staging slots 8
// and 9) receives the padded copies of a repacking schedule, A then B.
hipError_t run_sgemm_schedule(const SgemmSchedule& s, const float* a, int lda, const float* b, int ldb, float* c,
                              int ldc, uint32_t m, uint32_t n, uint32_t k, const float* residual, int ldr,
                              float* partial, float* packed, hipStream_t stream) {
  if (s.gemv) {
    const bool vec = (k % 4 == 0) && aligned16(a) && aligned16(b);
    const dim3 grid((m + 3) / 4);
    if (vec)
      hipLaunchKernelGGL(gemv_f32_kernel<true>, grid, dim3(256), 0, stream, a, b, c, (int)m, (int)k);
    else
      hipLaunchKernelGGL(gemv_f32_kernel<false>, grid, dim3(256), 0, stream, a, b, c, (int)m, (int)k);
    return hipGetLastError();
  }
  if (s.repack) {
    float* pa = packed != nullptr ? packed : static_cast<float*>(staging(8, (size_t)m * s.k4 * sizeof(float)));
    float* pb = packed != nullptr ? packed + (size_t)m * s.k4
                                  : static_cast<float*>(staging(9, (size_t)s.k4 * s.n4 * sizeof(float)));
    if (pa == nullptr || pb == nullptr) return hipErrorOutOfMemory;
    const PadJob ja{a, pa, (int)m, (int)k, lda, (int)m, (int)s.k4};
    const PadJob jb{b, pb, (int)k, (int)n, ldb, (int)s.k4, (int)s.n4};
    const uint32_t blocks_a = pad_blocks(m, s.k4);
    const uint32_t blocks_b = pad_blocks(s.k4, s.n4);
    hipLaunchKernelGGL(pack_pad_kernel, dim3(blocks_a + blocks_b), dim3(256), 0, stream, ja, jb, blocks_a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    a = pa;
    lda = (int)s.k4;
    b = pb;
    ldb = (int)s.n4;
    k = s.k4;
  }
  auto run = [&](SgemmPlan p, const float* ap, float* cp, const float* rp, uint32_t rows) {
    float* part = nullptr;
    if (p.splits > 1) {
      part = partial != nullptr ? partial
                                : static_cast<float*>(staging(6, (size_t)p.splits * rows * n * sizeof(float)));
      if (part == nullptr) p = make_plan(p.tile, 1, k);
    }
    return run_sgemm_plan(p, ap, lda, 0, b, ldb, 0, cp, ldc, 0, rows, n, k, 1, rp, ldr, part, stream);
  };
  if (!s.tail_split) return run(s.plan[0], a, c, residual, m);
  const uint32_t head = s.head_rows;
  const hipError_t e = run(s.plan[0], a, c, residual, head);
  if (e != hipSuccess) return e;
  return run(s.plan[1], a + (size_t)head * lda, c + (size_t)head * ldc,
             residual ? residual + (size_t)head * ldr : nullptr, m - head);
}

uint64_t schedule_partial_floats(const SgemmSchedule& s, uint32_t m, uint32_t n) {
  if (s.gemv) return 0;
  uint64_t need = s.plan[0].splits > 1 ? (uint64_t)s.plan[0].splits * s.head_rows * n : 0;
  if (s.tail_split && s.plan[1].splits > 1)
    need = std::max<uint64_t>(need, (uint64_t)s.plan[1].splits * (m - s.head_rows) * n);
  return need;
}

// Floats of scratch the schedule needs in one array: the split-K partials
// rounded up to 256 bytes, then the padded copies of A and B.
uint64_t schedule_scratch_floats(const SgemmSchedule& s, uint32_t m, uint32_t n) {
  return ((schedule_partial_floats(s, m, n) + 63) & ~63ull) + schedule_repack_floats(s, m);
}

}  // namespace

hipError_t launch_sgemm_f32_ex(const float* a, int lda, const float* b, int ldb, float* c, int ldc, uint32_t m,
                               uint32_t n, uint32_t k, const float* residual, int ldr, hipStream_t stream,
                               int* path_detail) {
  const SgemmSchedule s =
      schedule_sgemm(aligned16(a) && aligned16(b), lda, ldb, m, n, k, residual != nullptr, ~0ull);
  if (path_detail) *path_detail = s.gemv ? PROM_DETAIL_PATH_HIP_GEMV_F32 : PROM_DETAIL_PATH_HIP_MFMA_F32;
  return run_sgemm_schedule(s, a, lda, b, ldb, c, ldc, m, n, k, residual, ldr, nullptr, nullptr, stream);
}

int sgemm_f32_unreduced_slices(int lda, int ldb, uint32_t m, uint32_t n, uint32_t k, int max_slices) {
  const SgemmSchedule s = schedule_sgemm(true, lda, ldb, m, n, k, false, ~0ull);
  if (s.gemv || s.repack || s.tail_split || s.plan[0].splits <= 1 || s.plan[0].splits > max_slices) return 1;
  return s.plan[0].splits;
}

hipError_t launch_sgemm_f32_unreduced(const float* a, int lda, const float* b, int ldb, float* c, int ldc,
                                      uint32_t m, uint32_t n, uint32_t k, float* partial, size_t partial_floats,
                                      int max_slices, hipStream_t stream, int* slices) {
  *slices = 1;
  const SgemmSchedule s = schedule_sgemm(aligned16(a) && aligned16(b), lda, ldb, m, n, k, false, ~0ull);
  if (s.gemv || s.repack || s.tail_split || s.plan[0].splits <= 1 || s.plan[0].splits > max_slices ||
      partial == nullptr || (uint64_t)s.plan[0].splits * m * n > partial_floats)
    return run_sgemm_schedule(s, a, lda, b, ldb, c, ldc, m, n, k, nullptr, 0, nullptr, nullptr, stream);
  *slices = s.plan[0].splits;
  return run_sgemm_plan(s.plan[0], a, lda, 0, b, ldb, 0, c, ldc, 0, m, n, k, 1, nullptr, 0, partial, stream,
                        false);
}

}  // namespace prom

// Scratch of the allocation-free entry (prometheus_reactor_runtime_sgemm_device_noalloc):
// the split-K partial slices go here instead of into runtime-allocated staging.
// Host code never takes this array's name as an address; init_sgemm_scratch
// obtains each device's copy with hipGetSymbolAddress once, at device set-up,
// and the kernels receive that pointer.
static __device__ __align__(256) float scratch[PROM_SGEMM_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace prom {
namespace {
constexpr int kScratchMaxDevices = 64;
float* g_scratch_ptr[kScratchMaxDevices];  // device address of `scratch` per device ordinal
}  // namespace

hipError_t init_sgemm_scratch(int device) {
  if (device < 0 || device >= kScratchMaxDevices) return hipErrorInvalidDevice;
  if (g_scratch_ptr[device] != nullptr) return hipSuccess;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    return e != hipSuccess ? e : hipErrorInvalidSymbol;
  }
  g_scratch_ptr[device] = static_cast<float*>(ptr);
  return hipSuccess;
}

int launch_sgemm_f32_noalloc(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                             int device, hipStream_t stream, int* path_detail) {
  float* part = (device >= 0 && device < kScratchMaxDevices) ? g_scratch_ptr[device] : nullptr;
  if (part == nullptr) return PROM_DETAIL_SCRATCH_UNAVAILABLE;
  // The same plan as launch_sgemm_f32 (bit-identical results); a plan whose
  // partials do not fit the array is refused rather than changed.
  // The split-K partials and, for a repacking plan, the padded operand
  // copies share the array: [partials | padded A | padded B].
  const SgemmSchedule s = schedule_sgemm(aligned16(a) && aligned16(b), (int)k, (int)n, m, n, k, false, ~0ull);
  const uint64_t part_floats = (schedule_partial_floats(s, m, n) + 63) & ~63ull;
  if (schedule_scratch_floats(s, m, n) * sizeof(float) > PROM_SGEMM_NOALLOC_SCRATCH_BYTES)
    return PROM_DETAIL_SCRATCH_LIMIT;
  if (path_detail) *path_detail = s.gemv ? PROM_DETAIL_PATH_HIP_GEMV_F32 : PROM_DETAIL_PATH_HIP_MFMA_F32;
  return run_sgemm_schedule(s, a, (int)k, b, (int)n, c, (int)n, m, n, k, nullptr, 0, part, part + part_floats,
                            stream) == hipSuccess
             ? PROM_OK
             : PROM_DETAIL_HIP_LAUNCH_FAILED;
}

hipError_t launch_sgemm_f32_geglu(const float* a, int lda, const float* w, float* h, int ldh, uint32_t m, uint32_t f,
                                  uint32_t k, hipStream_t stream) {
  if (m == 0 || f == 0 || k == 0) return hipErrorNotSupported;
  const int ldb = (int)(2 * f);
  const bool ok = f % 64 == 0 && buffer_path(aligned16(a) && aligned16(w), lda, 0, ldb, 0, m, 2 * f, k, (int)k, 4) &&
                  ldh % 4 == 0 && aligned16(h);
  if (!ok) return hipErrorNotSupported;
  const int tiles_m = (int)((m + 127) / 128), tiles_n = (int)(f / 64);
  hipLaunchKernelGGL(sgemm_f32_dl128w8_geglu_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, stream, a, w,
                     h, (int)m, (int)f, (int)k, tiles_m, tiles_n, lda, ldb, ldh);
  return hipGetLastError();
}

hipError_t launch_sgemm_f32_variant(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                                    uint32_t tile, uint32_t k_slices, hipStream_t stream) {
  if (tile >= (uint32_t)kTileShapes || k_slices < 1u || k_slices > 16u) return hipErrorInvalidValue;
  const SgemmPlan p = make_plan((int)tile, (int)k_slices, k);
  const bool aligned = aligned16(a) && aligned16(b);
  if (p.splits != (int)k_slices || (tile >= 3 && !buffer_path(aligned, (int)k, 0, (int)n, 0, m, n, k, p.k_len, tile)))
    return hipErrorInvalidValue;
  float* partial = nullptr;
  if (p.splits > 1) {
    partial = static_cast<float*>(staging(6, (size_t)p.splits * m * n * sizeof(float)));
    if (partial == nullptr) return hipErrorOutOfMemory;
  }
  return run_sgemm_plan(p, a, (int)k, 0, b, (int)n, 0, c, (int)n, 0, m, n, k, 1, nullptr, 0, partial, stream);
}

hipError_t launch_sgemm_f32_batched(const float* a, int lda, long long sa, const float* b, int ldb, long long sb,
                                    float* c, int ldc, long long sc, uint32_t m, uint32_t n, uint32_t k,
                                    uint32_t batch, hipStream_t stream) {
  if (batch == 0 || m == 0 || n == 0) return hipSuccess;
  if (batch == 1) return launch_sgemm_f32_ex(a, lda, b, ldb, c, ldc, m, n, k, nullptr, 0, stream, nullptr);
  return run_sgemm_plan(plan_sgemm(aligned16(a) && aligned16(b), lda, sa, ldb, sb, m, n, k, batch), a, lda, sa, b, ldb,
                        sb, c, ldc, sc, m, n, k, batch, nullptr, 0, nullptr, stream);
}

hipError_t launch_sgemm_f32(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                            hipStream_t stream, int* path_detail) {
  return launch_sgemm_f32_ex(a, (int)k, b, (int)n, c, (int)n, m, n, k, nullptr, 0, stream, path_detail);
}

}  // namespace prom

using namespace prom;

extern "C" PROM_REACTOR_API int prometheus_reactor_sgemm_plan(uint32_t m, uint32_t n, uint32_t k,
                                                              PrometheusSgemmPlanInfo* out_plan) {
  // Callers built before scratch_bytes existed pass the shorter struct; the
  // tail field is written only when the caller's struct holds it.
  if (out_plan == nullptr || out_plan->struct_size < offsetof(PrometheusSgemmPlanInfo, scratch_bytes))
    return PROM_ERROR;
  const uint32_t size = out_plan->struct_size;
  const bool has_scratch = size >= sizeof(PrometheusSgemmPlanInfo);
  memset(out_plan, 0, has_scratch ? sizeof(*out_plan) : offsetof(PrometheusSgemmPlanInfo, scratch_bytes));
  out_plan->struct_size = size;
  if (m == 0u || n == 0u || k == 0u) {
    out_plan->detail_code = PROM_ERROR;
    return PROM_ERROR;
  }
  if (!gemm_shape_fits(m, n, k)) {
    out_plan->detail_code = PROM_DETAIL_SIZE_OVERFLOW;
    return PROM_ERROR;
  }
  const SgemmSchedule s = schedule_sgemm(true, (int)k, (int)n, m, n, k, false, ~0ull);
  out_plan->head_rows = s.head_rows;
  if (s.gemv) {
    out_plan->detail_code = PROM_DETAIL_PATH_HIP_GEMV_F32;
    out_plan->launches = 1;
    return PROM_OK;
  }
  out_plan->detail_code = PROM_DETAIL_PATH_HIP_MFMA_F32;
  out_plan->products = s.tail_split ? 2u : 1u;
  out_plan->repacked = s.repack ? 1u : 0u;
  out_plan->repack_bytes = schedule_repack_floats(s, m) * sizeof(float);
  const uint32_t kk = s.repack ? s.k4 : k;
  const int ldb_eff = s.repack ? (int)s.n4 : (int)n;
  for (uint32_t i = 0; i < out_plan->products; ++i) {
    const SgemmPlan& p = s.plan[i];
    const uint32_t rows = i == 0 ? s.head_rows : m - s.head_rows;
    const bool buf = buffer_path(true, (int)kk, 0, ldb_eff, 0, rows, n, kk, p.k_len, p.tile);
    const int tile = (p.tile >= 3 && !buf) ? kStagedFallback[p.tile] : p.tile;
    out_plan->tile_m[i] = (uint32_t)kTileM[tile];
    out_plan->tile_n[i] = (uint32_t)kTileN[tile];
    out_plan->direct_to_lds[i] = tile >= 3 ? 1u : 0u;
    out_plan->k_slices[i] = (uint32_t)p.splits;
    out_plan->k_slice_len[i] = (uint32_t)p.k_len;
    out_plan->launches += p.splits > 1 ? 2u : 1u;
  }
  if (s.repack) out_plan->launches += 2u;
  out_plan->partial_bytes = schedule_partial_floats(s, m, n) * sizeof(float);
  out_plan->estimated_us = s.cost_us;
  if (has_scratch) out_plan->scratch_bytes = schedule_scratch_floats(s, m, n) * sizeof(float);
  return PROM_OK;
}
