// bf16 GEMM with fp32 accumulate on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// C[m,n] (fp32) = A[m,k] (bf16) @ B[k,n] (bf16), row-major.  The reference has
// no bf16 GEMM (its closest is fp16 storage / fp32 accumulate,
// internal/prometheus/shaders/sdslv/production/sgemm/sgemm_fp16_storage_fp32_accum.sdslv);
// the bf16 bit patterns and their fp32 widening follow
// internal/prometheus/gemma4e2b_m1_rtx.go:1005-1014.
//
//   * workgroup = 4 wave64, macro tile 128x128, K tile 64, LDS double-buffered;
//   * each wave owns 64x64 = 2x2 MFMA 32x32x16 blocks;
//   * MFMA operands want 8 consecutive k per lane, so A is stored [m][k] and
//     B is transposed into [n][k] on the way into LDS (pairs of k packed into
//     one 32-bit LDS store); operand reads are 128-bit;
//   * exact tails by zero-filled loads and masked stores; the 128-bit global
//     path needs k % 8 == 0 and n % 8 == 0, other shapes use 16-bit loads.
#include <type_traits>


#include "reactor_internal.h"

namespace prom {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kLds = kBK + 8;  // row pitch in bf16 elements (144 bytes, 16-byte aligned)
constexpr int kGroupM = 8;

// Round-to-nearest-even fp32 -> bf16, as gemma4e2b_m1_rtx.go:1009-1014 (finite inputs).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float v) {
  const uint32_t bits = __float_as_uint(v);
  return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

// xcd_pid gives each XCD a contiguous range of tile ids, so the tiles an XCD
// runs together are neighbours in the grouped order below and share their A
// and B panels in its L2.  (With the remap applied only when n % 8 == 0, the
// C5 QKV grid of 765 tiles gave each XCD one A panel and 32 B panels at a
// time.)
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

// Strides are leading dimensions in elements.  Epilogue: v = A@B (+ R when R is
// non-null, R may alias C); stored as fp32 into C, or as bf16 (round to nearest
// even) into Cb when Cb is non-null.
template <bool kVec>
__global__ __launch_bounds__(256, 2) void gemm_bf16_mfma_kernel(const uint16_t* __restrict__ A,
                                                                const uint16_t* __restrict__ B, float* C,
                                                                int M, int N, int K, int tiles_m, int tiles_n,
                                                                int lda, int ldb, int ldc, const float* R, int ldr,
                                                                uint16_t* Cb) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM][kLds];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][kBN][kLds];

  int tm, tn;
  map_tile(tiles_m, tiles_n, &tm, &tn);
  const int row0 = tm * kBM;
  const int col0 = tn * kBN;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;

  // A: thread -> (row = tid/2, 32 consecutive k starting at (tid%2)*32): 4 x 16 bytes.
  const int a_row = tid >> 1;
  const int a_k = (tid & 1) * 32;
  // B: unit u in {tid, tid+256}: k pair = u/16 (0..31), 8 consecutive n at (u%16)*8.
  u32x4 ra[4];
  u32x4 rb[4];  // [unit][row of pair]

  auto load_tile = [&](int k0) {
    const int gr = row0 + a_row;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int gk = k0 + a_k + 8 * h;
      u32x4 v = {0u, 0u, 0u, 0u};
      if constexpr (kVec) {
        if (gr < M && gk < K) v = *reinterpret_cast<const u32x4*>(A + (size_t)gr * lda + gk);
      } else {
        uint16_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = (gr < M && gk + j < K) ? A[(size_t)gr * lda + gk + j] : (uint16_t)0;
        v.x = (uint32_t)e[0] | ((uint32_t)e[1] << 16);
        v.y = (uint32_t)e[2] | ((uint32_t)e[3] << 16);
        v.z = (uint32_t)e[4] | ((uint32_t)e[5] << 16);
        v.w = (uint32_t)e[6] | ((uint32_t)e[7] << 16);
      }
      ra[h] = v;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int unit = tid + 256 * u;
      const int kp = unit >> 4;
      const int gn = col0 + (unit & 15) * 8;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int gk = k0 + 2 * kp + p;
        u32x4 v = {0u, 0u, 0u, 0u};
        if constexpr (kVec) {
          if (gk < K && gn < N) v = *reinterpret_cast<const u32x4*>(B + (size_t)gk * ldb + gn);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) e[j] = (gk < K && gn + j < N) ? B[(size_t)gk * ldb + gn + j] : (uint16_t)0;
          v.x = (uint32_t)e[0] | ((uint32_t)e[1] << 16);
          v.y = (uint32_t)e[2] | ((uint32_t)e[3] << 16);
          v.z = (uint32_t)e[4] | ((uint32_t)e[5] << 16);
          v.w = (uint32_t)e[6] | ((uint32_t)e[7] << 16);
        }
        rb[2 * u + p] = v;
      }
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 4; ++h) *reinterpret_cast<u32x4*>(&As[buf][a_row][a_k + 8 * h]) = ra[h];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int unit = tid + 256 * u;
      const int kp = unit >> 4;
      const int n0 = (unit & 15) * 8;
      const u32x4 lo = rb[2 * u + 0];  // row k = 2kp
      const u32x4 hi = rb[2 * u + 1];  // row k = 2kp + 1
      const uint32_t lw[4] = {lo.x, lo.y, lo.z, lo.w};
      const uint32_t hw[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // element n0+2j: low halves; element n0+2j+1: high halves
        const uint32_t even = (lw[j] & 0xFFFFu) | (hw[j] << 16);
        const uint32_t odd = (lw[j] >> 16) | (hw[j] & 0xFFFF0000u);
        *reinterpret_cast<uint32_t*>(&Bs[buf][n0 + 2 * j][2 * kp]) = even;
        *reinterpret_cast<uint32_t*>(&Bs[buf][n0 + 2 * j + 1][2 * kp]) = odd;
      }
    }
  };

  floatx16 acc00 = {}, acc01 = {}, acc10 = {}, acc11 = {};
  const int k_tiles = (K + kBK - 1) / kBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 8;
  const int am = wm * 64 + lrow;
  const int bn = wn * 64 + lrow;

  for (int kt = 0; kt < k_tiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < k_tiles;
    if (more) load_tile((kt + 1) * kBK);
#pragma unroll
    for (int s = 0; s < kBK / 16; ++s) {
      const int kc = 16 * s + lk;
      const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(&As[cur][am][kc]);
      const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(&As[cur][am + 32][kc]);
      const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(&Bs[cur][bn][kc]);
      const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(&Bs[cur][bn + 32][kc]);
      acc00 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc00, 0, 0, 0);
      acc01 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc01, 0, 0, 0);
      acc10 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc10, 0, 0, 0);
      acc11 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc11, 0, 0, 0);
    }
    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

  const int lgrp = (lane >> 5) * 4;
  auto store_block = [&](const floatx16& acc, int mi, int ni) {
    const int col = col0 + wn * 64 + ni * 32 + lrow;
    if (col >= N) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + wm * 64 + mi * 32 + 8 * (r >> 2) + lgrp + (r & 3);
      if (row < M) {
        float v = acc[r];
        if (R != nullptr) v += R[(size_t)row * ldr + col];
        if (Cb != nullptr)
          Cb[(size_t)row * ldc + col] = f32_to_bf16_rne(v);
        else
          C[(size_t)row * ldc + col] = v;
      }
    }
  };
  store_block(acc00, 0, 0);
  store_block(acc01, 0, 1);
  store_block(acc10, 1, 0);
  store_block(acc11, 1, 1);
}

// ---------------------------------------------------------------------------
// Large-tile kernel: 512 threads = 8 wave64, macro tile 256x256, K tile 64.
// Waves are 2 (m) x 4 (n); each owns 128x64 = 4x2 MFMA 32x32x16 blocks (128
// fp32 accumulators per lane).  A stays [m][k] in LDS (operands are 128-bit
// reads); B stays row-major [k][n] as it arrives from HBM, and each B operand
// is assembled with two ds_read_b64_tr_b16 transpose reads: within a 16-lane
// group, lane L points at row (L/4) and column 4*(L%4) of a 4x16 sub-block and
// receives the 4 k-consecutive values of column L.  No transposing stores.
// Requires k % 8 == 0, n % 8 == 0 (whole 16-byte chunks are in or out of range).
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kBM2 = 256;
constexpr int kBN2 = 256;
constexpr int kBK2 = 64;
constexpr int kLdsA2 = kBK2 + 8;   // 144-byte A rows
constexpr int kLdsB2 = kBN2 + 16;  // 544-byte B rows: 4 consecutive rows land on distinct banks

// Tile (tm, tn) of grouped position pid: groups of kGroupM rows of tiles,
// column-major inside a group.
__device__ __forceinline__ void pid_tile2(int pid, int tiles_m, int tiles_n, int* tm, int* tn) {
  const int per_group = kGroupM * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroupM;
  const int group_m = min(tiles_m - first_m, kGroupM);
  const int in_group = pid - group * per_group;
  *tm = first_m + in_group % group_m;
  *tn = in_group / group_m;
}

__device__ __forceinline__ void map_tile2(int tiles_m, int tiles_n, int* tm, int* tn) {
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

template <bool kBuf, int kStoreAt>
__global__ __launch_bounds__(512, 1) void gemm_bf16_mfma_256_kernel(const uint16_t* __restrict__ A,
                                                                   const uint16_t* __restrict__ B, float* C, int M,
                                                                   int N, int K, int tiles_m, int tiles_n, int lda,
                                                                   int ldb, int ldc, const float* R, int ldr,
                                                                   uint16_t* Cb) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM2][kLdsA2];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][kBK2][kLdsB2];

  int tm, tn;
  map_tile2(tiles_m, tiles_n, &tm, &tn);
  const int row0 = tm * kBM2;
  const int col0 = tn * kBN2;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2;  // 0..1
  const int wn = wave & 3;   // 0..3

  u32x4 ra[4], rb[4];
  // Branch-free path (kBuf): buffer loads return zero past the end of A or B, which
  // covers rows >= M and k >= K (K is a multiple of the K tile there); columns >= N
  // read the next row of B but only feed output columns that are never stored.
  const __amdgpu_buffer_rsrc_t rsa =
      __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, kBuf ? (int)((size_t)M * lda * 2) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb =
      __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, kBuf ? (int)((size_t)K * ldb * 2) : 0, 0x00020000);
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 512 * u;  // A: 256 rows x 8 chunks
      const int r = c >> 3;
      const int kc = (c & 7) * 8;
      const int gr = row0 + r, gk = k0 + kc;
      if constexpr (kBuf) {
        ra[u] = __builtin_amdgcn_raw_buffer_load_b128(rsa, (uint32_t)((gr * lda + gk) * 2), 0, 0);
      } else {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (gr < M && gk < K) v = *reinterpret_cast<const u32x4*>(A + (size_t)gr * lda + gk);
        ra[u] = v;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 512 * u;  // B: 64 k rows x 32 chunks
      const int kr = c >> 5;
      const int nc = (c & 31) * 8;
      const int gk = k0 + kr, gn = col0 + nc;
      if constexpr (kBuf) {
        rb[u] = __builtin_amdgcn_raw_buffer_load_b128(rsb, (uint32_t)((gk * ldb + gn) * 2), 0, 0);
      } else {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (gk < K && gn < N) v = *reinterpret_cast<const u32x4*>(B + (size_t)gk * ldb + gn);
        rb[u] = v;
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 512 * u;
      *reinterpret_cast<u32x4*>(&As[buf][c >> 3][(c & 7) * 8]) = ra[u];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 512 * u;
      *reinterpret_cast<u32x4*>(&Bs[buf][c >> 5][(c & 31) * 8]) = rb[u];
    }
  };

  floatx16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[i][0] = floatx16{};
    acc[i][1] = floatx16{};
  }

  const int k_tiles = (K + kBK2 - 1) / kBK2;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 8;
  // transpose-read coordinates inside a 16(k) x 32(n) operand block
  const int tr_row = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  for (int kt = 0; kt < k_tiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < k_tiles;
    if (more) load_tile((kt + 1) * kBK2);
#pragma unroll
    for (int s = 0; s < kBK2 / 16; ++s) {
      bf16x8 af[4], bfr[2];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
        af[mi] = *reinterpret_cast<const bf16x8*>(&As[cur][wm * 128 + mi * 32 + lrow][16 * s + lk]);
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int col = wn * 64 + ni * 32 + tr_col;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)(&Bs[cur][16 * s + tr_row][col]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)(&Bs[cur][16 * s + tr_row + 4][col]));
        const short w8[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        bfr[ni] = __builtin_bit_cast(bf16x8, w8);
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
      }
      // The other buffer was last read before the previous barrier, so the next
      // tile may be written into it at any point of this iteration.
      if (s == kStoreAt && more) store_tile(cur ^ 1);
    }
    __syncthreads();
  }

  const int lgrp = (lane >> 5) * 4;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int col = col0 + wn * 64 + ni * 32 + lrow;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = row0 + wm * 128 + mi * 32 + 8 * (r >> 2) + lgrp + (r & 3);
        if (row < M) {
          float v = acc[mi][ni][r];
          if (R != nullptr) v += R[(size_t)row * ldr + col];
          if (Cb != nullptr)
            Cb[(size_t)row * ldc + col] = f32_to_bf16_rne(v);
          else
            C[(size_t)row * ldc + col] = v;
        }
      }
    }
  }
}

// Direct-to-LDS variant of the 8-wave large tile.  Tiles travel HBM -> LDS
// with buffer_load_dwordx4 ... lds (no staging registers, no ds_write), so
// tile kt+1 streams into the other stage during all of tile kt's MFMAs.  Each
// wave instruction fills 1 KiB of LDS, lane i at +16*i, which fixes an
// unpadded layout; the global address each lane fetches applies an XOR
// swizzle on 16-byte chunks so that the MFMA operand reads are bank-conflict
// free: A (256 x 64, 128-byte rows) chunk c of row R sits at c ^ ((R&7) ^ ((R>>3)&1)),
// B (64 x 256, 512-byte rows) chunk c of row k at c ^ {0,4,10,14}[k&3].
// The two stages are separate LDS arrays and the K loop is unrolled by two so
// that reads of one stage are visibly independent of the DMA into the other.
__device__ __forceinline__ int swz_a(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int swz_b(int k) { return (0xEA40 >> (4 * (k & 3))) & 15; }  // {0,4,10,14}

//
// kSwiGLU: B is [K, 2F] = [W1 | W3] and the output is h = silu(x W1) * (x W3)
// in bf16 [M, F].  A tile then covers 128 output columns: in each wave's 64
// B columns the first 32 are gate (W1) columns and the last 32 the matching
// up (W3) columns, so accumulator blocks ni = 0 and 1 hold g and u of the same
// outputs and the product is formed in registers (N is F here).
template <bool kSwiGLU>
__global__ __launch_bounds__(512, 1) void gemm_bf16_mfma_dl_kernel(const uint16_t* __restrict__ A,
                                                                  const uint16_t* __restrict__ B, float* C, int M,
                                                                  int N, int K, int tiles_m, int tiles_n, int lda,
                                                                  int ldb, int ldc, const float* R, int ldr,
                                                                  uint16_t* Cb) {
  __shared__ __attribute__((aligned(1024))) uint16_t S0[2 * kBM2 * kBK2];
  __shared__ __attribute__((aligned(1024))) uint16_t S1[2 * kBM2 * kBK2];

  int tm, tn;
  map_tile2(tiles_m, tiles_n, &tm, &tn);
  const int row0 = tm * kBM2;
  const int col0 = kSwiGLU ? tn * (kBN2 / 2) : tn * kBN2;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2;
  const int wn = wave & 3;

  const __amdgpu_buffer_rsrc_t rsa =
      __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)((size_t)M * lda * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb =
      __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, (int)((size_t)K * ldb * 2), 0x00020000);

  // Per-lane source offsets (bytes) of this wave's 4 A and 4 B instructions at
  // k0 = 0; the k offset of a tile travels in the scalar soffset.
  uint32_t a_off[4], b_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = wave * 4 + i;
    const int r = 8 * q + (lane >> 3);
    const int c = (lane & 7) ^ swz_a(r);
    a_off[i] = (uint32_t)(((row0 + r) * lda + 8 * c) * 2);
    const int kr = 2 * q + (lane >> 5);
    const int cb = (lane & 31) ^ swz_b(kr);
    int gcol = col0 + 8 * cb;
    if constexpr (kSwiGLU) {
      const int e = 8 * cb;  // tile column: wave block e / 64, gate half if e % 64 < 32
      gcol = col0 + (e >> 6) * 32 + (e & 31) + ((e & 32) ? N : 0);
    }
    b_off[i] = (uint32_t)((kr * ldb + gcol) * 2);
  }
  typedef __attribute__((address_space(3))) void lds_void;
  auto issue = [&](uint16_t* stage, int k0) {
    const int sa = __builtin_amdgcn_readfirstlane(k0 * 2);
    const int sb = __builtin_amdgcn_readfirstlane(k0 * ldb * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = wave * 4 + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_void*)((char*)stage + q * 1024), 16, a_off[i], sa, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_void*)((char*)stage + 32768 + q * 1024), 16, b_off[i], sb,
                                               0, 0);
    }
  };

  // Operand addresses.  A row R = wm*128 + mi*32 + lrow has swizzle swz_a(lrow)
  // for every mi, and chunk 2s + hk = 2s ^ hk, so the byte address of step s is
  // a_base ^ (32 s) plus the immediate mi*4096.  B rows 16s + tr_row (+4) share
  // swizzle swz_b(tr_row); chunk (wn*8 + 4ni + x) ^ sw = ((wn*8 + x) ^ sw) ^ 4ni,
  // so its address is b_base ^ (64 ni) plus the immediates 8192 s (+2048).
  const int lrow = lane & 31;
  const int hk = lane >> 5;
  const int tr_row = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_e = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const uint32_t a_base = (uint32_t)((wm * 128 + lrow) * 128 + ((hk ^ swz_a(lrow)) << 4));
  const uint32_t b_base =
      (uint32_t)(32768 + tr_row * 512 + (((wn * 8 + (tr_e >> 3)) ^ swz_b(tr_row)) << 4) + (tr_e & 7) * 2);
  struct Frags {
    bf16x8 a[4], b[2];
  };
  auto read_frags = [&](const uint16_t* stage, int s) {
    Frags f;
    const char* st = (const char*)stage;
    const uint32_t as = a_base ^ (uint32_t)(32 * s);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) f.a[mi] = *reinterpret_cast<const bf16x8*>(st + as + mi * 4096);
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const uint32_t bs = (b_base ^ (uint32_t)(64 * ni)) + 8192 * s;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(st + bs));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(st + bs + 2048));
      f.b[ni] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
    return f;
  };

  floatx16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[i][0] = floatx16{};
    acc[i][1] = floatx16{};
  }
  auto compute = [&](const uint16_t* stage) {
#pragma unroll
    for (int s = 0; s < kBK2 / 16; ++s) {
      const Frags fc = read_frags(stage, s);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fc.a[mi], fc.b[ni], acc[mi][ni], 0, 0, 0);
    }
  };

  const int k_tiles = K / kBK2;
  issue(S0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int kt = 0; kt < k_tiles; ++kt) {
    // stage kt&1 holds tile kt; the other stage was last read before the previous barrier
    uint16_t* cur = (kt & 1) ? S1 : S0;
    uint16_t* nxt = (kt & 1) ? S0 : S1;
    if (kt + 1 < k_tiles) issue(nxt, (kt + 1) * kBK2);
    compute(cur);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  const int lgrp = (lane >> 5) * 4;
  if constexpr (kSwiGLU) {
    const int col = col0 + wn * 32 + lrow;
    if (col < N) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = row0 + wm * 128 + mi * 32 + 8 * (r >> 2) + lgrp + (r & 3);
          if (row < M) {
            const float g = acc[mi][0][r], u = acc[mi][1][r];
            Cb[(size_t)row * ldc + col] = f32_to_bf16_rne(silu_mul(g, u));
          }
        }
      }
    }
    return;
  }
  auto store_block = [&](const floatx16& v16, int mi, int ni) {
    const int col = col0 + wn * 64 + ni * 32 + lrow;
    if (col >= N) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + wm * 128 + mi * 32 + 8 * (r >> 2) + lgrp + (r & 3);
      if (row < M) {
        float v = v16[r];
        if (R != nullptr) v += R[(size_t)row * ldr + col];
        if (Cb != nullptr)
          Cb[(size_t)row * ldc + col] = f32_to_bf16_rne(v);
        else
          C[(size_t)row * ldc + col] = v;
      }
    }
  };
  store_block(acc[0][0], 0, 0);
  store_block(acc[0][1], 0, 1);
  store_block(acc[1][0], 1, 0);
  store_block(acc[1][1], 1, 1);
  store_block(acc[2][0], 2, 0);
  store_block(acc[2][1], 2, 1);
  store_block(acc[3][0], 3, 0);
  store_block(acc[3][1], 3, 1);
}

// Multi-stage variant of the direct-to-LDS kernel: K tile 32, five 32 KB LDS
// stages (the whole 160 KB), so each tile's transfers are issued four tiles
// ahead of its MFMAs (one 32-k step of the whole tile takes ~1000-1800 cycles
// per SIMD, the HBM and Infinity Cache latency is longer; five stages
// measured 1-3 % faster than four on the C5 shapes and 8192^3).  A rows are 64 bytes here: chunk c of row
// R sits at c ^ ((R >> 2) & 3); B keeps the 512-byte rows and swizzle above.
// Waits count this wave's outstanding transfers (4 per tile) and a bare
// s_barrier publishes a tile: transfers of the next tiles stay in flight
// across it.  Faster than the two-stage kernel on long K and on grids of more
// than one workgroup per CU (C5's QKV, W1|W3 and W2 products, 8192^3: 6-16 %),
// slower on single-round grids with K <= 4096 (4096^3: -9 %).
constexpr int kBK4 = 32;
constexpr int kStage4 = kBM2 * kBK4 * 2 + kBK4 * kBN2 * 2;  // 16 KB A + 16 KB B

// s_waitcnt vmcnt(n), as inline assembly: the compiler does not see the
// transfers (inline assembly), and could drop a builtin wait it considers
// already satisfied.
#define PROM_WAIT_VMCNT(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")

__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <bool kSwiGLU, int kSt>
__device__ __forceinline__ void gemm_bf16_dl4_body(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                   float* C, int M, int N, int K, int tm, int tn, int kt0,
                                                   int k_tiles, int lda, int ldb, int ldc, const float* R, int ldr,
                                                   uint16_t* Cb, float2* part, int a_slice, int h_slice,
                                                   char* const (&S)[kSt]) {
  const int row0 = tm * kBM2;
  const int col0 = kSwiGLU ? tn * (kBN2 / 2) : tn * kBN2;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2;
  const int wn = wave & 3;

  // This wave's 2 A instructions (rows 16q..16q+15, 4 lanes per row) and 2 B
  // instructions (k rows 2q, 2q+1, 32 lanes per row), q = 2 wave + i.
  uint32_t a_off[2], b_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = wave * 2 + i;
    const int r = 16 * q + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    a_off[i] = a_slice > 0 ? (uint32_t)(((row0 + r) * 32 + 8 * c) * 2) : (uint32_t)(((row0 + r) * lda + 8 * c) * 2);
    const int kr = 2 * q + (lane >> 5);
    const int cb = (lane & 31) ^ swz_b(kr);
    int gcol = col0 + 8 * cb;
    if constexpr (kSwiGLU) {
      const int e = 8 * cb;
      gcol = col0 + (e >> 6) * 32 + (e & 31) + ((e & 32) ? N : 0);
    }
    b_off[i] = (uint32_t)((kr * ldb + gcol) * 2);
  }
  // The transfers are written as inline assembly (M0 = LDS destination of
  // the wave's 1 KB, 16 bytes per lane; buffer descriptors built here, raw,
  // range-checked: out-of-range rows read zero).  The compiler then does not
  // track them as LDS stores, so it adds no conservative vmcnt(0) before the
  // LDS reads of the other stages; the explicit vmcnt waits and barriers of the
  // K loop order every transfer before the reads of its tile.  M0 is declared
  // clobbered, so the compiler keeps no live value in it across a transfer.
  typedef int int4v __attribute__((ext_vector_type(4)));
  auto desc = [](const void* p, uint32_t bytes) {
    const unsigned long long a = (unsigned long long)p;
    int4v d;
    d.x = __builtin_amdgcn_readfirstlane((int)(a & 0xffffffffu));
    d.y = __builtin_amdgcn_readfirstlane((int)(a >> 32));
    d.z = __builtin_amdgcn_readfirstlane((int)bytes);
    d.w = 0x00020000;
    return d;
  };
  const int4v da = desc(A, (uint32_t)(a_slice > 0 ? (size_t)K * a_slice * 2 : (size_t)M * lda * 2));
  const int4v db = desc(B, (uint32_t)((size_t)K * ldb * 2));
  // Transfer j (0..3) of this wave for the tile at k0: A rows (j even) or B
  // rows (j odd) of instruction i = j / 2.
  auto issue_one = [&](char* stage, int k0, int j) __attribute__((always_inline)) {
    const int i = j >> 1;
    const int q = wave * 2 + i;
    const uint32_t base = (uint32_t)(size_t)(__attribute__((address_space(3))) char*)stage;
    if ((j & 1) == 0) {
      const int sa = __builtin_amdgcn_readfirstlane(a_slice > 0 ? k0 * a_slice * 2 : k0 * 2);
      const uint32_t la = __builtin_amdgcn_readfirstlane(base + q * 1024);
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(la), "v"(a_off[i]), "s"(da),
                   "s"(sa)
                   : "memory", "m0");
    } else {
      const int sb = __builtin_amdgcn_readfirstlane(k0 * ldb * 2);
      const uint32_t lb = __builtin_amdgcn_readfirstlane(base + 16384 + q * 1024);
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lb), "v"(b_off[i]), "s"(db),
                   "s"(sb)
                   : "memory", "m0");
    }
  };
  auto issue = [&](char* stage, int k0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) issue_one(stage, k0, j);
  };

  const int lrow = lane & 31;
  const int hk = lane >> 5;
  const int tr_row = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_e = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const uint32_t a_base = (uint32_t)((wm * 128 + lrow) * 64 + ((hk ^ ((lrow >> 2) & 3)) << 4));
  const uint32_t b_base =
      (uint32_t)(16384 + tr_row * 512 + (((wn * 8 + (tr_e >> 3)) ^ swz_b(tr_row)) << 4) + (tr_e & 7) * 2);

  floatx16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[i][0] = floatx16{};
    acc[i][1] = floatx16{};
  }
  struct Frags {
    bf16x8 a[4], b[2];
  };
  auto read = [&](const char* st, int s) {
    Frags f;
    const uint32_t as = a_base ^ (uint32_t)(32 * s);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) f.a[mi] = *reinterpret_cast<const bf16x8*>(st + as + mi * 2048);
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const uint32_t bs = (b_base ^ (uint32_t)(64 * ni)) + 8192 * s;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(st + bs));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(st + bs + 2048));
      f.b[ni] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
    return f;
  };
  // Step t: wait until this wave's transfers of tile t+1 have landed (the
  // kSt-3 tiles after it may stay in flight), barrier (tile t+1 complete for
  // all waves, tile t-1's stage free), issue tile t+kSt-1 into that stage, run
  // tile t, and read the first fragments of tile t+1 before the next barrier.
  // u = t % kSt is a compile-time constant (the loop is unrolled by kSt).
  auto wait_tiles = [&](int in_flight) {
    if (in_flight >= 2)
      PROM_WAIT_VMCNT(8);
    else if (in_flight == 1)
      PROM_WAIT_VMCNT(4);
    else
      PROM_WAIT_VMCNT(0);
  };
  Frags f0;
  // The tile's 16 MFMAs run in four groups of four, each followed by one of
  // the wave's four transfers of tile t+kSt-1: issued all at once after the
  // barrier, the 32 transfers of a workgroup queue at the texture unit and
  // hold back the MFMAs of the waves that issue them last.
  auto mma_quarter = [&](const Frags& f, int h) __attribute__((always_inline)) {
#pragma unroll
    for (int mi = 2 * h; mi < 2 * h + 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[mi], f.b[ni], acc[mi][ni], 0, 0, 0);
  };
  auto step = [&](int t, auto u_c) {
    constexpr int u = decltype(u_c)::value;
    wait_tiles(min(kSt - 3, k_tiles - t - 2));
    stage_barrier();
    const bool more = t + kSt - 1 < k_tiles;
    char* const next = S[(u + kSt - 1) % kSt];
    const int k_next = (kt0 + t + kSt - 1) * kBK4;
    const Frags f1 = read(S[u], 1);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      mma_quarter(g < 2 ? f0 : f1, g & 1);
      if (more) issue_one(next, k_next, g);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (t + 1 < k_tiles) f0 = read(S[(u + 1) % kSt], 0);
  };
#pragma unroll
  for (int j = 0; j < kSt - 1; ++j)
    if (j < k_tiles) issue(S[j], (kt0 + j) * kBK4);
  wait_tiles(min(kSt - 2, k_tiles - 1));  // tile 0 complete before its first reads
  stage_barrier();
  f0 = read(S[0], 0);
  const std::integral_constant<int, 0> u0{};
  const std::integral_constant<int, 1> u1{};
  const std::integral_constant<int, 2> u2{};
  const std::integral_constant<int, 3> u3{};
  const std::integral_constant<int, 4> u4{};
  int t = 0;
  for (; t + kSt <= k_tiles; t += kSt) {
    step(t, u0);
    step(t + 1, u1);
    step(t + 2, u2);
    step(t + 3, u3);
    if constexpr (kSt == 5) step(t + 4, u4);
  }
  if (t < k_tiles) step(t, u0);
  if (t + 1 < k_tiles) step(t + 1, u1);
  if (t + 2 < k_tiles) step(t + 2, u2);
  if constexpr (kSt == 5)
    if (t + 3 < k_tiles) step(t + 3, u3);

  const int lgrp = hk * 4;
  if constexpr (kSwiGLU) {
    const int col = col0 + wn * 32 + lrow;
    if (part != nullptr) {
      // one K slice of a split tile: the raw (gate, up) sums, [256 rows][128 columns]
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        const int rl = wm * 128 + mi * 32 + lgrp;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = 8 * (r >> 2) + (r & 3);
          if (row0 + rl + dr < M) part[(size_t)(rl + dr) * 128 + (col - col0)] = make_float2(acc[mi][0][r], acc[mi][1][r]);
        }
      }
      return;
    }
    if (col < N) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        const int rb = row0 + wm * 128 + mi * 32 + lgrp;
        // K-blocked H (h_slice rows per 32-column slice): a row step is 32
        uint16_t* hp = h_slice > 0 ? Cb + ((size_t)(col >> 5) * h_slice + rb) * 32 + (col & 31)
                                   : Cb + (size_t)rb * ldc + col;
        const size_t hstep = h_slice > 0 ? 32 : (size_t)ldc;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = 8 * (r >> 2) + (r & 3);
          if (rb + dr < M) {
            const float g = acc[mi][0][r], u = acc[mi][1][r];
            hp[(size_t)dr * hstep] = f32_to_bf16_rne(silu_mul(g, u));
          }
        }
      }
    }
    return;
  }
  auto store_block = [&](const floatx16& v16, int mi, int ni) {
    const int col = col0 + wn * 64 + ni * 32 + lrow;
    if (col >= N) return;
    const int rb = row0 + wm * 128 + mi * 32 + lgrp;
    const float* rp = R != nullptr ? R + (size_t)rb * ldr + col : nullptr;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int dr = 8 * (r >> 2) + (r & 3);
      if (rb + dr < M) {
        float v = v16[r];
        if (rp != nullptr) v += rp[(size_t)dr * ldr];
        if (Cb != nullptr)
          Cb[(size_t)(rb + dr) * ldc + col] = f32_to_bf16_rne(v);
        else
          C[(size_t)(rb + dr) * ldc + col] = v;
      }
    }
  };
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    store_block(acc[mi][0], mi, 0);
    store_block(acc[mi][1], mi, 1);
  }
}

__global__ __launch_bounds__(512, 1) void gemm_bf16_dl4_kernel(const uint16_t* __restrict__ A,
                                                              const uint16_t* __restrict__ B, float* C, int M, int N,
                                                              int K, int tiles_m, int tiles_n, int lda, int ldb,
                                                              int ldc, const float* R, int ldr, uint16_t* Cb,
                                                              int a_slice) {
  __shared__ __attribute__((aligned(1024))) char S0[kStage4];
  __shared__ __attribute__((aligned(1024))) char S1[kStage4];
  __shared__ __attribute__((aligned(1024))) char S2[kStage4];
  __shared__ __attribute__((aligned(1024))) char S3[kStage4];
  __shared__ __attribute__((aligned(1024))) char S4[kStage4];
  char* const st[5] = {S0, S1, S2, S3, S4};
  int tm, tn;
  map_tile2(tiles_m, tiles_n, &tm, &tn);
  gemm_bf16_dl4_body<false>(A, B, C, M, N, K, tm, tn, 0, K / kBK4, lda, ldb, ldc, R, ldr, Cb, nullptr, a_slice, 0,
                            st);
}

// Workgroups b < n_main take whole tiles (pids 0 .. n_main-1, XCD-contiguous);
// the rest take one of `splits` K slices of the tiles n_main .. (tiles of a
// final partial wave, split so that they fill it), writing their raw sums to
// part for swiglu_splitk_kernel.
__global__ __launch_bounds__(512, 1) void gemm_bf16_dl4_swiglu_kernel(const uint16_t* __restrict__ A,
                                                                     const uint16_t* __restrict__ B, int M, int N,
                                                                     int K, int tiles_m, int tiles_n, int lda, int ldb,
                                                                     int ldh, uint16_t* H, int n_main, int splits,
                                                                     float2* part, int a_slice, int h_slice) {
  __shared__ __attribute__((aligned(1024))) char S0[kStage4];
  __shared__ __attribute__((aligned(1024))) char S1[kStage4];
  __shared__ __attribute__((aligned(1024))) char S2[kStage4];
  __shared__ __attribute__((aligned(1024))) char S3[kStage4];
  __shared__ __attribute__((aligned(1024))) char S4[kStage4];
  char* const st[5] = {S0, S1, S2, S3, S4};
  const int b = (int)blockIdx.x;
  const int k_tiles = K / kBK4;
  int pid = 0, kt0 = 0, kn = k_tiles;
  float2* dst = nullptr;
  if (b < n_main) {
    pid = xcd_pid(b, n_main);
  } else {
    const int j = b - n_main;
    const int s = j % splits;
    pid = n_main + j / splits;
    kt0 = s * k_tiles / splits;
    kn = (s + 1) * k_tiles / splits - kt0;
    dst = part + (size_t)j * (kBM2 * 128);
  }
  int tm, tn;
  pid_tile2(pid, tiles_m, tiles_n, &tm, &tn);
  gemm_bf16_dl4_body<true>(A, B, nullptr, M, N, K, tm, tn, kt0, kn, lda, ldb, ldh, nullptr, 0, H, dst, a_slice,
                           h_slice, st);
}

// h = silu(g) * u for the split tiles: (g, u) summed over the K slices in
// slice order, then silu_mul as in the GEMM epilogue.
__global__ __launch_bounds__(256) void swiglu_splitk_kernel(const float2* __restrict__ part, uint16_t* __restrict__ H,
                                                            int ldh, int M, int tiles_m, int tiles_n, int n_main,
                                                            int splits, int h_slice) {
  const int ti = (int)blockIdx.y;
  const int e = (int)(blockIdx.x * 256 + threadIdx.x);  // element of the 256 x 128 tile
  const int rl = e >> 7, cl = e & 127;
  int tm, tn;
  pid_tile2(n_main + ti, tiles_m, tiles_n, &tm, &tn);
  const int row = tm * kBM2 + rl;
  if (row >= M) return;
  const float2* p = part + (size_t)ti * splits * (kBM2 * 128) + e;
  float g = p[0].x, u = p[0].y;
  for (int s = 1; s < splits; ++s) {
    g += p[(size_t)s * (kBM2 * 128)].x;
    u += p[(size_t)s * (kBM2 * 128)].y;
  }
  const int col = tn * 128 + cl;
  const size_t at = h_slice > 0 ? ((size_t)(col >> 5) * h_slice + row) * 32 + (col & 31) : (size_t)row * ldh + col;
  H[at] = f32_to_bf16_rne(silu_mul(g, u));
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The four-stage kernel wins once a CU runs more than one tile in turn or the
// K loop is long (measured on MI355X; see its comment).
// The multi-stage kernel from 240 tiles (C5's 255-tile output projection:
// 115.3 -> 111.7 us) or K >= 8192.
inline bool use_four_stage(int tiles, uint32_t k) { return tiles >= 240 || k >= 8192; }

}  // namespace

namespace {

enum class Bf16Path { kFourStage, kTwoStage, kStaged256, kSmall };

// The kernel launch_gemm_bf16_ex runs for a shape and its operands' layout.
Bf16Path bf16_path(const uint16_t* a, int lda, const uint16_t* b, int ldb, uint32_t m, uint32_t n, uint32_t k,
                   bool* vec_out) {
  const bool vec = (k % 8 == 0) && (n % 8 == 0) && (lda % 8 == 0) && (ldb % 8 == 0) && aligned16(a) && aligned16(b);
  if (vec_out) *vec_out = vec;
  const int tiles = (int)((m + kBM2 - 1) / kBM2) * (int)((n + kBN2 - 1) / kBN2);
  if (!vec || tiles < 128) return Bf16Path::kSmall;
  const bool range = (size_t)(m + kBM2) * lda * 2 < (1ull << 31) && (size_t)k * ldb * 2 < (1ull << 31);
  if (range && k % kBK4 == 0 && use_four_stage(tiles, k)) return Bf16Path::kFourStage;
  if (range && k % kBK2 == 0) return Bf16Path::kTwoStage;
  return Bf16Path::kStaged256;
}

bool swiglu_fused_ok(const uint16_t* a, int lda, const uint16_t* w13, uint32_t m, uint32_t f, uint32_t k) {
  return f % 128 == 0 && k % kBK4 == 0 && lda % 8 == 0 && aligned16(a) && aligned16(w13) &&
         (size_t)(m + kBM2) * lda * 2 < (1ull << 31) && (size_t)k * 2 * f * 2 < (1ull << 31);
}

// K-blocked A ([k/32][a_slice][32], a_slice >= m rounded up to 256 rows) keeps
// every byte offset below 2^31.
bool blocked_range(int a_slice, uint32_t m, uint32_t k) {
  return a_slice >= (int)((m + kBM2 - 1) / kBM2 * kBM2) && (size_t)k * a_slice * 2 < (1ull << 31);
}

}  // namespace

bool gemm_bf16_takes_blocked_a(const uint16_t* a, int lda, const uint16_t* b, int ldb, uint32_t m, uint32_t n,
                               uint32_t k) {
  return bf16_path(a, lda, b, ldb, m, n, k, nullptr) == Bf16Path::kFourStage;
}

bool gemm_bf16_swiglu_takes_blocked_a(const uint16_t* a, int lda, const uint16_t* w13, uint32_t m, uint32_t f,
                                      uint32_t k) {
  const int tiles = (int)((m + kBM2 - 1) / kBM2) * (int)(f / 128);
  return swiglu_fused_ok(a, lda, w13, m, f, k) && use_four_stage(tiles, k);
}

hipError_t launch_gemm_bf16_ex(const uint16_t* a, int lda, const uint16_t* b, int ldb, float* c, uint16_t* cb,
                               int ldc, uint32_t m, uint32_t n, uint32_t k, const float* residual, int ldr,
                               hipStream_t stream, int* path_detail, int a_slice) {
  bool vec = false;
  const Bf16Path path = bf16_path(a, lda, b, ldb, m, n, k, &vec);
  if (a_slice > 0 && (path != Bf16Path::kFourStage || !blocked_range(a_slice, m, k))) return hipErrorNotSupported;
  if (path != Bf16Path::kSmall) {
    const int tiles_m2 = (int)((m + kBM2 - 1) / kBM2);
    const int tiles_n2 = (int)((n + kBN2 - 1) / kBN2);
    const dim3 grid2((unsigned)(tiles_m2 * tiles_n2));
    if (path == Bf16Path::kFourStage)
      hipLaunchKernelGGL(gemm_bf16_dl4_kernel, grid2, dim3(512), 0, stream, a, b, c, (int)m, (int)n, (int)k, tiles_m2,
                         tiles_n2, lda, ldb, ldc, residual, ldr, cb, a_slice);
    else if (path == Bf16Path::kTwoStage)
      hipLaunchKernelGGL(gemm_bf16_mfma_dl_kernel<false>, grid2, dim3(512), 0, stream, a, b, c, (int)m, (int)n, (int)k,
                         tiles_m2, tiles_n2, lda, ldb, ldc, residual, ldr, cb);
    else
      hipLaunchKernelGGL((gemm_bf16_mfma_256_kernel<false, 1>), grid2, dim3(512), 0, stream, a, b, c, (int)m, (int)n,
                         (int)k, tiles_m2, tiles_n2, lda, ldb, ldc, residual, ldr, cb);
    if (path_detail) *path_detail = PROM_DETAIL_PATH_HIP_MFMA_BF16;
    return hipGetLastError();
  }
  const int tiles_m = (int)((m + kBM - 1) / kBM);
  const int tiles_n = (int)((n + kBN - 1) / kBN);
  const dim3 grid((unsigned)(tiles_m * tiles_n));
  if (vec)
    hipLaunchKernelGGL(gemm_bf16_mfma_kernel<true>, grid, dim3(256), 0, stream, a, b, c, (int)m, (int)n, (int)k,
                       tiles_m, tiles_n, lda, ldb, ldc, residual, ldr, cb);
  else
    hipLaunchKernelGGL(gemm_bf16_mfma_kernel<false>, grid, dim3(256), 0, stream, a, b, c, (int)m, (int)n, (int)k,
                       tiles_m, tiles_n, lda, ldb, ldc, residual, ldr, cb);
  if (path_detail) *path_detail = PROM_DETAIL_PATH_HIP_MFMA_BF16;
  return hipGetLastError();
}

hipError_t launch_gemm_bf16_swiglu(const uint16_t* a, int lda, const uint16_t* w13, uint16_t* h, int ldh, uint32_t m,
                                   uint32_t f, uint32_t k, hipStream_t stream, void* part_ws, size_t part_bytes,
                                   uint32_t* launches, int a_slice, int h_slice) {
  if (launches) *launches = 1;
  // Fused path conditions: whole 128-column output tiles, K a multiple of the K
  // tile, 16-byte aligned rows, byte offsets below 2^31; otherwise the caller
  // runs the GEMM and the elementwise SwiGLU separately.
  if (!swiglu_fused_ok(a, lda, w13, m, f, k)) return hipErrorNotSupported;
  const int tiles_m2 = (int)((m + kBM2 - 1) / kBM2);
  const int tiles_n2 = (int)(f / 128);
  const dim3 grid((unsigned)(tiles_m2 * tiles_n2));
  const bool four = use_four_stage(tiles_m2 * tiles_n2, k);
  // K-blocked A or H only on the four-stage kernel.
  if ((a_slice > 0 && (!four || !blocked_range(a_slice, m, k))) ||
      (h_slice > 0 && (!four || h_slice < tiles_m2 * kBM2 || (size_t)f * h_slice * 2 >= (1ull << 31))))
    return hipErrorInvalidValue;
  if (four) {
    // One workgroup per CU: the tiles of a final wave that would run at most
    // half full are split along K into as many slices as fill it (at most 4,
    // each of 4 K tiles or more), their partial sums going to part_ws.
    const int total = tiles_m2 * tiles_n2;
    const int cus = ctx().props.multiProcessorCount > 0 ? ctx().props.multiProcessorCount : 256;
    const int rem = total % cus;
    const int splits = rem > 0 ? std::min(cus / rem, 4) : 0;
    const int k_tiles = (int)(k / kBK4);
    const size_t need = (size_t)rem * splits * kBM2 * 128 * sizeof(float2);
    if (total > cus && splits >= 2 && k_tiles >= 4 * splits && part_ws != nullptr && need <= part_bytes) {
      const int n_main = total - rem;
      hipLaunchKernelGGL(gemm_bf16_dl4_swiglu_kernel, dim3((unsigned)(n_main + rem * splits)), dim3(512), 0, stream, a,
                         w13, (int)m, (int)f, (int)k, tiles_m2, tiles_n2, lda, (int)(2 * f), ldh, h, n_main, splits,
                         reinterpret_cast<float2*>(part_ws), a_slice, h_slice);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(swiglu_splitk_kernel, dim3(kBM2 * 128 / 256, (unsigned)rem), dim3(256), 0, stream,
                         reinterpret_cast<const float2*>(part_ws), h, ldh, (int)m, tiles_m2, tiles_n2, n_main, splits,
                         h_slice);
      if (launches) *launches = 2;
    } else {
      hipLaunchKernelGGL(gemm_bf16_dl4_swiglu_kernel, grid, dim3(512), 0, stream, a, w13, (int)m, (int)f, (int)k,
                         tiles_m2, tiles_n2, lda, (int)(2 * f), ldh, h, total, 1, nullptr, a_slice, h_slice);
    }
  } else if (k % kBK2 == 0)
    hipLaunchKernelGGL(gemm_bf16_mfma_dl_kernel<true>, grid, dim3(512), 0, stream, a, w13, nullptr, (int)m, (int)f,
                       (int)k, tiles_m2, tiles_n2, lda, (int)(2 * f), ldh, nullptr, 0, h);
  else
    return hipErrorNotSupported;
  return hipGetLastError();
}

hipError_t launch_gemm_bf16(const uint16_t* a, const uint16_t* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                            hipStream_t stream, int* path_detail) {
  return launch_gemm_bf16_ex(a, (int)k, b, (int)n, c, nullptr, (int)n, m, n, k, nullptr, 0, stream, path_detail, 0);
}

}  // namespace prom
