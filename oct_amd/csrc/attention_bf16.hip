// Flash-style bf16 attention on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// O = softmax(Q K^T * scale) V per head, full (non-causal) attention, head_dim
// 128; Q, K, V, O are bf16 [T, ld] with head h at column h*128.  The
// reference's attention (main_transformer_joint_attention_streaming.sdslv:23-86)
// keeps a whole score row in LDS, one workgroup per (token, head), and caps the
// sequence at 1056 keys; this kernel streams K/V tiles with an online softmax
// so the sequence length is unbounded.
//
//   * workgroup = 4 wave64 = 128 queries of one head; each wave owns 32 queries;
//   * per 64-key tile: K and V [64][128] are staged in LDS in their HBM layout,
//     double-buffered (the next tile is fetched into registers during the
//     current tile's MFMAs);
//   * scores are computed transposed, S^T = K Q^T, so that a lane owns one
//     query and 32 of its scores: the row max / row sum need one cross-lane
//     step (lanes l and l^32), not a 32-lane reduction;
//   * O^T = V^T P^T accumulates in 4 MFMA blocks (128 d x 32 queries); P
//     stays in registers: the key order inside each 16-key MFMA step is the
//     permutation the S^T accumulator layout hands out, and the V^T operand is
//     built in the same key order by two ds_read_b64_tr_b16 transpose reads;
//   * softmax runs in the log2 domain: max on raw scores, one FMA and one
//     v_exp_f32 per score, running max/sum in fp32; O is rescaled only when
//     some query's maximum grew (in the DMA-fed kernel only when it grew by
//     more than 2^8, see kLazyLog2); masking only on the last, partial tile.
//     The DiT block's queries and keys are per-head RMS-normalised, which
//     bounds every score; when the bound allows (kDirectLog2) the kernel
//     takes p = 2^s with no running maximum at all, one v_exp_f32 per score;
//     P and O go to bf16 with the hardware round-to-nearest-even pair
//     conversion (VALU work per tile is the bound of this kernel, not MFMA);
//   * the output tile is staged through LDS for 128-bit coalesced stores;
//   * the 1-D grid runs a head's query blocks on one XCD (block_coords).
//
// Two kernels share that design: flash_attn_bf16_dma_kernel (the DiT block's,
// tiles moved HBM -> LDS by DMA, less VALU work per tile; see its comment)
// and flash_attn_bf16_kernel (tiles staged through registers), kept as the
// cross-check of the parity tests.
#include <type_traits>

#include "reactor_internal.h"

namespace prom {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kD = 128;     // head dim
constexpr int kQW = 32;     // queries per wave
constexpr int kKB = 64;     // keys per tile
constexpr int kKP = kD + 8;   // K row pitch (bf16): 68 words, 16 rows on distinct 16-byte bank groups
constexpr int kVP = kD + 16;  // V row pitch (bf16): 72 words, 4 consecutive rows on distinct banks
constexpr float kNegBig = -1.0e30f;
// Growth of a query's maximum (log2 units) below which the DMA-fed kernel
// keeps the older maximum as the softmax reference:
// probabilities then reach 2^8 before O/l normalises them, well inside bf16
// and fp32 range, and the result is the same softmax.
constexpr float kLazyLog2 = 8.0f;
// Largest score magnitude (log2 units) for which the DiT kernel drops the
// running maximum: with |s| <= 64, p = 2^s and the running sum of up to 2^31
// keys stay far inside fp32 and bf16 range and never underflow to zero.
constexpr float kDirectLog2 = 64.0f;

// The grid is 1-D over (head, query block) pairs, head-major, renumbered by
// xcd_pid: an XCD runs the query blocks of one or two heads at a time, so a
// K/V tile reaches its L2 once per head instead of once per query block (with
// the blocks of a head spread over all 8 XCDs, each L2 held tiles of about 8
// heads at once).
__device__ __forceinline__ void block_coords(int T, int* head, int* qb) {
  const int nqb = (T + 4 * kQW - 1) / (4 * kQW);
  const int p = xcd_pid((int)blockIdx.x, (int)gridDim.x);
  *head = p / nqb;
  *qb = p - *head * nqb;
}

__global__ __launch_bounds__(256, 2) void flash_attn_bf16_kernel(const uint16_t* __restrict__ Q,
                                                                 const uint16_t* __restrict__ K,
                                                                 const uint16_t* __restrict__ V,
                                                                 uint16_t* __restrict__ O, int T, int ldq, int ldk,
                                                                 int ldv, int ldo, float scale_log2) {
  // K and V tiles are [64 keys][128 d], double-buffered; V keeps its HBM
  // layout and its operand is assembled with LDS transpose reads.
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kKB][kKP];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][kKB][kVP];

  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int head, qb;
  block_coords(T, &head, &qb);
  const int q0 = qb * (4 * kQW) + wave * kQW;
  const int lq = lane & 31;
  const int hi = lane >> 5;  // lane half
  const int qi = q0 + lq;

  // Q^T operand (B of S^T = K Q^T): lane holds Q[qi][16s + 8*hi .. +7] for s = 0..7.
  bf16x8 qf[8];
  {
    const uint16_t* qrow = Q + (size_t)qi * ldq + head * kD;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (qi < T) v = *reinterpret_cast<const u32x4*>(qrow + 16 * s + 8 * hi);
      qf[s] = __builtin_bit_cast(bf16x8, v);
    }
  }

  // global -> register staging for one K tile and one V tile: 1024 + 1024
  // 16-byte chunks, 4 + 4 per thread
  u32x4 rk[4], rv[4];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 256 * u;
      const int key = c >> 4;
      const int dc = (c & 15) * 8;
      u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
      if (k0 + key < T) {
        kv = *reinterpret_cast<const u32x4*>(K + (size_t)(k0 + key) * ldk + head * kD + dc);
        vv = *reinterpret_cast<const u32x4*>(V + (size_t)(k0 + key) * ldv + head * kD + dc);
      }
      rk[u] = kv;
      rv[u] = vv;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 256 * u;
      *reinterpret_cast<u32x4*>(&Ks[buf][c >> 4][(c & 15) * 8]) = rk[u];
      *reinterpret_cast<u32x4*>(&Vs[buf][c >> 4][(c & 15) * 8]) = rv[u];
    }
  };

  floatx16 o[4] = {};  // O^T blocks: d = 32*db + 8*(r/4) + 4*hi + r%4, query lq
  float m_run = kNegBig;
  float l_run = 0.0f;

  // transpose-read coordinates: lane's 4 keys start at row 4*hi + (lane&15)/4
  // (+8 for the second half), its 4 d values at column 16*((lane>>4)&1) + 4*(lane&3)
  const int tr_row = 4 * hi + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  const int n_tiles = (T + kKB - 1) / kKB;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < n_tiles; ++kt) {
    const int k0 = kt * kKB;
    const int cur = kt & 1;
    const bool more = kt + 1 < n_tiles;
    if (more) load_tile(k0 + kKB);

    // S^T for two 32-key blocks (raw scores).
    const uint16_t* kb_base = &Ks[cur][lq][8 * hi];
    floatx16 s0 = {}, s1 = {};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bf16x8 ka = *reinterpret_cast<const bf16x8*>(kb_base + 16 * s);
      const bf16x8 kb = *reinterpret_cast<const bf16x8*>(kb_base + 32 * kKP + 16 * s);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kb, qf[s], s1, 0, 0, 0);
    }
    // Keys past T (last tile only) get a huge negative raw score.
    if (k0 + kKB > T) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 8 * (r >> 2) + 4 * hi + (r & 3);
        if (k0 + kr >= T) s0[r] = kNegBig;
        if (k0 + 32 + kr >= T) s1[r] = kNegBig;
      }
    }
    // Tile max on raw scores (scale > 0 commutes with max), then the log2
    // domain: p = 2^(s * scale_log2 - m) with one FMA per score.
    float mt = kNegBig;
#pragma unroll
    for (int r = 0; r < 16; ++r) mt = fmaxf(mt, fmaxf(s0[r], s1[r]));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt * scale_log2);
    float lt = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], scale_log2, -m_new));
      s1[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], scale_log2, -m_new));
      lt += s0[r] + s1[r];
    }
    lt += __shfl_xor(lt, 32, 64);
    // Rescale the running sum and O only when some query's maximum grew
    // (alpha = 1 exactly for the others); after the first tiles this is rare.
    if (__builtin_amdgcn_read_exec() & __ballot(m_new > m_run)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      }
    }
    l_run += lt;
    m_run = m_new;
    // P^T operands: chunk c covers keys 16c..16c+15 of the tile in the
    // accumulator's order: lane half hi holds keys 16c + 4*hi + 0..3 (regs
    // 8*(c%2)+0..3 of block c/2) and 16c + 8 + 4*hi + 0..3 (regs +4..7).
    // Hardware round-to-nearest-even fp32 -> bf16 pairs.
    bf16x8 pc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const floatx16& sb = (c < 2) ? s0 : s1;
      const int base = 8 * (c & 1);
      pc[c] = bf16x8{(__bf16)sb[base + 0], (__bf16)sb[base + 1], (__bf16)sb[base + 2], (__bf16)sb[base + 3],
                     (__bf16)sb[base + 4], (__bf16)sb[base + 5], (__bf16)sb[base + 6], (__bf16)sb[base + 7]};
    }
    // O^T += V^T P^T.  The V^T operand for chunk c needs, for d = 32*db + lq,
    // the same 8 keys in the same order: two transpose reads of 4 keys each.
    const uint16_t* vb_base = &Vs[cur][tr_row][tr_col];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb_base + (16 * c) * kVP + 32 * db));
        const s16x4 hv =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb_base + (16 * c + 8) * kVP + 32 * db));
        const bf16x8 vt = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hv, 0, 1, 2, 3, 4, 5, 6, 7));
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vt, pc[c], o[db], 0, 0, 0);
      }
    }
    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Normalise and stage the wave's [32 q][128 d] output through LDS (K buffer 0
  // is free after the final barrier: 4 waves x 32 rows x 136 fit in 2 x 64 x 136).
  uint16_t* stage = &Ks[0][0][0] + wave * (kQW * kKP);
  const float inv_l = 1.0f / l_run;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * db + 8 * (r >> 2) + 4 * hi + (r & 3);
      stage[lq * kKP + d] = __builtin_bit_cast(uint16_t, (__bf16)(o[db][r] * inv_l));
    }
  }
  __syncthreads();
  // 32 rows x 128 d = 512 16-byte chunks per wave, 8 per lane.
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int c = lane + 64 * u;
    const int row = c >> 4;
    const int dc = (c & 15) * 8;
    const int q = q0 + row;
    if (q < T)
      *reinterpret_cast<u32x4*>(O + (size_t)q * ldo + head * kD + dc) =
          *reinterpret_cast<const u32x4*>(&stage[row * kKP + dc]);
  }
}

// ---------------------------------------------------------------------------
// Default kernel: the same work mapping, operand layouts and arithmetic as
// flash_attn_bf16_kernel, with the per-tile VALU work cut down -- this kernel
// is bound by VALU issue (its MFMAs are 32 per tile per wave, its softmax
// about as many cycles), and the register-staged tile loads spent a third of
// that VALU work on 64-bit address arithmetic:
//   * K and V tiles go HBM -> LDS by buffer_load ... lds (16 bytes per lane,
//     offsets precomputed once) into unpadded 256-byte rows, two stages each
//     (64 KiB, two workgroups per CU): no global-load addresses, no staging
//     registers, no LDS stores.  K row r keeps 16-byte chunk c at slot
//     c ^ (r & 15), so each 16-lane group of the S^T operand reads (16 rows,
//     one chunk) hits 16 distinct bank groups; V row r keeps chunk c at
//     c ^ 4(r & 3), so the transpose reads (4 rows x 16 d per 16-lane group,
//     two groups side by side) are conflict-free over 32 lanes;
//   * the tile maximum is a chain of three-input maxima;
//   * the running sum adds the bf16 P values themselves, two per
//     v_dot2_f32_bf16 against (1, 1): the normaliser is the sum of exactly the
//     weights the P V MFMAs use, and half the additions;
//   * the running sum stays a per-lane partial; its two lane halves are added
//     once at the end.
// The transfers are inline assembly (M0 = the wave's 1 KiB LDS destination,
// M0 declared clobbered) and the waits before each barrier too: the compiler
// would otherwise wait for every transfer before the next LDS read (it cannot
// tell the stages apart), or drop a builtin wait it considers satisfied.
constexpr int kTileB = kKB * kD * 2;  // one K or V tile, 16 KiB
constexpr int kDmaLds = 4 * kTileB;   // K and V, two stages each
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
struct Bf16Pairs {
  bf16x2 v[4];
};

// kQNormRope: the DiT block's per-head RMSNorm (weights qn, eps) and RoPE
// (table rope [T][64] of (cos, sin)) are applied to the raw Q rows here, as
// k_norm_rope_kernel (dit_block.hip) applies them to K, with the same
// arithmetic: per 8-channel chunk the sum of squares of its four (even, odd)
// pairs, the 16 chunk sums of the head added pairwise over chunk index bits
// 3, 2, 1, 0 (bits 3..1 are this lane's own chunks s ^ 4, s ^ 2, s ^ 1; bit 0
// is the other lane half), then the scaled, rotated pairs rounded to bf16.
template <bool kQNormRope>
__global__ __launch_bounds__(256, 2) void flash_attn_bf16_dma_kernel(const uint16_t* __restrict__ Q,
                                                                     const uint16_t* __restrict__ K,
                                                                     const uint16_t* __restrict__ V,
                                                                     uint16_t* __restrict__ O, int T, int ldq,
                                                                     int ldk, int ldv, int ldo, float scale_log2,
                                                                     const float2* __restrict__ rope,
                                                                     const float* __restrict__ qn,
                                                                     const float* __restrict__ kn, float eps,
                                                                     int o_slice) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int head, qb;
  block_coords(T, &head, &qb);
  const int q0 = qb * (4 * kQW) + wave * kQW;
  const int lq = lane & 31;
  const int hi = lane >> 5;
  const int qi = q0 + lq;
  const int n_tiles = (T + kKB - 1) / kKB;

  // HBM -> LDS transfers; the buffer range ends with the head's last row
  // (row T-1, 128 columns), so the rows of the last tile past T read zero.
  // The entry point bounds T * ld * 2 below 2^31 and ld below 2^24, so the
  // byte offsets below (at most 63 rows of a tile past row T - 1) fit 32 bits.
  typedef int int4v __attribute__((ext_vector_type(4)));
  auto desc = [](const void* ptr, uint32_t bytes) {
    const unsigned long long a = (unsigned long long)ptr;
    int4v d;
    d.x = __builtin_amdgcn_readfirstlane((int)(a & 0xffffffffu));
    d.y = __builtin_amdgcn_readfirstlane((int)(a >> 32));
    d.z = __builtin_amdgcn_readfirstlane((int)bytes);
    d.w = 0x00020000;
    return d;
  };
  const int4v rs_k = desc(K + head * kD, (uint32_t)(((size_t)(T - 1) * ldk + kD) * 2));
  const int4v rs_v = desc(V + head * kD, (uint32_t)(((size_t)(T - 1) * ldv + kD) * 2));
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // 1 KiB block 4*wave + i of a tile: rows 16*wave + 4i .. +3, lane -> (row, slot)
    const uint32_t row = (uint32_t)(16 * wave + 4 * i + (lane >> 4));
    const uint32_t slot = (uint32_t)(lane & 15);
    koff[i] = (row * (uint32_t)ldk + 8u * (slot ^ (row & 15u))) * 2u;
    voff[i] = (row * (uint32_t)ldv + 8u * (slot ^ (4u * (row & 3u)))) * 2u;
  }
  // Transfer x (0..7) of this wave for tile j: K block x (x < 4) or V block
  // x - 4, 1 KiB each.
  auto issue_one = [&](int j, int x) __attribute__((always_inline)) {
    const bool kx = x < 4;
    const int i = x & 3;
    char* st = lds + (kx ? 0 : 2 * kTileB) + (j & 1) * kTileB;
    const uint32_t add = (uint32_t)j * (uint32_t)(kKB * 2) * (uint32_t)(kx ? ldk : ldv);
    const uint32_t base = (uint32_t)(size_t)(__attribute__((address_space(3))) char*)st;
    const uint32_t la = __builtin_amdgcn_readfirstlane(base + (4 * wave + i) * 1024);
    if (kx)
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(la), "v"(koff[i] + add),
                   "s"(rs_k)
                   : "memory", "m0");
    else
      asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(la), "v"(voff[i] + add),
                   "s"(rs_v)
                   : "memory", "m0");
  };
  auto issue_tile = [&](int j) {
#pragma unroll
    for (int x = 0; x < 8; ++x) issue_one(j, x);
  };

  bf16x8 qf[8];
  {
    const uint16_t* qrow = Q + (size_t)qi * ldq + head * kD;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (qi < T) v = *reinterpret_cast<const u32x4*>(qrow + 16 * s + 8 * hi);
      qf[s] = __builtin_bit_cast(bf16x8, v);
    }
  }
  // Q's RoPE entries (chunk c = 2 s + hi holds channels 8 c .. 8 c + 7 of the
  // head: 32 contiguous bytes of the 256-byte-aligned table) are loaded here
  // and used after tile 0's transfers are issued.
  floatx4 qtab[kQNormRope ? 8 : 1][2];
  if constexpr (kQNormRope) {
    const floatx4* trow = reinterpret_cast<const floatx4*>(rope + (size_t)min(qi, T - 1) * 64);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int c = 2 * s + hi;
      qtab[s][0] = trow[2 * c];
      qtab[s][1] = trow[2 * c + 1];
    }
  }

  // Score bound of the per-head-normalised queries and keys: |q| <= sqrt(128)
  // max|q_norm|, |k| <= sqrt(128) max|k_norm| (RMSNorm output has RMS <= 1,
  // RoPE keeps the norm, bf16 rounding grows it by at most 2^-9), so every
  // score in log2 units is at most 128 max|q_norm| max|k_norm| scale_log2 in
  // magnitude.  When that is <= kDirectLog2 the softmax needs no running
  // maximum: p = 2^s directly, and O / sum(p) is the same softmax
  // (mathematically identical to subtracting the maximum; the probabilities
  // are rounded to bf16 with the same relative error).  The scale goes into
  // Q as it is normalised, so a score needs one v_exp_f32 and nothing else.
  bool direct = false;
  if constexpr (kQNormRope) {
    float wq = fmaxf(fabsf(qn[lane]), fabsf(qn[lane + 64]));
    float wk = fmaxf(fabsf(kn[lane]), fabsf(kn[lane + 64]));
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
      wq = fmaxf(wq, __shfl_xor(wq, sh));
      wk = fmaxf(wk, __shfl_xor(wk, sh));
    }
    const float bound = 128.0f * wq * wk * scale_log2 * 1.01f;
    direct = __builtin_amdgcn_readfirstlane((int)(bound <= kDirectLog2)) != 0;
  }

  // operand addresses within a stage (bytes)
  const int k_lane = lq * 256;
  const int k_swz = lq & 15;
  const int tr_row = 4 * hi + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int v_swz = 4 * (tr_row & 3);
  const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};

  floatx16 o[4] = {};
  float m_run = kNegBig;
  float l_part = 0.0f;  // this lane half's share of the running sum

  // One tile; kStage (0 or 1) is a compile-time constant so that the stage
  // offsets fold into the LDS instructions' offset fields.
  auto tile = [&](int t, auto stage_c, auto direct_c) {
    constexpr int kStage = decltype(stage_c)::value;
    constexpr bool kDirect = decltype(direct_c)::value;
    const int k0 = t * kKB;
    // tile t has landed (this wave's transfers; the barrier covers the
    // others'), and every wave is past tile t-1, whose stages take tile t+1
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const bool more = t + 1 < n_tiles;
    const char* kst = lds + kStage * kTileB;
    const char* vst = lds + (2 + kStage) * kTileB;

    // S^T for two 32-key blocks (raw scores).  Each pair of MFMAs is followed
    // by one of the wave's 8 transfers of tile t+1 (issued together after the
    // barrier, a workgroup's 32 transfers queue at the texture unit and hold
    // back the MFMAs of the waves that issue them last).
    // The K operands are read one step ahead: the transfers' asm statements
    // (memory clobbers) keep the compiler from hoisting the reads itself.
    floatx16 s0 = {}, s1 = {};
    auto k_pair = [&](int s, bf16x8& ka, bf16x8& kb) __attribute__((always_inline)) {
      const int off = ((2 * s + hi) ^ k_swz) << 4;
      ka = *reinterpret_cast<const bf16x8*>(kst + k_lane + off);
      kb = *reinterpret_cast<const bf16x8*>(kst + k_lane + 32 * 256 + off);
    };
    bf16x8 ka, kb;
    k_pair(0, ka, kb);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      bf16x8 na = ka, nb = kb;
      if (s + 1 < 8) k_pair(s + 1, na, nb);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kb, qf[s], s1, 0, 0, 0);
      if (more) issue_one(t + 1, s);
      ka = na;
      kb = nb;
    }
    if (k0 + kKB > T) {  // the last, partial tile: keys past T get a huge negative score
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 8 * (r >> 2) + 4 * hi + (r & 3);
        if (k0 + kr >= T) s0[r] = kNegBig;
        if (k0 + 32 + kr >= T) s1[r] = kNegBig;
      }
    }
    if constexpr (kDirect) {
      // scores are already in log2 units (the scale is inside Q) and bounded
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s0[r] = __builtin_amdgcn_exp2f(s0[r]);
        s1[r] = __builtin_amdgcn_exp2f(s1[r]);
      }
    } else {
      float mt = fmaxf(s0[0], s1[0]);
#pragma unroll
      for (int r = 1; r < 16; ++r) asm("v_max3_f32 %0, %1, %2, %3" : "=v"(mt) : "v"(mt), "v"(s0[r]), "v"(s1[r]));
      mt = max_halves(mt);
      // Lazy rescaling: the reference maximum m_run moves only when the tile's
      // maximum exceeds it by more than kLazyLog2, so p <= 2^kLazyLog2 and O and
      // the running sum are rescaled in a handful of tiles, not in most.
      const float m_cand = fmaxf(m_run, mt * scale_log2);
      const bool grow = m_cand > m_run + kLazyLog2;
      if (__builtin_amdgcn_read_exec() & __ballot(grow)) {
        const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_cand) : 1.0f;
        l_part *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      }
      if (grow) m_run = m_cand;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s0[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], scale_log2, -m_run));
        s1[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], scale_log2, -m_run));
      }
    }
    // P^T operands (keys of chunk c in the accumulator's order, see
    // flash_attn_bf16_kernel), and their sum two at a time
    bf16x8 pc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const floatx16& sb = (c < 2) ? s0 : s1;
      const int base = 8 * (c & 1);
      pc[c] = bf16x8{(__bf16)sb[base + 0], (__bf16)sb[base + 1], (__bf16)sb[base + 2], (__bf16)sb[base + 3],
                     (__bf16)sb[base + 4], (__bf16)sb[base + 5], (__bf16)sb[base + 6], (__bf16)sb[base + 7]};
      const Bf16Pairs pairs = __builtin_bit_cast(Bf16Pairs, pc[c]);
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) l_part = __builtin_amdgcn_fdot2_f32_bf16(pairs.v[pr], ones, l_part, false);
    }
    // O^T += V^T P^T
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int col = tr_col + 32 * db;
        const int coff = (((col >> 3) ^ v_swz) << 4) + ((col & 7) << 1);
        const char* r0 = vst + (16 * c + tr_row) * 256 + coff;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)r0);
        const s16x4 hv = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(r0 + 8 * 256));
        const bf16x8 vt = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hv, 0, 1, 2, 3, 4, 5, 6, 7));
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vt, pc[c], o[db], 0, 0, 0);
      }
    }
  };
  issue_tile(0);
  if constexpr (kQNormRope) {
    float chunk_ss[8];  // sum of squares of chunk 2 s + hi
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const u32x4 w = __builtin_bit_cast(u32x4, qf[s]);
      float ss = 0.0f;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float e = __uint_as_float(w[p] << 16), o = __uint_as_float(w[p] & 0xffff0000u);
        ss += e * e + o * o;
      }
      chunk_ss[s] = ss;
    }
    float x[8], y[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) x[s] = chunk_ss[s] + chunk_ss[s ^ 4];
#pragma unroll
    for (int s = 0; s < 8; ++s) y[s] = x[s] + x[s ^ 2];
    const float z = y[0] + y[1];
    const float inv = 1.0f / sqrtf(sum_halves(z) / 128.0f + eps) * (direct ? scale_log2 : 1.0f);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const u32x4 w = __builtin_bit_cast(u32x4, qf[s]);
      // weights of chunks 2 s and 2 s + 1: the same addresses in every lane,
      // held in scalar registers (scalar loads), then the lane half's chunk
      float wv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float we = qn[16 * s + i], wo = qn[16 * s + 8 + i];
        asm("" : "+s"(we), "+s"(wo));
        wv[i] = hi ? wo : we;
      }
      const float tv[8] = {qtab[s][0].x, qtab[s][0].y, qtab[s][0].z, qtab[s][0].w,
                           qtab[s][1].x, qtab[s][1].y, qtab[s][1].z, qtab[s][1].w};
      u32x4 r;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float e = __uint_as_float(w[p] << 16), o = __uint_as_float(w[p] & 0xffff0000u);
        const float cs_p = tv[2 * p], sn_p = tv[2 * p + 1];
        const float ne = e * inv * wv[2 * p], no = o * inv * wv[2 * p + 1];
        r[p] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(ne * cs_p - no * sn_p)) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(ne * sn_p + no * cs_p)) << 16);
      }
      qf[s] = __builtin_bit_cast(bf16x8, r);
    }
  }
  const std::integral_constant<int, 0> st0{};
  const std::integral_constant<int, 1> st1{};
  // (Peeling the last two tiles out of the loop, so that the steady tiles
  // carry no branches around their transfers, measured 6 us slower in the C5
  // block.)
  const std::integral_constant<bool, false> with_max{};
  int t = 0;
  if (kQNormRope && direct) {
    const std::integral_constant<bool, kQNormRope> no_max{};  // the direct path exists only with the norms
    for (; t + 1 < n_tiles; t += 2) {
      tile(t, st0, no_max);
      tile(t + 1, st1, no_max);
    }
    if (t < n_tiles) tile(t, st0, no_max);
  } else {
    for (; t + 1 < n_tiles; t += 2) {
      tile(t, st0, with_max);
      tile(t + 1, st1, with_max);
    }
    if (t < n_tiles) tile(t, st0, with_max);
  }

  // Normalise and stage the wave's [32 q][128 d] output through LDS (34 KiB
  // from offset 0); the barrier ends every wave's reads of the stages.
  __syncthreads();
  const float l_run = sum_halves(l_part);
  uint16_t* stage = reinterpret_cast<uint16_t*>(lds) + wave * (kQW * kKP);
  const float inv_l = 1.0f / l_run;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * db + 8 * (r >> 2) + 4 * hi + (r & 3);
      stage[lq * kKP + d] = __builtin_bit_cast(uint16_t, (__bf16)(o[db][r] * inv_l));
    }
  }
  __syncthreads();
  if (o_slice > 0) {
    // K-blocked O ([D/32][o_slice][32], for the output GEMM): each store
    // instruction writes 16 rows of one 32-column slice, 1 KiB contiguous
    // (lanes 16j .. 16j + 15: chunk j of 16 rows, so each 16-lane LDS read
    // touches 16 distinct bank groups).
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int row = (lane & 15) + 16 * (u & 1), blk = u >> 1, chunk = lane >> 4;
      const int q = q0 + row;
      if (q < T)
        *reinterpret_cast<u32x4*>(O + ((size_t)(head * 4 + blk) * o_slice + q) * 32 + 8 * chunk) =
            *reinterpret_cast<const u32x4*>(&stage[row * kKP + 32 * blk + 8 * chunk]);
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int c = lane + 64 * u;
    const int row = c >> 4;
    const int dc = (c & 15) * 8;
    const int q = q0 + row;
    if (q < T)
      *reinterpret_cast<u32x4*>(O + (size_t)q * ldo + head * kD + dc) =
          *reinterpret_cast<const u32x4*>(&stage[row * kKP + dc]);
  }
}

}  // namespace

// Q/K/V/O bf16 [T, ld*] with `heads` heads of 128 columns each.  variant 0
// is the DMA-fed kernel, 1 the register-staged one (kept as a cross-check).
hipError_t launch_flash_attn_bf16(const uint16_t* q, int ldq, const uint16_t* k, int ldk, const uint16_t* v, int ldv,
                                  uint16_t* o, int ldo, int T, int heads, float scale, hipStream_t stream,
                                  int variant) {
  const dim3 grid((unsigned)((T + 4 * kQW - 1) / (4 * kQW) * heads));
  const float scale_log2 = scale * 1.4426950408889634f;
  if (variant == 1) {
    hipLaunchKernelGGL(flash_attn_bf16_kernel, grid, dim3(256), 0, stream, q, k, v, o, T, ldq, ldk, ldv, ldo,
                       scale_log2);
    return hipGetLastError();
  }
  if (variant != 0) return hipErrorInvalidValue;
  static bool lds_raised = false;
  if (!lds_raised) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(flash_attn_bf16_dma_kernel<false>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, kDmaLds);
    if (e != hipSuccess) return e;
    lds_raised = true;
  }
  hipLaunchKernelGGL(flash_attn_bf16_dma_kernel<false>, grid, dim3(256), kDmaLds, stream, q, k, v, o, T, ldq, ldk,
                     ldv, ldo, scale_log2, nullptr, nullptr, nullptr, 0.0f, 0);
  return hipGetLastError();
}

// The DiT block's attention: the DMA-fed kernel with the per-head RMSNorm
// (qn, eps) and RoPE (rope, [T][64]) applied to the raw Q rows on load; K
// holds rows normalised with kn, whose largest weight bounds the scores.
hipError_t launch_flash_attn_bf16_qnorm_rope(const uint16_t* q, int ldq, const uint16_t* k, int ldk, const uint16_t* v,
                                            int ldv, uint16_t* o, int ldo, int T, int heads, float scale,
                                            const float2* rope, const float* qn, const float* kn, float eps,
                                            hipStream_t stream, int o_slice) {
  const dim3 grid((unsigned)((T + 4 * kQW - 1) / (4 * kQW) * heads));
  static bool lds_raised = false;
  if (!lds_raised) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(flash_attn_bf16_dma_kernel<true>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, kDmaLds);
    if (e != hipSuccess) return e;
    lds_raised = true;
  }
  hipLaunchKernelGGL(flash_attn_bf16_dma_kernel<true>, grid, dim3(256), kDmaLds, stream, q, k, v, o, T, ldq, ldk, ldv,
                     ldo, scale * 1.4426950408889634f, rope, qn, kn, eps, o_slice);
  return hipGetLastError();
}

}  // namespace prom
