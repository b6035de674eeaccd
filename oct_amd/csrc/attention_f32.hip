// FP32 flash attention on CDNA4 MFMA (v_mfma_f32_32x32x2_f32) for the fp32
// transformer blocks: the Gemma-shaped decoder layer (causal, every query
// head on one K/V head, head_dim 256) and the resident Z-Image blocks (30
// heads of 128, full attention).  The reference's streaming attention keeps a
// score row in workgroup memory and never writes scores to global memory
// (shaders/sdslv/production/zimage/main_transformer_joint_attention_streaming.sdslv:20-86);
// this kernel does the same with tiles of keys and an online softmax, so no
// [heads, T, T] score tensor exists.
//
//   * a wave owns 32 queries of one query head; a workgroup's waves share one
//     K/V head and one key range: either several query heads over the same 32
//     queries (multi-query attention: the K/V tile serves every head), or
//     consecutive 32-query blocks of one head;
//   * per 32-key tile, K^T [d][32] and V [32][d] go from HBM straight to LDS
//     (buffer_load ... lds, 16 bytes per lane, no register staging) into two
//     stages: the next tile streams in during the current tile's MFMAs; rows
//     are placed so the two lane halves of every operand read fall on
//     opposite halves of the banks;
//   * S^T = K Q^T: a lane owns one query and 16 of the tile's 32 keys, so the
//     row max and sum need one exchange between lanes l and l^32.  Q stays in
//     registers for the whole kernel, its head dimension consumed in the
//     order (8p + 4h + j) so each lane loads it with 128-bit reads;
//   * O^T = V^T P^T accumulates in d/32 MFMA blocks: the B operand of MFMA step
//     r is exactly accumulator register r of S^T (keys 8(r/4) + 4h + r%4), so
//     P never leaves the registers, and V^T's operand is a plain row read;
//   * softmax in the log2 domain (one FMA and one v_exp_f32 per score), O and
//     the running sum rescaled only when some query's maximum grew;
//   * causal: tiles entirely above a workgroup's last query are never
//     visited; masking only on the diagonal and partial tiles;
//   * when the grid would leave most of the chip idle (the causal layer at
//     T = 512 has 16 query blocks), the key range is split over the grid's z
//     dimension: each split writes its unnormalised O, running max and sum, and
//     a combine kernel merges the splits in a fixed order (deterministic).
//
// Head dim 256 with query heads sharing a K/V head in eights (the Gemma-shaped
// layer's multi-query attention) has a kernel of its own: 16-query waves on
// v_mfma_f32_16x16x4_f32 halve the Q and O^T registers (64 + 64), so a
// workgroup of eight waves, one per query head, runs two waves per SIMD and
// one wave's softmax overlaps the other's MFMAs; 16-key tiles keep two LDS
// stages at 64 KB and let the key range be split finely enough that the
// causal triangle's work spreads over the whole chip.
#include <math.h>

#include <algorithm>

#include "reactor_internal.h"

namespace prom {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kQW = 32;  // queries per wave
constexpr int kKB = 32;  // keys per tile

// One LDS stage: K^T [d rows][32 keys] then V [32 keys][d], unpadded.  The two
// lane halves of an MFMA operand read rows 4 apart (c and c + 4 of K^T, keys k
// and k + 4 of V); so that they fall on opposite halves of the banks, K^T row c
// sits in row slot c ^ ((c >> 2) & 1) and V row k has its 128-byte halves
// exchanged when (k >> 2) & 1 (column c stored at c ^ 32).  Both are applied
// by choosing each lane's source in the HBM -> LDS transfers.
template <int kD>
struct AttnTile {
  static constexpr int kKtBytes = kD * kKB * 4;
  static constexpr int kStage = 2 * kKtBytes;  // K^T and V are the same size
};

// Work mapping of one launch (decided on the host by plan_attention).
struct AttnLaunch {
  AttnF32Params p;
  int wh;            // query heads per workgroup: wave w serves head y*wh + w % wh
  int wq;            // 32-query blocks per workgroup: wave w serves block x*wq + w / wh
  int chunk;         // key tiles per split
  int splits;        // gridDim.z
  int qspan;         // queries per workgroup (one key range)
  int tkeys;         // keys per tile
  float scale_log2;  // score scale times log2(e)
};

// Key tiles of tkeys keys that the queries qbase .. qbase + qspan - 1 visit.
__device__ __host__ inline int key_tiles(const AttnF32Params& p, int qbase, int qspan, int tkeys) {
  const int kend = p.causal ? min(p.T, qbase + qspan) : p.T;
  return (kend + tkeys - 1) / tkeys;
}

template <int kD, int kW>
__device__ __forceinline__ void flash_attn_f32_body(const AttnLaunch& a, char* S0, char* S1) {
  using Cfg = AttnTile<kD>;
  constexpr int kXfer = Cfg::kKtBytes / 1024 / kW;  // 1 KB transfers per wave for each of K^T and V
  static_assert(kXfer * 1024 * kW == Cfg::kKtBytes, "tile does not divide over the workgroup");
  typedef __attribute__((address_space(3))) void lds_void;

  const AttnF32Params& p = a.p;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31;
  const int hi = lane >> 5;
  const int hq = (int)blockIdx.y * a.wh + wave % a.wh;
  const int hkv = ((int)blockIdx.y * a.wh) / p.group;
  const int qbase = (int)blockIdx.x * a.wq * kQW;
  const int q0 = qbase + (wave / a.wh) * kQW;
  const int qi = q0 + lq;

  const int t_begin = (int)blockIdx.z * a.chunk;
  const int t_end = min(key_tiles(p, qbase, a.wq * kQW, kKB), t_begin + a.chunk);
  if (t_begin >= t_end) return;  // the whole workgroup: this split has no keys for it

  // Q operand (B of S^T = K Q^T): qr[4p + j] = Q[qi][8p + 4*hi + j].
  float qr[kD / 2];
  {
    const float* qrow = p.q + (size_t)hq * p.q_hs + (size_t)qi * p.q_rs;
#pragma unroll
    for (int pp = 0; pp < kD / 8; ++pp) {
      floatx4 v = {0.f, 0.f, 0.f, 0.f};
      if (qi < p.T) v = *reinterpret_cast<const floatx4*>(qrow + 8 * pp + 4 * hi);
      qr[4 * pp + 0] = v.x;
      qr[4 * pp + 1] = v.y;
      qr[4 * pp + 2] = v.z;
      qr[4 * pp + 3] = v.w;
    }
  }

  // HBM -> LDS transfers, 16 bytes per lane.  The buffer ranges end at the
  // head's K^T / V extent, so reads past it (keys >= T of the last rows) return
  // zero; keys >= T inside the range are masked out of the softmax.
  const __amdgpu_buffer_rsrc_t rs_kt = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.kt + (size_t)hkv * p.kt_hs), (short)0, (int)((size_t)kD * p.kt_rs * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_v = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.v + (size_t)hkv * p.v_hs), (short)0, (int)((size_t)p.T * p.v_rs * 4), 0x00020000);
  uint32_t kt_off[kXfer], v_off[kXfer];
#pragma unroll
  for (int i = 0; i < kXfer; ++i) {
    const int blk = kXfer * wave + i;  // 1 KB block of the stage
    // K^T: slots 8*blk .. 8*blk+7, lane -> slot 8*blk + lane/8, keys 4*(lane%8) ..
    const int slot = 8 * blk + (lane >> 3);
    const int c = slot ^ ((slot >> 2) & 1);
    kt_off[i] = (uint32_t)((c * p.kt_rs + 4 * (lane & 7)) * 4);
    // V: rows of kD floats; lane -> row, 16-byte position pos, source chunk pos ^ 8*((row >> 2) & 1)
    const int e = 1024 / 16 * blk + lane;  // 16-byte chunk index within the V tile
    const int row = e / (kD / 4);
    const int pos = e % (kD / 4);
    v_off[i] = (uint32_t)((row * p.v_rs + 4 * (pos ^ (8 * ((row >> 2) & 1)))) * 4);
  }
  // The key offset of V rows goes into the vector offset, which the buffer's
  // range check covers, so rows past T read as zero (the scalar offset is not
  // range-checked).
  auto issue = [&](char* stage, int k0) {
    const int skt = __builtin_amdgcn_readfirstlane(k0 * 4);
    const uint32_t vk = (uint32_t)(k0 * p.v_rs * 4);
#pragma unroll
    for (int i = 0; i < kXfer; ++i) {
      const int blk = kXfer * wave + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_kt, (lds_void*)(stage + blk * 1024), 16, kt_off[i], skt, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_v, (lds_void*)(stage + Cfg::kKtBytes + blk * 1024), 16,
                                               v_off[i] + vk, 0, 0, 0);
    }
  };

  floatx16 o[kD / 32];  // O^T block cb: d = 32cb + 8(r/4) + 4hi + r%4, query qi
#pragma unroll
  for (int cb = 0; cb < kD / 32; ++cb) o[cb] = floatx16{};
  float m_run = -INFINITY;  // running max of the scaled scores, log2 domain
  float l_run = 0.0f;

  // Operand addresses within a stage (floats).  K^T row c = 8p + 4hi + j sits
  // in slot c ^ hi; V row k = 8(r/4) + 4hi + r%4 holds column c at c ^ 32hi.
  const int kt_lane = 4 * hi * kKB + lq;
  const int v_lane = 4 * hi * kD + lq;

  auto compute = [&](const char* stage, int k0) {
    const float* kts = reinterpret_cast<const float*>(stage);
    const float* vs = reinterpret_cast<const float*>(stage + Cfg::kKtBytes);
    // S^T (raw scores) in two independent accumulation chains.
    floatx16 sa = {}, sb = {};
#pragma unroll
    for (int pp = 0; pp < kD / 8; pp += 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sa = __builtin_amdgcn_mfma_f32_32x32x2f32(kts[kt_lane + (8 * pp + (j ^ hi)) * kKB], qr[4 * pp + j], sa, 0,
                                                  0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sb = __builtin_amdgcn_mfma_f32_32x32x2f32(kts[kt_lane + (8 * pp + 8 + (j ^ hi)) * kKB], qr[4 * pp + 4 + j],
                                                  sb, 0, 0, 0);
      if ((pp & 7) == 6) __builtin_amdgcn_sched_barrier(0);  // bound the operand reads in flight
    }
    floatx16 s = sa + sb;
    // Keys past T, and (causal) keys after the query, are excluded.
    if (k0 + kKB > p.T || (p.causal && k0 + kKB - 1 > q0)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 8 * (r >> 2) + 4 * hi + (r & 3);
        if (key >= p.T || (p.causal && key > qi)) s[r] = -INFINITY;
      }
    }
    float mt = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
    mt = max_halves(mt);
    const float m_new = fmaxf(m_run, mt * a.scale_log2);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;  // a query with no visible key yet
    float lt = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], a.scale_log2, -m_use));
      lt += s[r];
    }
    lt = sum_halves(lt);
    if (__builtin_amdgcn_read_exec() & __ballot(m_new > m_run)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      l_run *= alpha;
#pragma unroll
      for (int cb = 0; cb < kD / 32; ++cb)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[cb][r] *= alpha;
    }
    l_run += lt;
    m_run = m_new;
    // O^T += V^T P^T: step r pairs keys 8(r/4) + r%4 (lanes 0-31) and +4 (lanes 32-63).
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = 8 * (r >> 2) + (r & 3);
#pragma unroll
      for (int cb = 0; cb < kD / 32; ++cb)
        o[cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(vs[v_lane + kr * kD + ((32 * cb) ^ (32 * hi))], s[r], o[cb], 0,
                                                     0, 0);
      if ((r & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
  };

  issue(S0, t_begin * kKB);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // Unrolled by two so that the reads of one stage are visibly independent of
  // the transfers into the other.
  int t = t_begin;
  for (; t + 1 < t_end; t += 2) {
    issue(S1, (t + 1) * kKB);
    compute(S0, t * kKB);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 2 < t_end) issue(S0, (t + 2) * kKB);
    compute(S1, (t + 1) * kKB);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (t < t_end) compute(S0, t * kKB);  // odd count: the last tile was issued into S0

  if (qi >= p.T) return;
  if (a.splits == 1) {
    const float inv_l = 1.0f / l_run;
    float* orow = p.o + (size_t)qi * p.o_rs + (size_t)hq * kD;
#pragma unroll
    for (int cb = 0; cb < kD / 32; ++cb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const floatx4 v = {o[cb][4 * g] * inv_l, o[cb][4 * g + 1] * inv_l, o[cb][4 * g + 2] * inv_l,
                           o[cb][4 * g + 3] * inv_l};
        *reinterpret_cast<floatx4*>(orow + 32 * cb + 8 * g + 4 * hi) = v;
      }
  } else {
    // Partial of split z: unnormalised O [z][T][Hq][d], (max, sum) [z][T][Hq].
    const size_t row = ((size_t)blockIdx.z * p.T + qi) * p.q_heads + hq;
    float* orow = p.part_o + row * kD;
#pragma unroll
    for (int cb = 0; cb < kD / 32; ++cb)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<floatx4*>(orow + 32 * cb + 8 * g + 4 * hi) =
            floatx4{o[cb][4 * g], o[cb][4 * g + 1], o[cb][4 * g + 2], o[cb][4 * g + 3]};
    if (hi == 0) {
      p.part_ml[2 * row] = m_run;
      p.part_ml[2 * row + 1] = l_run;
    }
  }
}

// Two LDS stages each; the kernels differ in head dim and waves per workgroup.
__global__ __launch_bounds__(128, 1) void flash_attn_f32_d64_kernel(const AttnLaunch a) {
  __shared__ __attribute__((aligned(1024))) char S0[AttnTile<64>::kStage];
  __shared__ __attribute__((aligned(1024))) char S1[AttnTile<64>::kStage];
  flash_attn_f32_body<64, 2>(a, S0, S1);
}

__global__ __launch_bounds__(128, 1) void flash_attn_f32_d128_kernel(const AttnLaunch a) {
  __shared__ __attribute__((aligned(1024))) char S0[AttnTile<128>::kStage];
  __shared__ __attribute__((aligned(1024))) char S1[AttnTile<128>::kStage];
  flash_attn_f32_body<128, 2>(a, S0, S1);
}

__global__ __launch_bounds__(256, 1) void flash_attn_f32_d256_kernel(const AttnLaunch a) {
  __shared__ __attribute__((aligned(1024))) char S0[AttnTile<256>::kStage];
  __shared__ __attribute__((aligned(1024))) char S1[AttnTile<256>::kStage];
  flash_attn_f32_body<256, 4>(a, S0, S1);
}

// ---- head dim 256, query heads sharing a K/V head in eights ----------------
// Workgroup (x, y): work item x (a block of 16 queries and a split of its key
// tiles) of query heads 8y .. 8y + 7 (wave w: head 8y + w).  MFMA 16x16x4 f32
// operand layout: A[i][k] from lane i + 16k, B[k][j] from lane j + 16k, D[i][j]
// in lane j + 16(i/4), register i%4.  A lane's group g = lane / 16 and query
// lq = lane % 16:
//   * S^T = K Q^T: step 4pp + j takes head-dim index 16pp + 4g + j from lane
//     group g (the A operand is K^T row 16pp + 4g + j at key lq, the B operand
//     Q[q0 + lq][same index]); the accumulator holds keys 4g + r of query lq;
//   * O^T = V^T P^T: step r pairs key 4g + r with lane group g, so its B
//     operand is accumulator register r of S^T and its A operand is V row
//     4g + r at head-dim 16cb + lq; O^T block cb holds head-dim 16cb + 4g + r.
// LDS stage: K^T [256 slots][16 keys] then V [16 keys][256].  Head-dim row c of
// K^T sits in slot c ^ ((c >> 2) & 3), and the 16-float chunk b of V row k at
// chunk b ^ ((k >> 2) & 3), so the four lane groups of every operand read use
// four different quarters of the banks.
constexpr int kHQ = 16;                    // queries per wave
constexpr int kHK = 16;                    // keys per tile
constexpr int kHD = 256;                   // head dim
constexpr int kHKtBytes = kHD * kHK * 4;   // K^T tile: 16 KB
constexpr int kHStage = 2 * kHKtBytes;     // K^T then V

// Maximum over lanes l, l ^ 16, l ^ 32, l ^ 48 (one query's four key groups).
__device__ __forceinline__ float max_quarters(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max_halves(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ __forceinline__ float sum_quarters(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return sum_halves(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

__global__ __launch_bounds__(512, 1) void flash_attn_f32_d256_h8_kernel(const AttnLaunch a) {
  __shared__ __attribute__((aligned(1024))) char S0[kHStage];
  __shared__ __attribute__((aligned(1024))) char S1[kHStage];
  typedef __attribute__((address_space(3))) void lds_void;

  const AttnF32Params& p = a.p;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;
  const int lq = lane & 15;
  const int hq = (int)blockIdx.y * 8 + wave;
  const int hkv = ((int)blockIdx.y * 8) / p.group;
  // Work item blockIdx.x -> (query block, split): the grid lists only splits
  // that have keys, the last (most loaded, under a causal mask) query blocks
  // first, so no workgroup is empty and the longest start first.
  int item = (int)blockIdx.x;
  int qb = (p.T + kHQ - 1) / kHQ - 1;
  for (; qb >= 0; --qb) {
    const int n = (key_tiles(p, qb * kHQ, kHQ, kHK) + a.chunk - 1) / a.chunk;
    if (item < n) break;
    item -= n;
  }
  if (qb < 0) return;  // past the list (the host sizes the grid to it)
  const int split = item;
  const int q0 = qb * kHQ;
  const int qi = q0 + lq;
  const int t_begin = split * a.chunk;
  const int t_end = min(key_tiles(p, q0, kHQ, kHK), t_begin + a.chunk);

  // Q operand: qr[4pp + j] = Q[qi][16pp + 4g + j].
  float qr[64];
  {
    const float* qrow = p.q + (size_t)hq * p.q_hs + (size_t)qi * p.q_rs + 4 * g;
#pragma unroll
    for (int pp = 0; pp < 16; ++pp) {
      floatx4 v = {0.f, 0.f, 0.f, 0.f};
      if (qi < p.T) v = *reinterpret_cast<const floatx4*>(qrow + 16 * pp);
      qr[4 * pp + 0] = v.x;
      qr[4 * pp + 1] = v.y;
      qr[4 * pp + 2] = v.z;
      qr[4 * pp + 3] = v.w;
    }
  }

  // HBM -> LDS: wave w moves K^T slots 32w .. 32w + 31 and V rows 2w, 2w + 1
  // (1 KB per instruction, 16 bytes per lane).  The K^T range is the head's
  // [256][kt_rs] block, so key columns past T read the rows' padding (masked
  // out of the softmax); V's key offset is in the range-checked vector offset,
  // so V rows past T read as zero.
  const __amdgpu_buffer_rsrc_t rs_kt = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.kt + (size_t)hkv * p.kt_hs), (short)0, (int)((size_t)kHD * p.kt_rs * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_v = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.v + (size_t)hkv * p.v_hs), (short)0, (int)((size_t)p.T * p.v_rs * 4), 0x00020000);
  uint32_t kt_off[2], v_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int blk = 2 * wave + i;
    const int slot = 16 * blk + (lane >> 2);
    const int c = slot ^ ((slot >> 2) & 3);
    kt_off[i] = (uint32_t)((c * p.kt_rs + 4 * (lane & 3)) * 4);
    v_off[i] = (uint32_t)((blk * p.v_rs + 16 * ((lane >> 2) ^ ((blk >> 2) & 3)) + 4 * (lane & 3)) * 4);
  }
  auto issue = [&](char* stage, int k0) {
    const int skt = __builtin_amdgcn_readfirstlane(k0 * 4);
    const uint32_t vk = (uint32_t)(k0 * p.v_rs * 4);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int blk = 2 * wave + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_kt, (lds_void*)(stage + blk * 1024), 16, kt_off[i], skt, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_v, (lds_void*)(stage + kHKtBytes + blk * 1024), 16,
                                               v_off[i] + vk, 0, 0, 0);
    }
  };

  floatx4 o[16];  // O^T block cb: head-dim 16cb + 4g + r, query qi
#pragma unroll
  for (int cb = 0; cb < 16; ++cb) o[cb] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // running max of the scaled scores, log2 domain
  float l_run = 0.0f;

  // Operand addresses within a stage (floats): K^T head-dim 16pp + 4g + j is in
  // slot 16pp + 4g + (j ^ g); V key 4g + r, chunk cb is at chunk cb ^ g.
  int kt_lane[4], v_lane[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    kt_lane[j] = (4 * g + (j ^ g)) * kHK + lq;
    v_lane[j] = 4 * g * kHD + ((j ^ g) << 4) + lq;
  }

  auto compute = [&](const char* stage, int k0) {
    const float* kts = reinterpret_cast<const float*>(stage);
    const float* vs = reinterpret_cast<const float*>(stage + kHKtBytes);
    // S^T (raw scores) in two independent accumulation chains.
    floatx4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int pp = 0; pp < 16; pp += 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sa = __builtin_amdgcn_mfma_f32_16x16x4f32(kts[kt_lane[j] + 256 * pp], qr[4 * pp + j], sa, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sb = __builtin_amdgcn_mfma_f32_16x16x4f32(kts[kt_lane[j] + 256 * (pp + 1)], qr[4 * pp + 4 + j], sb, 0, 0,
                                                  0);
      if ((pp & 3) == 2) __builtin_amdgcn_sched_barrier(0);  // bound the operand reads in flight
    }
    floatx4 s = sa + sb;
    // Keys past T, and (causal) keys after the query, are excluded.
    if (k0 + kHK > p.T || (p.causal && k0 + kHK - 1 > q0)) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 4 * g + r;
        if (key >= p.T || (p.causal && key > qi)) s[r] = -INFINITY;
      }
    }
    const float mt = max_quarters(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
    const float m_new = fmaxf(m_run, mt * a.scale_log2);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;  // a query with no visible key yet
    float lt = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], a.scale_log2, -m_use));
      lt += s[r];
    }
    lt = sum_quarters(lt);
    if (__builtin_amdgcn_read_exec() & __ballot(m_new > m_run)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      l_run *= alpha;
#pragma unroll
      for (int cb = 0; cb < 16; ++cb) o[cb] *= alpha;
    }
    l_run += lt;
    m_run = m_new;
    // O^T += V^T P^T.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int cb = 0; cb < 16; ++cb)
        o[cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(vs[v_lane[cb & 3] + r * kHD + (cb & ~3) * 16], s[r], o[cb], 0,
                                                     0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  issue(S0, t_begin * kHK);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int t = t_begin;
  for (; t + 1 < t_end; t += 2) {
    issue(S1, (t + 1) * kHK);
    compute(S0, t * kHK);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t + 2 < t_end) issue(S0, (t + 2) * kHK);
    compute(S1, (t + 1) * kHK);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (t < t_end) compute(S0, t * kHK);  // odd count: the last tile was issued into S0

  if (qi >= p.T) return;
  if (a.splits == 1) {
    const float inv_l = 1.0f / l_run;
    float* orow = p.o + (size_t)qi * p.o_rs + (size_t)hq * kHD + 4 * g;
#pragma unroll
    for (int cb = 0; cb < 16; ++cb) *reinterpret_cast<floatx4*>(orow + 16 * cb) = o[cb] * inv_l;
  } else {
    const size_t row = ((size_t)split * p.T + qi) * p.q_heads + hq;
    float* orow = p.part_o + row * kHD + 4 * g;
#pragma unroll
    for (int cb = 0; cb < 16; ++cb) *reinterpret_cast<floatx4*>(orow + 16 * cb) = o[cb];
    if (g == 0) {
      p.part_ml[2 * row] = m_run;
      p.part_ml[2 * row + 1] = l_run;
    }
  }
}

// Merges the splits of (token, query head) pairs, one wave each: splits with
// keys for the token are added in split order with weights 2^(m_z - max m).
// Splits are read in batches of 16 whose loads (max, sum and O) all issue
// together; a later batch with a larger maximum rescales what came before.
template <int kD>
__global__ __launch_bounds__(256) void flash_attn_f32_combine_kernel(const AttnLaunch a) {
  constexpr int kBatch = 16;
  constexpr int kC4 = (kD / 4 + 63) / 64;  // floatx4 columns per lane
  const AttnF32Params& p = a.p;
  const int pair = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = (int)(threadIdx.x & 63);
  if (pair >= p.T * p.q_heads) return;
  const int t = pair / p.q_heads;
  const int hq = pair - t * p.q_heads;
  const int qbase = (t / a.qspan) * a.qspan;
  const int nv = (key_tiles(p, qbase, a.qspan, a.tkeys) + a.chunk - 1) / a.chunk;
  const size_t stride = (size_t)p.T * p.q_heads;  // rows between splits
  floatx4 acc[kC4];
#pragma unroll
  for (int c = 0; c < kC4; ++c) acc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
  float mstar = -INFINITY, l = 0.0f;
  for (int z0 = 0; z0 < nv; z0 += kBatch) {
    float m[kBatch], lz[kBatch];
    floatx4 v[kBatch][kC4];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const size_t row = (size_t)min(z0 + i, nv - 1) * stride + pair;  // past nv: a valid row, weight zero
      m[i] = z0 + i < nv ? p.part_ml[2 * row] : -INFINITY;
      lz[i] = p.part_ml[2 * row + 1];
#pragma unroll
      for (int c = 0; c < kC4; ++c) {
        const int c4 = lane + 64 * c;
        v[i][c] = c4 < kD / 4 ? reinterpret_cast<const floatx4*>(p.part_o + row * kD)[c4] : floatx4{0.f, 0.f, 0.f, 0.f};
      }
    }
    float mb = mstar;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) mb = fmaxf(mb, m[i]);
    if (mb > mstar) {  // finite: the first batch holds split 0, whose keys every token sees
      const float alpha = __builtin_amdgcn_exp2f(mstar - mb);
      l *= alpha;
#pragma unroll
      for (int c = 0; c < kC4; ++c) acc[c] *= alpha;
      mstar = mb;
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const float w = __builtin_amdgcn_exp2f(m[i] - mstar);  // zero past nv and for splits without keys for t
      l += w * lz[i];
#pragma unroll
      for (int c = 0; c < kC4; ++c) acc[c] += w * v[i][c];
    }
  }
  const float inv = 1.0f / l;
#pragma unroll
  for (int c = 0; c < kC4; ++c) {
    const int c4 = lane + 64 * c;
    if (c4 < kD / 4) reinterpret_cast<floatx4*>(p.o + (size_t)t * p.o_rs + (size_t)hq * kD)[c4] = acc[c] * inv;
  }
}

struct AttnPlanF32 {
  bool h8;  // the head-dim-256 kernel for query heads sharing a K/V head in eights
  int waves, wh, wq, chunk, splits, qspan, tkeys;
  int items;  // h8: work items (query block, split) per head group
  size_t partial_bytes;
};

// Sum over query blocks of ceil(tiles_b / c): the (query block, split) items
// that have keys when the key range is cut into chunks of c tiles of kHK keys
// (the count flash_attn_f32_d256_h8_kernel decodes its work items by).
int h8_items(int T, int causal, int c) {
  AttnF32Params p{};
  p.T = T;
  p.causal = causal;
  int w = 0;
  for (int b = 0; b * kHQ < T; ++b) w += (key_tiles(p, b * kHQ, kHQ, kHK) + c - 1) / c;
  return w;
}

// Head dims 64 / 128 use two-wave workgroups (two resident per SIMD-quad);
// 256 uses four waves (its Q and O^T registers need a SIMD each), or, when
// query heads share a K/V head in eights, the eight-wave 16-query kernel.
// Query heads sharing a K/V head go into one workgroup; otherwise its waves
// take consecutive query blocks.  A grid of fewer workgroups than CUs splits
// the key range: the generic kernels into about one workgroup-split per CU;
// the 16-query kernel (one workgroup per CU) into the chunk of c tiles that
// minimises rounds(c) * c, rounds being its work items (its whole grid) over
// 256, the larger c on ties (fewer partials).
AttnPlanF32 plan_attention(int T, int q_heads, int group, int d, int causal) {
  AttnPlanF32 pl{};
  const int qblocks16 = (T + kHQ - 1) / kHQ;
  if (d == 256 && group % 8 == 0 && q_heads % 8 == 0) {
    pl.h8 = true;
    pl.waves = 8;
    pl.wh = 8;
    pl.wq = 1;
    pl.qspan = kHQ;
    pl.tkeys = kHK;
    const int qblocks = qblocks16;
    const int tiles = (T + kHK - 1) / kHK;
    const long long hgroups = q_heads / 8;
    long long best = -1;
    pl.chunk = tiles;  // enough workgroups without a split
    for (int c = 1; c <= tiles && qblocks * hgroups < 256; ++c) {
      const long long rounds = (hgroups * h8_items(T, causal, c) + 255) / 256;
      const long long cost = rounds * c;
      if (best < 0 || cost <= best) {
        best = cost;
        pl.chunk = c;
      }
      if (rounds == 1) break;  // larger chunks only lengthen the one round
    }
    pl.items = h8_items(T, causal, pl.chunk);
  } else {
    pl.waves = d == 256 ? 4 : 2;
    pl.wh = 1;
    for (int w = pl.waves; w > 1; w >>= 1)
      if (group % w == 0) {
        pl.wh = w;
        break;
      }
    pl.wq = pl.waves / pl.wh;
    pl.qspan = pl.wq * kQW;
    pl.tkeys = kKB;
    const long long wgs = (long long)((T + pl.qspan - 1) / pl.qspan) * (q_heads / pl.wh);
    const int tiles = (T + kKB - 1) / kKB;
    pl.chunk = tiles;
    if (wgs < 256 && tiles >= 2)
      pl.chunk = (int)std::max(1LL, std::min((long long)tiles, (tiles * wgs + 255) / 256));
  }
  const int tiles = (T + pl.tkeys - 1) / pl.tkeys;
  pl.splits = (tiles + pl.chunk - 1) / pl.chunk;
  pl.partial_bytes = pl.splits > 1 ? (size_t)pl.splits * T * q_heads * (d + 2) * sizeof(float) : 0;
  return pl;
}

template <int kD, int kW>
hipError_t launch_plan(const AttnLaunch& a, const AttnPlanF32& pl, hipStream_t stream) {
  const dim3 grid((unsigned)((a.p.T + a.qspan - 1) / a.qspan), (unsigned)(a.p.q_heads / a.wh), (unsigned)a.splits);
  if (pl.h8)
    hipLaunchKernelGGL(flash_attn_f32_d256_h8_kernel, dim3((unsigned)pl.items, (unsigned)(a.p.q_heads / 8)), dim3(512),
                       0, stream, a);
  else if constexpr (kD == 64)
    hipLaunchKernelGGL(flash_attn_f32_d64_kernel, grid, dim3(64 * kW), 0, stream, a);
  else if constexpr (kD == 128)
    hipLaunchKernelGGL(flash_attn_f32_d128_kernel, grid, dim3(64 * kW), 0, stream, a);
  else
    hipLaunchKernelGGL(flash_attn_f32_d256_kernel, grid, dim3(64 * kW), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  const int pairs = a.p.T * a.p.q_heads;
  hipLaunchKernelGGL(flash_attn_f32_combine_kernel<kD>, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

bool flash_attn_f32_supported(int head_dim) { return head_dim == 64 || head_dim == 128 || head_dim == 256; }

size_t flash_attn_f32_partial_bytes(int T, int q_heads, int group, int head_dim, int causal) {
  if (!flash_attn_f32_supported(head_dim) || T <= 0) return 0;
  return plan_attention(T, q_heads, group, head_dim, causal).partial_bytes;
}

void flash_attn_f32_bind_partials(AttnF32Params& p, int head_dim, void* buffer) {
  const AttnPlanF32 pl = plan_attention(p.T, p.q_heads, p.group, head_dim, p.causal);
  p.part_o = static_cast<float*>(buffer);
  p.part_ml = buffer == nullptr ? nullptr : p.part_o + (size_t)pl.splits * p.T * p.q_heads * head_dim;
}

hipError_t launch_flash_attn_f32(const AttnF32Params& p, int head_dim, float scale, hipStream_t stream) {
  if (!flash_attn_f32_supported(head_dim) || p.T <= 0 || p.q_heads <= 0 || p.group <= 0 || p.q_heads % p.group != 0 ||
      (p.q_rs & 3) != 0 || (p.v_rs & 3) != 0 || (p.o_rs & 3) != 0 || (p.q_hs & 3) != 0 || (p.v_hs & 3) != 0 ||
      (reinterpret_cast<uintptr_t>(p.q) & 15) != 0 || (reinterpret_cast<uintptr_t>(p.v) & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(p.o) & 15) != 0)
    return hipErrorInvalidValue;
  // The HBM -> LDS transfers move 16-byte chunks of K^T rows and V rows and
  // address each head's K^T and V with 32-bit byte offsets.
  if ((p.kt_rs & 3) != 0 || (p.kt_hs & 3) != 0 || (reinterpret_cast<uintptr_t>(p.kt) & 15) != 0 ||
      (size_t)head_dim * p.kt_rs * 4 >= (1ull << 31) || (size_t)p.T * p.v_rs * 4 >= (1ull << 31) ||
      p.kt_rs < p.T || p.v_rs < head_dim)
    return hipErrorInvalidValue;
  const AttnPlanF32 pl = plan_attention(p.T, p.q_heads, p.group, head_dim, p.causal);
  if (pl.splits > 1 && (p.part_o == nullptr || p.part_ml == nullptr)) return hipErrorInvalidValue;
  AttnLaunch a{};
  a.p = p;
  a.wh = pl.wh;
  a.wq = pl.wq;
  a.chunk = pl.chunk;
  a.splits = pl.splits;
  a.qspan = pl.qspan;
  a.tkeys = pl.tkeys;
  a.scale_log2 = scale * 1.4426950408889634f;
  if (head_dim == 64) return launch_plan<64, 2>(a, pl, stream);
  if (head_dim == 128) return launch_plan<128, 2>(a, pl, stream);
  return launch_plan<256, 4>(a, pl, stream);
}

}  // namespace prom
