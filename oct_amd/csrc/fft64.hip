// Binary64 complex FFT (forward, unnormalised, power-of-two lengths <= 2^20).
//
// Contract: internal/fft/fft.go:206-258 (bit-reversal permutation, then
// iterative radix-2 decimation-in-time butterflies with the n/2 roots
// w_j = cos(-2*pi/n*j) + i sin(-2*pi/n*j)); entry validation and status codes:
// internal/prometheus/native/reactor_concept_fft.cpp:97-104 and :36-76; the
// host-side twiddle table, cached per length, follows :50-57.
//
// MI355X design.  A length L <= 4096 transform is held entirely in LDS by one
// workgroup (64 KiB of double2): the bit-reversed load, log2(L) butterfly
// stages separated by barriers, and the store.  It performs exactly the
// reference's butterflies with its twiddles and no contraction, so its output
// is bit-identical to the CPU contract.  Longer transforms use the four-step
// factorisation N = N1 * N2 (N1, N2 <= 1024 for N <= 2^20), with n = N2*n1 + n2
// and k = k1 + N1*k2:
//   pass 1: for every column n2, an N1-point transform over x[N2*n1 + n2],
//           multiplied by W_N^(n2*k1) on the way out and stored as T(k1, n2);
//   pass 2: for every row k1, an N2-point transform over T(k1, n2), stored
//           to X[k1 + N1*k2].
// T holds its rows in tiles of G = 4096/N2 (T(k1, n2) at
// (k1/G)*N2*G + n2*G + k1%G), so that pass 2 reads whole tiles.
// Both passes run fft_wave_pass_kernel: a wave holds 1024 points in
// registers, a workgroup four adjacent columns (rows), so that strided loads
// and stores touch 64-byte runs; the whole 16 MiB working set of a 2^20-point
// transform stays resident in the MI355X's 256 MiB Infinity Cache between the
// passes.
#include <math.h>
#include <string.h>

#include <vector>

#include "reactor_internal.h"

namespace prom {

namespace {

constexpr uint32_t kFftThreads = 256;
constexpr uint32_t kFftMaxLds = 4096;  // double2 elements per workgroup (64 KiB)
constexpr uint32_t kFftMaxLog2 = 20;
constexpr uint32_t kFftPerThread = kFftMaxLds / kFftThreads;  // elements each thread loads and stores

// Go's complex product (xu - yv) + (xv + yu)i with every operation rounded.
__device__ __forceinline__ double2 cmul(double2 w, double2 v) {
#pragma clang fp contract(off)
  double2 t;
  t.x = w.x * v.x - w.y * v.y;
  t.y = w.x * v.y + w.y * v.x;
  return t;
}

// One workgroup transforms `seqs` sequences of length L = 2^log2l.  Global
// sequence q = blockIdx.x * seqs + s reads element i at
// in[q * in_seq + i * in_elem] and writes element k at out[q * out_seq + k * out_elem].
// seq_fast_in / seq_fast_out pick the thread order of the global accesses
// (adjacent threads on adjacent sequences when the sequences are adjacent in
// memory).  post multiplies output k of sequence q by W_N^(q*k).
//
// The sub-transform's twiddles W_L^j = roots[j * N / L] (j < L/2) are copied
// to LDS once.  Butterfly stages run two at a time: a thread loads the four
// elements p, p+h, p+2h, p+3h of a stage pair (h = 2^(lg-1)), performs the two
// stage-lg butterflies and then the two stage-(lg+1) butterflies in
// registers, and stores them back -- the same operations on the same values as
// one stage per barrier, with half the barriers and LDS round trips.
__global__ __launch_bounds__(256) void fft_lds_kernel(const double2* __restrict__ in, double2* __restrict__ out,
                                                      const double2* __restrict__ roots, uint32_t n_total,
                                                      uint32_t log2l, uint32_t log2seqs, uint64_t in_seq,
                                                      uint64_t in_elem, uint64_t out_seq, uint64_t out_elem,
                                                      int post, int seq_fast_in, int seq_fast_out) {
#pragma clang fp contract(off)
  extern __shared__ double2 smem[];
  const uint32_t L = 1u << log2l;
  const uint32_t seqs = 1u << log2seqs;
  const uint32_t total = L << log2seqs;
  double2* buf = smem;
  double2* tw = smem + total;
  const uint32_t tstride = n_total >> log2l;
  for (uint32_t j = threadIdx.x; j < (L >> 1); j += blockDim.x) tw[j] = roots[(size_t)j * tstride];
  // Hardware deals workgroups to the 8 XCDs round-robin; remap so that each
  // XCD takes a contiguous range of sequences and the 128-byte lines shared
  // by neighbouring sequences (strided passes) are filled in one L2.
  uint32_t blk = blockIdx.x;
  if ((gridDim.x & 7u) == 0u) blk = (blk & 7u) * (gridDim.x >> 3) + (blk >> 3);
  const uint64_t q0 = (uint64_t)blk << log2seqs;
  // Every global load of the thread is issued before the first LDS store, so
  // the strided reads overlap instead of waiting one at a time.
  double2 v[kFftPerThread];
#pragma unroll
  for (uint32_t u = 0; u < kFftPerThread; ++u) {
    const uint32_t e = threadIdx.x + u * kFftThreads;
    if (e < total) {
      const uint32_t s = seq_fast_in ? (e & (seqs - 1)) : (e >> log2l);
      const uint32_t i = seq_fast_in ? (e >> log2seqs) : (e & (L - 1));
      v[u] = in[(q0 + s) * in_seq + (uint64_t)i * in_elem];
    }
  }
#pragma unroll
  for (uint32_t u = 0; u < kFftPerThread; ++u) {
    const uint32_t e = threadIdx.x + u * kFftThreads;
    if (e < total) {
      const uint32_t s = seq_fast_in ? (e & (seqs - 1)) : (e >> log2l);
      const uint32_t i = seq_fast_in ? (e >> log2seqs) : (e & (L - 1));
      const uint32_t r = log2l == 0 ? 0u : (__brev(i) >> (32u - log2l));
      buf[(s << log2l) + r] = v[u];
    }
  }
  __syncthreads();
  uint32_t lg = 1;
  for (; lg + 1 <= log2l; lg += 2) {
    const uint32_t h = 1u << (lg - 1);
    const uint32_t groups = total >> 2;
    for (uint32_t g = threadIdx.x; g < groups; g += blockDim.x) {
      const uint32_t s = g >> (log2l - 2);
      const uint32_t gg = g & ((L >> 2) - 1);
      const uint32_t j = gg & (h - 1);
      const uint32_t p = (s << log2l) + ((gg >> (lg - 1)) << (lg + 1)) + j;
      const double2 a0 = buf[p], a1 = buf[p + h], a2 = buf[p + 2 * h], a3 = buf[p + 3 * h];
      const double2 w1 = tw[j << (log2l - lg)];
      double2 t = cmul(w1, a1);
      const double2 b0 = make_double2(a0.x + t.x, a0.y + t.y);
      const double2 b1 = make_double2(a0.x - t.x, a0.y - t.y);
      t = cmul(w1, a3);
      const double2 b2 = make_double2(a2.x + t.x, a2.y + t.y);
      const double2 b3 = make_double2(a2.x - t.x, a2.y - t.y);
      t = cmul(tw[j << (log2l - lg - 1)], b2);
      buf[p] = make_double2(b0.x + t.x, b0.y + t.y);
      buf[p + 2 * h] = make_double2(b0.x - t.x, b0.y - t.y);
      t = cmul(tw[(j + h) << (log2l - lg - 1)], b3);
      buf[p + h] = make_double2(b1.x + t.x, b1.y + t.y);
      buf[p + 3 * h] = make_double2(b1.x - t.x, b1.y - t.y);
    }
    __syncthreads();
  }
  if (lg == log2l) {  // an odd stage count leaves the last stage (span L) alone
    const uint32_t half = L >> 1;
    for (uint32_t b = threadIdx.x; b < (total >> 1); b += blockDim.x) {
      const uint32_t s = b >> (log2l - 1);
      const uint32_t j = b & (half - 1);
      const uint32_t p = (s << log2l) + j;
      const double2 t = cmul(tw[j], buf[p + half]);
      const double2 a = buf[p];
      buf[p] = make_double2(a.x + t.x, a.y + t.y);
      buf[p + half] = make_double2(a.x - t.x, a.y - t.y);
    }
    __syncthreads();
  }
  const uint32_t half_n = n_total >> 1;
  double2 w[kFftPerThread];
#pragma unroll
  for (uint32_t u = 0; u < kFftPerThread; ++u) {
    const uint32_t e = threadIdx.x + u * kFftThreads;
    if (e < total) {
      const uint32_t s = seq_fast_out ? (e & (seqs - 1)) : (e >> log2l);
      const uint32_t k = seq_fast_out ? (e >> log2seqs) : (e & (L - 1));
      v[u] = buf[(s << log2l) + k];
      if (post) {
        const uint64_t p = (q0 + s) * (uint64_t)k;  // < N
        w[u] = roots[p < half_n ? p : p - half_n];
      }
    }
  }
#pragma unroll
  for (uint32_t u = 0; u < kFftPerThread; ++u) {
    const uint32_t e = threadIdx.x + u * kFftThreads;
    if (e < total) {
      const uint32_t s = seq_fast_out ? (e & (seqs - 1)) : (e >> log2l);
      const uint32_t k = seq_fast_out ? (e >> log2seqs) : (e & (L - 1));
      double2 r = v[u];
      if (post) {
        const uint64_t p = (q0 + s) * (uint64_t)k;
        const double2 wt = p < half_n ? w[u] : make_double2(-w[u].x, -w[u].y);
        r = cmul(wt, r);
      }
      out[(q0 + s) * out_seq + (uint64_t)k * out_elem] = r;
    }
  }
}

// LDS index with one unused slot after every 16 elements: 16-element groups
// written by neighbouring lanes land on distinct bank groups.
__device__ __forceinline__ uint32_t pad16(uint32_t i) { return i + (i >> 4); }

// Lengths L >= 16.  Each of the first total/16 threads owns 16 consecutive
// bit-reversed positions 16b..16b+15 of one sequence: position 16b + k holds
// x[rev(16b + k)] = x[rev'(b) + rev4(k) * L/16] (rev' over log2(L)-4 bits),
// so the thread loads those 16 inputs directly (stride L/16, the bit-reversal
// done by register placement), runs butterfly stages 1-4 in registers -- the
// same operations, operands and twiddles as one stage per barrier -- and
// writes its 16 results contiguously to LDS (padded).  The remaining stages
// (span >= 32) run two per barrier as in fft_lds_kernel, on padded indices.
// Against fft_lds_kernel this removes the bank-conflicted bit-reversed
// scatter and two LDS round trips with their barriers.  kThreads is the
// workgroup size: 256, or 1024 for a single sequence of up to 4096 points,
// whose stages are latency-bound on one workgroup (the threads past the
// register phase's total/16 take the LDS stages and the stores).
template <uint32_t kThreads>
__device__ __forceinline__ void fft_reg16_body(const double2* __restrict__ in, double2* __restrict__ out,
                                               const double2* __restrict__ roots, uint32_t n_total, uint32_t log2l,
                                               uint32_t log2seqs, uint64_t in_seq, uint64_t in_elem,
                                               uint64_t out_seq, uint64_t out_elem, int post, int seq_fast_in,
                                               int seq_fast_out) {
#pragma clang fp contract(off)
  constexpr uint32_t kPer = kFftMaxLds / kThreads;  // output elements per thread
  extern __shared__ double2 smem[];
  const uint32_t L = 1u << log2l;
  const uint32_t seqs = 1u << log2seqs;
  const uint32_t total = L << log2seqs;
  double2* buf = smem;
  double2* tw = smem + pad16(total);
  const uint32_t tstride = n_total >> log2l;
  for (uint32_t j = threadIdx.x; j < (L >> 1); j += blockDim.x) tw[j] = roots[(size_t)j * tstride];
  uint32_t blk = blockIdx.x;
  if ((gridDim.x & 7u) == 0u) blk = (blk & 7u) * (gridDim.x >> 3) + (blk >> 3);
  const uint64_t q0 = (uint64_t)blk << log2seqs;

  const uint32_t lgq = log2l - 4;        // log2 of 16-element groups per sequence
  const uint32_t groups = total >> 4;    // <= 256
  const uint32_t g = threadIdx.x;
  double2 a[16];
  uint32_t s = 0, b = 0;
  if (g < groups) {
    s = seq_fast_in ? (g & (seqs - 1)) : (g >> lgq);
    b = seq_fast_in ? (g >> log2seqs) : (g & ((1u << lgq) - 1));
    const uint32_t base = lgq == 0 ? 0u : (__brev(b) >> (32u - lgq));
    const double2* src = in + (q0 + s) * in_seq;
#pragma unroll
    for (uint32_t m = 0; m < 16; ++m) {
      const uint32_t k = ((m & 1u) << 3) | ((m & 2u) << 1) | ((m & 4u) >> 1) | ((m & 8u) >> 3);  // rev4(m)
      a[k] = src[(uint64_t)(base + (m << lgq)) * in_elem];
    }
  }
  __syncthreads();  // twiddles in LDS
  if (g < groups) {
#pragma unroll
    for (uint32_t lg = 1; lg <= 4; ++lg) {
      const uint32_t half = 1u << (lg - 1);
#pragma unroll
      for (uint32_t p = 0; p < 16; ++p) {
        if (p & half) continue;
        const double2 t = cmul(tw[(p & (half - 1)) << (log2l - lg)], a[p + half]);
        const double2 x = a[p];
        a[p] = make_double2(x.x + t.x, x.y + t.y);
        a[p + half] = make_double2(x.x - t.x, x.y - t.y);
      }
    }
    double2* dst = buf + 17u * ((s << lgq) + b);  // pad16((s << log2l) + 16 b)
#pragma unroll
    for (uint32_t k = 0; k < 16; ++k) dst[k] = a[k];
  }
  __syncthreads();
  uint32_t lg = 5;
  for (; lg + 1 <= log2l; lg += 2) {
    const uint32_t h = 1u << (lg - 1);
    const uint32_t quads = total >> 2;
    for (uint32_t q = threadIdx.x; q < quads; q += blockDim.x) {
      const uint32_t sq = q >> (log2l - 2);
      const uint32_t gg = q & ((L >> 2) - 1);
      const uint32_t j = gg & (h - 1);
      const uint32_t p = (sq << log2l) + ((gg >> (lg - 1)) << (lg + 1)) + j;
      const uint32_t i0 = pad16(p), i1 = pad16(p + h), i2 = pad16(p + 2 * h), i3 = pad16(p + 3 * h);
      const double2 a0 = buf[i0], a1 = buf[i1], a2 = buf[i2], a3 = buf[i3];
      const double2 w1 = tw[j << (log2l - lg)];
      double2 t = cmul(w1, a1);
      const double2 b0 = make_double2(a0.x + t.x, a0.y + t.y);
      const double2 b1 = make_double2(a0.x - t.x, a0.y - t.y);
      t = cmul(w1, a3);
      const double2 b2 = make_double2(a2.x + t.x, a2.y + t.y);
      const double2 b3 = make_double2(a2.x - t.x, a2.y - t.y);
      t = cmul(tw[j << (log2l - lg - 1)], b2);
      buf[i0] = make_double2(b0.x + t.x, b0.y + t.y);
      buf[i2] = make_double2(b0.x - t.x, b0.y - t.y);
      t = cmul(tw[(j + h) << (log2l - lg - 1)], b3);
      buf[i1] = make_double2(b1.x + t.x, b1.y + t.y);
      buf[i3] = make_double2(b1.x - t.x, b1.y - t.y);
    }
    __syncthreads();
  }
  if (lg == log2l) {  // an odd count of LDS stages leaves the last stage (span L) alone
    const uint32_t half = L >> 1;
    for (uint32_t bb = threadIdx.x; bb < (total >> 1); bb += blockDim.x) {
      const uint32_t sq = bb >> (log2l - 1);
      const uint32_t j = bb & (half - 1);
      const uint32_t p = (sq << log2l) + j;
      const uint32_t i0 = pad16(p), i1 = pad16(p + half);
      const double2 t = cmul(tw[j], buf[i1]);
      const double2 x = buf[i0];
      buf[i0] = make_double2(x.x + t.x, x.y + t.y);
      buf[i1] = make_double2(x.x - t.x, x.y - t.y);
    }
    __syncthreads();
  }
  const uint32_t half_n = n_total >> 1;
  double2 v[kPer], w[kPer];
#pragma unroll
  for (uint32_t u = 0; u < kPer; ++u) {
    const uint32_t e = threadIdx.x + u * kThreads;
    if (e < total) {
      const uint32_t so = seq_fast_out ? (e & (seqs - 1)) : (e >> log2l);
      const uint32_t k = seq_fast_out ? (e >> log2seqs) : (e & (L - 1));
      v[u] = buf[pad16((so << log2l) + k)];
      if (post) {
        const uint64_t pp = (q0 + so) * (uint64_t)k;  // < N
        w[u] = roots[pp < half_n ? pp : pp - half_n];
      }
    }
  }
#pragma unroll
  for (uint32_t u = 0; u < kPer; ++u) {
    const uint32_t e = threadIdx.x + u * kThreads;
    if (e < total) {
      const uint32_t so = seq_fast_out ? (e & (seqs - 1)) : (e >> log2l);
      const uint32_t k = seq_fast_out ? (e >> log2seqs) : (e & (L - 1));
      double2 r = v[u];
      if (post) {
        const uint64_t pp = (q0 + so) * (uint64_t)k;
        const double2 wt = pp < half_n ? w[u] : make_double2(-w[u].x, -w[u].y);
        r = cmul(wt, r);
      }
      out[(q0 + so) * out_seq + (uint64_t)k * out_elem] = r;
    }
  }
}

__global__ __launch_bounds__(256) void fft_reg16_kernel(const double2* __restrict__ in, double2* __restrict__ out,
                                                        const double2* __restrict__ roots, uint32_t n_total,
                                                        uint32_t log2l, uint32_t log2seqs, uint64_t in_seq,
                                                        uint64_t in_elem, uint64_t out_seq, uint64_t out_elem,
                                                        int post, int seq_fast_in, int seq_fast_out) {
  fft_reg16_body<256>(in, out, roots, n_total, log2l, log2seqs, in_seq, in_elem, out_seq, out_elem, post,
                      seq_fast_in, seq_fast_out);
}

__global__ __launch_bounds__(1024) void fft_reg16_wide_kernel(const double2* __restrict__ in,
                                                              double2* __restrict__ out,
                                                              const double2* __restrict__ roots, uint32_t n_total,
                                                              uint32_t log2l, uint32_t log2seqs, uint64_t in_seq,
                                                              uint64_t in_elem, uint64_t out_seq, uint64_t out_elem,
                                                              int post, int seq_fast_in, int seq_fast_out) {
  fft_reg16_body<1024>(in, out, roots, n_total, log2l, log2seqs, in_seq, in_elem, out_seq, out_elem, post,
                       seq_fast_in, seq_fast_out);
}

// ---------------------------------------------------------------------------
// Four-step passes of the long transforms (N > 4096, sub-transform lengths
// L in [64, 1024]).  One wave holds 1024 elements in registers, 16 per lane:
// 1024/L whole sequences.  Element e of a wave (e = s*L + pos, position pos of
// its sequence s in bit-reversed order) moves through three register phases,
// each running the butterfly stages of four bits of pos:
//   phase 1: lane = e bits 4-9,        element j = e bits 0-3 (stages 1-4);
//   phase 2: lane = e bits 0-3, 8-9,   j = e bits 4-7         (stages 5-8);
//   phase 3: lane = e bits 0-3, 6-7,   j = e bits 4-5, 8-9    (stages 9-10).
// Between phases the wave exchanges its elements through its own 16 KiB of
// LDS (16-byte slot e ^ ((e >> 4) & 15): the 16 lanes of each access touch 16
// distinct bank groups); LDS operations of one wave complete in order, so the
// exchange needs no workgroup barrier and the four waves of a workgroup run
// their stages independently.  Each butterfly is the reference's (same
// operands, twiddle W_L^((p mod half) * L/2^t), no contraction); only the
// order in which independent butterflies run differs from fft_reg16_kernel.
// Global loads and stores run in memory order through a workgroup tile
// (fft_wave_pass_body); each thread issues all 16 of its loads at once (64 KiB
// per workgroup in flight).
//
// Twiddles come from a compact per-length table built on the host from the
// same roots: the stage twiddles of each pass (L/2 entries), lo[j] = W_N^j
// (j < 1024) and hi[h] = W_N^(1024 h) (h < N/1024), staged in LDS once per
// workgroup.  The four-step twiddle W_N^p, p = n2 * k1, is hi[p >> 10] *
// lo[p & 1023] (one extra rounded product; well inside fft.go:176-192's
// 1e-12 agreement bound), which replaces a scattered read of the N/2-entry
// roots table per output element.
constexpr uint32_t kPassWaves = 4;
constexpr uint32_t kWaveElems = 1024;

__device__ __forceinline__ uint32_t xslot(uint32_t e) { return e ^ ((e >> 4) & 15u); }

// Streaming 16-byte accesses for the passes' data: every element is read once
// and written once per pass, so neither side is kept in the L2.  With ordinary
// accesses the dirty lines a pass leaves behind are written back while the
// next pass runs, which made the first pass 1.7x slower than the second;
// streaming both sides takes 2^20 points from 33.4 to 28 us.
typedef double stream_double2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ double2 load_stream(const double2* p) {
  const stream_double2 v = __builtin_nontemporal_load(reinterpret_cast<const stream_double2*>(p));
  return make_double2(v.x, v.y);
}

__device__ __forceinline__ void store_stream(double2* p, double2 v) {
  const stream_double2 w = {v.x, v.y};
  __builtin_nontemporal_store(w, reinterpret_cast<stream_double2*>(p));
}

__device__ __forceinline__ void butterfly(double2& x, double2& y, double2 w) {
#pragma clang fp contract(off)
  const double2 t = cmul(w, y);
  const double2 u = x;
  x = make_double2(u.x + t.x, u.y + t.y);
  y = make_double2(u.x - t.x, u.y - t.y);
}

// A workgroup takes R = 4096/L adjacent sequences q = blk*R + r.  Pass 1
// (kColumns) reads column q of x (element i at x[i*N2 + q]) and writes the
// twiddled outputs to T in tiles of G = 4096/N2 rows, T[(k/G)*N2*G + q*G + k%G];
// pass 2 reads row q of T (element i at T[(q/G)*N2*G + i*G + q%G], R = G, so one
// workgroup's rows are one contiguous 64 KiB tile) and writes X[q + k*N1].  The
// global loads and stores go in memory order through a 64 KiB LDS tile (the
// 16-byte slot of tile index f at sslot(f)): inputs f = i*R + r, outputs
// f = ((k/G)*R + r)*G + k%G in pass 1 and f = k*R + r in pass 2, so
// consecutive lanes move consecutive addresses -- runs of 64 bytes (the
// column reads and the final transposed writes at L = 1024), 256 bytes (the
// tiled T writes) or whole tiles (the T reads).  The tile and the waves'
// exchange buffers share the same LDS, ordered by workgroup barriers.
__device__ __forceinline__ uint32_t sslot(uint32_t f) { return f ^ ((f >> 4) & 15u) ^ ((f >> 8) & 15u); }
// Pass 1's output tile: bits 4-7 enter rotated by two, which keeps the tiled
// (k/G, r, k%G) order conflict-free at N >= 2^19 (at most two-way below).
__device__ __forceinline__ uint32_t oslot1(uint32_t f) {
  const uint32_t x = (f >> 4) & 15u;
  return f ^ (((x << 2) | (x >> 2)) & 15u) ^ ((f >> 8) & 15u);
}

// The transform size is a template parameter: every shift, mask and LDS slot
// offset that depends only on it is a compile-time constant, which removed
// about half of the kernels' integer instructions (at one wave per SIMD each
// VALU instruction costs the wave its issue slot).
template <bool kColumns, uint32_t log2n1, uint32_t log2n2>
__device__ __forceinline__ void fft_wave_pass_body(const double2* __restrict__ in, double2* __restrict__ out,
                                                   const double2* __restrict__ tables, uint32_t tw_off,
                                                   uint32_t lo_off) {
#pragma clang fp contract(off)
  extern __shared__ double2 smem[];
  constexpr uint32_t log2l = kColumns ? log2n1 : log2n2;
  constexpr uint32_t hi_count = 1u << (log2n1 + log2n2 - 10u);
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  constexpr uint32_t L = 1u << log2l;
  constexpr uint32_t lgr = 12u - log2l;  // log2 of sequences per workgroup
  constexpr uint32_t lgg = 12u - log2n2;  // log2 of the T tile height G
  constexpr uint32_t lgs = 10u - log2l;  // log2 of sequences per wave
  double2* xb = smem + wave * kWaveElems;
  double2* tw = smem + kPassWaves * kWaveElems;
  double2* lo = tw + (L >> 1);
  double2* hi = lo + 1024;
  uint32_t blk = blockIdx.x;
  if ((gridDim.x & 7u) == 0u) blk = (blk & 7u) * (gridDim.x >> 3) + (blk >> 3);
  const uint64_t qwg = (uint64_t)blk << lgr;
  const uint64_t q0 = qwg + ((uint64_t)wave << lgs);

  // Table entries of this thread (tw: L/2 <= 512, lo: 1024, hi: N/1024 <= 1024
  // entries over 256 threads) and the 16 tile elements: every load is issued
  // before the first LDS store (a loop of load-then-store waits one memory
  // round trip per iteration).  Table indices past the end are clamped, so
  // the surplus threads load and store the last entry again (same value,
  // same slot).
  constexpr uint32_t kT = kPassWaves * 64;
  constexpr uint32_t tw_last = (L >> 1) - 1u, hi_last = hi_count - 1u;
  double2 rt[2], rl[4], rh[4];
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) rt[u] = tables[tw_off + min(tid + u * kT, tw_last)];
  if constexpr (kColumns) {
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
      rl[u] = tables[lo_off + tid + u * kT];
      rh[u] = tables[lo_off + 1024u + min(tid + u * kT, hi_last)];
    }
  }
  {
    double2 v[16];
#pragma unroll
    for (uint32_t m = 0; m < 16; ++m) {
      const uint32_t f = tid + m * kT;
      const uint32_t r = f & ((1u << lgr) - 1u);
      const uint64_t i = f >> lgr;
      v[m] = load_stream(in + (kColumns ? qwg + r + (i << log2n2) : (qwg << log2n2) + (i << lgg) + r));
    }
#pragma unroll
    for (uint32_t u = 0; u < 2; ++u) tw[min(tid + u * kT, tw_last)] = rt[u];
    if constexpr (kColumns) {
#pragma unroll
      for (uint32_t u = 0; u < 4; ++u) {
        lo[tid + u * kT] = rl[u];
        hi[min(tid + u * kT, hi_last)] = rh[u];
      }
    }
#pragma unroll
    for (uint32_t m = 0; m < 16; ++m) smem[sslot(tid + m * kT)] = v[m];
  }
  __syncthreads();

  // phase-1 reads: lane holds positions 16 b .. 16 b + 15 of its sequence s1,
  // i.e. inputs rev(b) + m * L/16 (see fft_reg16_body)
  constexpr uint32_t lgq = log2l - 4u;
  const uint32_t s1 = lane >> lgq;
  const uint32_t b1 = lane & ((1u << lgq) - 1u);
  const uint32_t base = __brev(b1) >> (32u - lgq);
  const uint32_t r1 = (wave << lgs) | s1;
  double2 a[16];
#pragma unroll
  for (uint32_t m = 0; m < 16; ++m) {
    const uint32_t k = ((m & 1u) << 3) | ((m & 2u) << 1) | ((m & 4u) >> 1) | ((m & 8u) >> 3);  // rev4(m)
    const uint32_t i = base + (m << lgq);
    a[k] = smem[sslot((i << lgr) | r1)];
  }
  __syncthreads();  // the tile is consumed; the exchange buffers overlay it

  // phase 1: stages 1-4 on the lane's 16 consecutive positions
#pragma unroll
  for (uint32_t t = 1; t <= 4; ++t) {
    const uint32_t half = 1u << (t - 1);
#pragma unroll
    for (uint32_t p = 0; p < 16; ++p) {
      if (p & half) continue;
      butterfly(a[p], a[p + half], tw[(p & (half - 1)) << (log2l - t)]);
    }
  }
#pragma unroll
  for (uint32_t j = 0; j < 16; ++j) xb[xslot(16u * lane + j)] = a[j];
  __builtin_amdgcn_wave_barrier();

  // phase 2: stages 5-8 (those below log2l)
  const uint32_t e2 = (lane & 15u) | ((lane >> 4) << 8);
#pragma unroll
  for (uint32_t j = 0; j < 16; ++j) a[j] = xb[xslot(e2 | (j << 4))];
#pragma unroll
  for (uint32_t t = 5; t <= 8; ++t) {
    if (t > log2l) break;
    const uint32_t hj = 1u << (t - 5);
    const uint32_t pmask = (1u << (t - 1)) - 1u;
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j) {
      if (j & hj) continue;
      const uint32_t pos = (e2 | (j << 4)) & (L - 1u);
      butterfly(a[j], a[j + hj], tw[(pos & pmask) << (log2l - t)]);
    }
  }
  uint32_t e_lane = e2, e_j[16];
#pragma unroll
  for (uint32_t j = 0; j < 16; ++j) e_j[j] = j << 4;
  if (log2l >= 9) {
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j) xb[xslot(e2 | (j << 4))] = a[j];
    __builtin_amdgcn_wave_barrier();
    // phase 3: stages 9-10
    const uint32_t e3 = (lane & 15u) | (((lane >> 4) & 3u) << 6);
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j) e_j[j] = ((j & 3u) << 4) | ((j >> 2) << 8);
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j) a[j] = xb[xslot(e3 | e_j[j])];
#pragma unroll
    for (uint32_t t = 9; t <= 10; ++t) {
      if (t > log2l) break;
      const uint32_t hj = 4u << (t - 9);
      const uint32_t pmask = (1u << (t - 1)) - 1u;
#pragma unroll
      for (uint32_t j = 0; j < 16; ++j) {
        if (j & hj) continue;
        const uint32_t pos = (e3 | e_j[j]) & (L - 1u);
        butterfly(a[j], a[j + hj], tw[(pos & pmask) << (log2l - t)]);
      }
    }
    e_lane = e3;
  }

  // outputs: element j of the lane is position k of sequence s, staged
  // through the tile in output memory order
  __syncthreads();  // every wave is done with its exchange buffer
#pragma unroll
  for (uint32_t j = 0; j < 16; ++j) {
    const uint32_t e = e_lane | e_j[j];
    const uint32_t s = e >> log2l;
    const uint32_t k = e & (L - 1u);
    double2 r = a[j];
    if constexpr (kColumns) {
      const uint64_t p = (q0 + s) * (uint64_t)k;  // < N
      r = cmul(cmul(hi[p >> 10], lo[p & 1023u]), r);
    }
    const uint32_t rq = (wave << lgs) | s;
    const uint32_t f = kColumns ? (((((k >> lgg) << lgr) | rq) << lgg) | (k & ((1u << lgg) - 1u))) : ((k << lgr) | rq);
    smem[kColumns ? oslot1(f) : sslot(f)] = r;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t m = 0; m < 16; ++m) {
    const uint32_t f = tid + m * kT;
    if constexpr (kColumns) {
      const uint64_t kk = f & ((1u << lgg) - 1u);
      const uint64_t r = (f >> lgg) & ((1u << lgr) - 1u);
      const uint64_t kg = f >> (lgg + lgr);
      store_stream(out + (kg << (log2n2 + lgg)) + ((qwg + r) << lgg) + kk, smem[oslot1(f)]);
    } else {
      const uint32_t r = f & ((1u << lgr) - 1u);
      const uint64_t k = f >> lgr;
      store_stream(out + qwg + r + (k << log2n1), smem[sslot(f)]);
    }
  }
}

// Pass 1 (twiddled outputs) and pass 2.  At most two workgroups fit a CU's
// LDS (104 or 72 KiB each), so the kernels may use 256 VGPRs.
template <uint32_t kLog2N1, uint32_t kLog2N2>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void fft_wave_pass1_kernel(
    const double2* __restrict__ in, double2* __restrict__ out, const double2* __restrict__ tables, uint32_t tw_off,
    uint32_t lo_off) {
  fft_wave_pass_body<true, kLog2N1, kLog2N2>(in, out, tables, tw_off, lo_off);
}

template <uint32_t kLog2N1, uint32_t kLog2N2>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void fft_wave_pass2_kernel(
    const double2* __restrict__ in, double2* __restrict__ out, const double2* __restrict__ tables, uint32_t tw_off,
    uint32_t lo_off) {
  fft_wave_pass_body<false, kLog2N1, kLog2N2>(in, out, tables, tw_off, lo_off);
}

uint32_t ilog2(uint32_t v) {
  uint32_t r = 0;
  while ((1u << r) < v) ++r;
  return r;
}

// Sequences per workgroup: enough to fill the chip with >= 512 workgroups when
// possible, within the LDS budget.
uint32_t pick_log2seqs(uint32_t log2l, uint32_t log2count) {
  uint32_t best = 0;
  while (best < log2count && ((1u << (best + 1)) << log2l) <= kFftMaxLds &&
         (log2count - (best + 1)) >= 9u)
    ++best;
  return best;
}

hipError_t launch_pass(const double2* in, double2* out, const double2* roots, uint32_t n, uint32_t log2l,
                       uint32_t log2count, uint64_t in_seq, uint64_t in_elem, uint64_t out_seq, uint64_t out_elem,
                       int post, int fast_in, int fast_out, hipStream_t stream) {
  const uint32_t log2seqs = pick_log2seqs(log2l, log2count);
  const uint32_t blocks = 1u << (log2count - log2seqs);
  // the sequences plus the L/2 twiddles of the sub-transform (at most 64 + 32 KiB)
  const size_t elems = (size_t)1 << (log2l + log2seqs);
  static bool lds_raised = false;
  if (!lds_raised) {
    // the sequences (padded for the 16-element kernel) plus the L/2 twiddles
    const int max_lds = (int)((kFftMaxLds + kFftMaxLds / 16 + kFftMaxLds / 2) * sizeof(double2));
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fft_lds_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, max_lds);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(fft_reg16_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, max_lds);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(fft_reg16_wide_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, max_lds);
    if (e != hipSuccess) return e;
    lds_raised = true;
  }
  if (log2l >= 4) {
    const size_t lds = (elems + elems / 16 + ((size_t)1 << log2l) / 2) * sizeof(double2);
    if (blocks == 1 && log2l >= 10)  // one long sequence: a 1024-thread workgroup
      hipLaunchKernelGGL(fft_reg16_wide_kernel, dim3(1), dim3(1024), lds, stream, in, out, roots, n, log2l, log2seqs,
                         in_seq, in_elem, out_seq, out_elem, post, fast_in, fast_out);
    else
      hipLaunchKernelGGL(fft_reg16_kernel, dim3(blocks), dim3(kFftThreads), lds, stream, in, out, roots, n, log2l,
                         log2seqs, in_seq, in_elem, out_seq, out_elem, post, fast_in, fast_out);
  } else {
    const size_t lds = (elems + ((size_t)1 << log2l) / 2) * sizeof(double2);
    hipLaunchKernelGGL(fft_lds_kernel, dim3(blocks), dim3(kFftThreads), lds, stream, in, out, roots, n, log2l,
                       log2seqs, in_seq, in_elem, out_seq, out_elem, post, fast_in, fast_out);
  }
  return hipGetLastError();
}

// One four-step pass of an n = 2^(log2n1 + log2n2) point transform
// (n in (4096, 2^20], N1 = 2^log2n1 >= N2): n/4096 workgroups of four waves,
// 1024 elements per wave; post selects pass 1 (columns of x to tiled T).
template <uint32_t kLog2N1, uint32_t kLog2N2>
hipError_t launch_wave_pass_t(const double2* in, double2* out, const double2* tables, uint32_t tw_off,
                              uint32_t lo_off, int post, hipStream_t stream) {
  constexpr uint32_t n = 1u << (kLog2N1 + kLog2N2);
  constexpr uint32_t log2l_1 = kLog2N1, log2l_2 = kLog2N2;
  static bool lds_raised = false;
  const uint32_t max_elems = kPassWaves * kWaveElems + 512 + 1024 + 1024;
  if (!lds_raised) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fft_wave_pass1_kernel<kLog2N1, kLog2N2>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)(max_elems * sizeof(double2)));
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(fft_wave_pass2_kernel<kLog2N1, kLog2N2>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)(max_elems * sizeof(double2)));
    if (e != hipSuccess) return e;
    lds_raised = true;
  }
  constexpr uint32_t hi_count = n / 1024;
  const size_t lds =
      (kPassWaves * kWaveElems + (1u << (post ? log2l_1 : log2l_2)) / 2 + (post ? 1024 + hi_count : 0)) *
      sizeof(double2);
  const dim3 grid(n / (kPassWaves * kWaveElems)), block(64 * kPassWaves);
  if (post)
    hipLaunchKernelGGL((fft_wave_pass1_kernel<kLog2N1, kLog2N2>), grid, block, lds, stream, in, out, tables, tw_off,
                       lo_off);
  else
    hipLaunchKernelGGL((fft_wave_pass2_kernel<kLog2N1, kLog2N2>), grid, block, lds, stream, in, out, tables, tw_off,
                       lo_off);
  return hipGetLastError();
}

hipError_t launch_wave_pass(const double2* in, double2* out, const double2* tables, uint32_t log2n1,
                            uint32_t log2n2, uint32_t tw_off, uint32_t lo_off, int post, hipStream_t stream) {
  // the split launch_fft64 makes: log2n1 = ceil(log2 n / 2), log2n2 = floor(log2 n / 2)
  switch (log2n1 * 16u + log2n2) {
    case 7u * 16u + 6u: return launch_wave_pass_t<7, 6>(in, out, tables, tw_off, lo_off, post, stream);
    case 7u * 16u + 7u: return launch_wave_pass_t<7, 7>(in, out, tables, tw_off, lo_off, post, stream);
    case 8u * 16u + 7u: return launch_wave_pass_t<8, 7>(in, out, tables, tw_off, lo_off, post, stream);
    case 8u * 16u + 8u: return launch_wave_pass_t<8, 8>(in, out, tables, tw_off, lo_off, post, stream);
    case 9u * 16u + 8u: return launch_wave_pass_t<9, 8>(in, out, tables, tw_off, lo_off, post, stream);
    case 9u * 16u + 9u: return launch_wave_pass_t<9, 9>(in, out, tables, tw_off, lo_off, post, stream);
    case 10u * 16u + 9u: return launch_wave_pass_t<10, 9>(in, out, tables, tw_off, lo_off, post, stream);
    case 10u * 16u + 10u: return launch_wave_pass_t<10, 10>(in, out, tables, tw_off, lo_off, post, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// Twiddles for length n (reactor_concept_fft.cpp:50-57 computes the same
// table on the host and caches it per length).  For n > 4096 the compact
// tables of the four-step passes follow the n/2 roots (fft_wave_pass_kernel):
// pass-1 stage twiddles (N1/2), pass-2 stage twiddles (N2/2), lo (1024), hi
// (n/1024), each entry copied from the roots (hi[h] = W_n^(1024 h), negated
// from roots[1024 h - n/2] past the half).  Caller holds ctx().mu.
const double2* fft64_roots(uint32_t n) {
  DeviceContext& c = ctx();
  if (c.fft_roots_n == n && c.fft_roots != nullptr) return static_cast<const double2*>(c.fft_roots);
  const uint32_t count = n / 2 > 0 ? n / 2 : 1;
  std::vector<double> host(2 * (size_t)count, 0.0);
  host[0] = 1.0;
  const double pi = 3.14159265358979323846;
  for (uint32_t j = 0; j < n / 2; ++j) {
    const double angle = -2.0 * pi / (double)n * (double)j;
    host[2 * j] = cos(angle);
    host[2 * j + 1] = sin(angle);
  }
  if (n > kFftMaxLds) {
    const uint32_t log2n = ilog2(n), n1 = 1u << ((log2n + 1) / 2), n2 = n / n1;
    auto push = [&](uint64_t idx) {  // W_n^idx, idx < n
      const bool neg = idx >= n / 2;
      const uint64_t r = neg ? idx - n / 2 : idx;
      host.push_back(neg ? -host[2 * r] : host[2 * r]);
      host.push_back(neg ? -host[2 * r + 1] : host[2 * r + 1]);
    };
    for (uint32_t j = 0; j < n1 / 2; ++j) push((uint64_t)j * n2);
    for (uint32_t j = 0; j < n2 / 2; ++j) push((uint64_t)j * n1);
    for (uint32_t j = 0; j < 1024; ++j) push(j);
    for (uint32_t h = 0; h < n / 1024; ++h) push((uint64_t)h * 1024);
  }
  void* dev = staging(7, host.size() * sizeof(double));
  if (dev == nullptr) return nullptr;
  if (hipMemcpyAsync(dev, host.data(), host.size() * sizeof(double), hipMemcpyHostToDevice, c.stream) != hipSuccess ||
      hipStreamSynchronize(c.stream) != hipSuccess) {
    (void)hipGetLastError();
    c.fft_roots_n = 0;
    return nullptr;
  }
  c.fft_roots = dev;
  c.fft_roots_n = n;
  return static_cast<const double2*>(dev);
}

hipError_t launch_fft64(const double2* in, double2* out, double2* temp, const double2* roots, uint32_t n,
                        hipStream_t stream) {
  const uint32_t log2n = ilog2(n);
  if ((1u << log2n) != n || log2n > kFftMaxLog2) return hipErrorInvalidValue;
  if (n <= kFftMaxLds) return launch_pass(in, out, roots, n, log2n, 0, 0, 1, 0, 1, 0, 0, 0, stream);
  const uint32_t log2n1 = (log2n + 1) / 2, log2n2 = log2n - log2n1;
  const uint64_t n1 = 1ull << log2n1, n2 = 1ull << log2n2;
  const double2* tables = roots + n / 2;
  const uint32_t tw2_off = (uint32_t)(n1 / 2), lo_off = (uint32_t)(n1 / 2 + n2 / 2);
  // pass 1: N2 columns of length N1 (stride N2), twiddled, to T (tiled rows k1)
  hipError_t e = launch_wave_pass(in, temp, tables, log2n1, log2n2, 0, lo_off, 1, stream);
  if (e != hipSuccess) return e;
  // pass 2: N1 rows of length N2, to X[k1 + N1*k2]
  return launch_wave_pass(temp, out, tables, log2n1, log2n2, tw2_off, lo_off, 0, stream);
}

}  // namespace prom

using namespace prom;

namespace {

bool fft64_request_valid(const void* input, const void* output, uint32_t count) {
  return input != nullptr && output != nullptr && count != 0u && (count & (count - 1u)) == 0u &&
         count <= (1u << kFftMaxLog2);
}

}  // namespace

extern "C" {

PROM_REACTOR_API int prometheus_reactor_runtime_fft64(void* handle, const double* input, double* output,
                                                      uint32_t count, uint32_t* stage, int* detail) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    set_status(stage, detail, PROM_STAGE_INIT, PROM_INVALID_HANDLE);
    return PROM_INVALID_HANDLE;
  }
  if (!fft64_request_valid(input, output, count)) {
    set_status(stage, detail, PROM_STAGE_INIT, PROM_FFT_DETAIL_INVALID_REQUEST);
    return PROM_ERROR;
  }
  set_status(stage, detail, PROM_STAGE_INIT, PROM_FFT_DETAIL_VULKAN_UNAVAILABLE);
  if (!rt->available) return PROM_ERROR;
  rt->requests++;
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  const size_t bytes = (size_t)count * 2 * sizeof(double);
  const double2* roots = fft64_roots(count);
  double2* din = static_cast<double2*>(staging(0, bytes));
  double2* dout = static_cast<double2*>(staging(1, bytes));
  double2* dtmp = count > kFftMaxLds ? static_cast<double2*>(staging(3, bytes)) : nullptr;
  // Injected faults (reactor_api.h:131-166) in the order the reference's FFT
  // executor meets them (PrometheusFft.concept:135-176): allocation, upload,
  // dispatch (a command that fails to end or to be submitted is a dispatch
  // failure there), readback.  An injected failure writes no output.
  const uint32_t tf = rt->test_flags;
  if ((tf & PROM_TESTCFG_FAIL_BUFFER_ALLOC) != 0u || roots == nullptr || din == nullptr || dout == nullptr ||
      (count > kFftMaxLds && dtmp == nullptr)) {
    set_status(stage, detail, PROM_STAGE_INIT, PROM_FFT_DETAIL_ALLOCATION_FAILED);
    return PROM_ERROR;
  }
  if ((tf & PROM_TESTCFG_FAIL_UPLOAD) != 0u || upload_host(din, input, bytes, cx.stream) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipStreamSynchronize(cx.stream);
    set_status(stage, detail, PROM_STAGE_TRANSFER_IN, PROM_FFT_DETAIL_UPLOAD_FAILED);
    return PROM_ERROR;
  }
  if ((tf & (PROM_TESTCFG_FAIL_DISPATCH | PROM_TESTCFG_FAIL_COMMAND_END | PROM_TESTCFG_FAIL_QUEUE_SUBMIT)) != 0u ||
      launch_fft64(din, dout, dtmp, roots, count, cx.stream) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipStreamSynchronize(cx.stream);
    set_status(stage, detail, PROM_STAGE_SUBMIT, PROM_FFT_DETAIL_DISPATCH_FAILED);
    return PROM_ERROR;
  }
  if ((tf & PROM_TESTCFG_FAIL_DOWNLOAD) != 0u) {
    (void)hipStreamSynchronize(cx.stream);
    set_status(stage, detail, PROM_STAGE_TRANSFER_OUT, PROM_FFT_DETAIL_READBACK_FAILED);
    return PROM_ERROR;
  }
  if (download_host(output, dout, bytes, cx.stream) != hipSuccess ||
      hipStreamSynchronize(cx.stream) != hipSuccess) {
    (void)hipGetLastError();
    set_status(stage, detail, PROM_STAGE_TRANSFER_OUT, PROM_FFT_DETAIL_READBACK_FAILED);
    return PROM_ERROR;
  }
  rt->successes++;
  set_status(stage, detail, PROM_STAGE_TRANSFER_OUT, 0);
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_fft64_device(void* handle, const double* input, double* output,
                                                             uint32_t count, uint32_t* stage, int* detail) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    set_status(stage, detail, PROM_STAGE_INIT, PROM_INVALID_HANDLE);
    return PROM_INVALID_HANDLE;
  }
  if (!fft64_request_valid(input, output, count)) {
    set_status(stage, detail, PROM_STAGE_INIT, PROM_FFT_DETAIL_INVALID_REQUEST);
    return PROM_ERROR;
  }
  set_status(stage, detail, PROM_STAGE_INIT, PROM_FFT_DETAIL_VULKAN_UNAVAILABLE);
  if (!rt->available) return PROM_ERROR;
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  const double2* roots = fft64_roots(count);
  double2* dtmp = count > kFftMaxLds ? static_cast<double2*>(staging(3, (size_t)count * sizeof(double2))) : nullptr;
  if (roots == nullptr || (count > kFftMaxLds && dtmp == nullptr)) {
    set_status(stage, detail, PROM_STAGE_INIT, PROM_FFT_DETAIL_ALLOCATION_FAILED);
    return PROM_ERROR;
  }
  if (launch_fft64(reinterpret_cast<const double2*>(input), reinterpret_cast<double2*>(output), dtmp, roots, count,
                   cx.stream) != hipSuccess) {
    (void)hipGetLastError();
    set_status(stage, detail, PROM_STAGE_SUBMIT, PROM_FFT_DETAIL_DISPATCH_FAILED);
    return PROM_ERROR;
  }
  set_status(stage, detail, PROM_STAGE_SUBMIT, 0);
  return PROM_OK;
}

}  // extern "C"
