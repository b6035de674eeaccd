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
//           multiplied by W_N^(n2*k1) on the way out and stored as T[k1*N2 + n2];
//   pass 2: for every row k1, an N2-point transform over T[k1*N2 + n2], stored
//           to X[k1 + N1*k2].
// Each workgroup takes several adjacent columns (rows) so that its strided
// loads and stores touch contiguous runs; the whole 16 MiB working set of a
// 2^20-point transform stays resident in the MI355X's 256 MiB Infinity Cache
// between the passes.
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

}  // namespace

// Twiddles for length n (reactor_concept_fft.cpp:50-57 computes the same
// table on the host and caches it per length).  Caller holds ctx().mu.
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
  // pass 1: N2 columns of length N1 (stride N2), twiddled, to T[k1*N2 + n2]
  hipError_t e = launch_pass(in, temp, roots, n, log2n1, log2n2, 1, n2, 1, n2, 1, 1, 1, stream);
  if (e != hipSuccess) return e;
  // pass 2: N1 rows of length N2 (contiguous), to X[k1 + N1*k2]
  return launch_pass(temp, out, roots, n, log2n2, log2n1, n2, 1, 1, n1, 0, 0, 1, stream);
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
  if (roots == nullptr || din == nullptr || dout == nullptr || (count > kFftMaxLds && dtmp == nullptr)) {
    set_status(stage, detail, PROM_STAGE_INIT, PROM_FFT_DETAIL_ALLOCATION_FAILED);
    return PROM_ERROR;
  }
  if (hipMemcpyAsync(din, input, bytes, hipMemcpyHostToDevice, cx.stream) != hipSuccess) {
    (void)hipGetLastError();
    set_status(stage, detail, PROM_STAGE_TRANSFER_IN, PROM_FFT_DETAIL_UPLOAD_FAILED);
    return PROM_ERROR;
  }
  if (launch_fft64(din, dout, dtmp, roots, count, cx.stream) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipStreamSynchronize(cx.stream);
    set_status(stage, detail, PROM_STAGE_SUBMIT, PROM_FFT_DETAIL_DISPATCH_FAILED);
    return PROM_ERROR;
  }
  if (hipMemcpyAsync(output, dout, bytes, hipMemcpyDeviceToHost, cx.stream) != hipSuccess ||
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
