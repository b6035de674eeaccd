// Batched complex-fp32 FFT (prometheus_reactor_runtime_fft and its
// benchmark-variant and diagnostics entries).
//
// Contract: reactor_vulkan_fft.c:59-128 (validation order and details, the
// radix-2 plan the diagnostics report), PrometheusFft.concept:98-176 (bit
// reversal, then log2(N) radix-2 passes; the inverse is scaled by 1/N on the
// final pass whether or not INVERSE_NORMALIZE is set; only element_count
// values per batch are written back, so padding between batches survives)
// and radix2_butterfly.sdslv:24-58 (DIT butterfly, twiddle exp(-+2*pi*i*j/span)
// for forward / inverse).
//
// MI355X design.  Lengths L <= 4096 run as one launch: a workgroup holds
// `seqs` whole sequences (batches) in LDS (L * seqs <= 4096 complex values,
// 32 KiB), loads them in bit-reversed order, runs the log2(L) stages two per
// barrier and stores them, scaling on the way out.  Longer lengths use the
// four-step factorisation N = N1 * N2 (N1, N2 <= 1024) in two launches per
// call, every batch in the grid's y dimension: pass 1 transforms the N2
// columns (stride N2) and multiplies by W_N^(n2*k1) into a scratch T, pass 2
// the N1 rows of T into X[k1 + N1*k2].  Twiddles are exact-argument
// sincospi values (the fraction 2j/L is exact in fp32 for L <= 2^20), so no
// table is built or cached; FMA contraction is allowed (no bit-exactness
// contract exists for the fp32 route; agreement with a binary64 DFT is the
// acceptance test, as in reactor_fft_api_tests.cpp:525-589).
#include <math.h>
#include <string.h>

#include "reactor_internal.h"

namespace prom {

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kMaxLds = 4096;                       // complex values per workgroup
constexpr uint32_t kPerThread = kMaxLds / kThreads;      // values each thread loads and stores
constexpr uint32_t kMaxLog2 = 20;
constexpr uint64_t kMaxElements = 65535ull * 256ull;     // element_count * batch_count
constexpr uint32_t kDirForward = 1u, kDirInverse = 2u;

__device__ __forceinline__ float2 cmul(float2 w, float2 v) {
  return make_float2(w.x * v.x - w.y * v.y, w.x * v.y + w.y * v.x);
}

// exp(sign * 2*pi*i * num / den) for den a power of two (num / den exact).
__device__ __forceinline__ float2 root(float sign, uint32_t num, uint32_t den) {
  float s, c;
  sincospif(sign * 2.0f * ((float)num / (float)den), &s, &c);
  return make_float2(c, s);
}

// One workgroup transforms `seqs` = 2^log2seqs sequences of length L = 2^log2l:
// sequence q = blockIdx.x * seqs + s (< nseq) of slice blockIdx.y reads
// element i at in[y * in_batch + q * in_seq + i * in_elem] and writes element
// k at out[y * out_batch + q * out_seq + k * out_elem].  With post set, output
// k of sequence q is multiplied by W_N^(q*k) (N = 2^log2n); every output is
// multiplied by scale.  seq_fast_in / seq_fast_out put adjacent threads on
// adjacent sequences (when those are adjacent in memory).
__global__ __launch_bounds__(kThreads) void fft32_lds_kernel(const float2* __restrict__ in, float2* __restrict__ out,
                                                             uint32_t log2l, uint32_t log2seqs, uint32_t nseq,
                                                             uint64_t in_batch, uint64_t in_seq, uint64_t in_elem,
                                                             uint64_t out_batch, uint64_t out_seq, uint64_t out_elem,
                                                             uint32_t log2n, int post, float sign, float scale,
                                                             int seq_fast_in, int seq_fast_out) {
  extern __shared__ float2 lds32[];
  const uint32_t L = 1u << log2l;
  const uint32_t seqs = 1u << log2seqs;
  const uint32_t total = L << log2seqs;
  float2* buf = lds32;
  float2* tw = lds32 + total;
  for (uint32_t j = threadIdx.x; j < (L >> 1); j += blockDim.x) tw[j] = root(sign, j, L);
  uint32_t blk = blockIdx.x;  // XCD-contiguous ranges of sequences, as the fp64 kernels
  if ((gridDim.x & 7u) == 0u) blk = (blk & 7u) * (gridDim.x >> 3) + (blk >> 3);
  const uint64_t q0 = (uint64_t)blk << log2seqs;
  const float2* src = in + (uint64_t)blockIdx.y * in_batch;
  float2* dst = out + (uint64_t)blockIdx.y * out_batch;
  float2 v[kPerThread];
#pragma unroll
  for (uint32_t u = 0; u < kPerThread; ++u) {
    const uint32_t e = threadIdx.x + u * kThreads;
    v[u] = make_float2(0.0f, 0.0f);
    if (e < total) {
      const uint32_t s = seq_fast_in ? (e & (seqs - 1)) : (e >> log2l);
      const uint32_t i = seq_fast_in ? (e >> log2seqs) : (e & (L - 1));
      if (q0 + s < nseq) v[u] = src[(q0 + s) * in_seq + (uint64_t)i * in_elem];
    }
  }
#pragma unroll
  for (uint32_t u = 0; u < kPerThread; ++u) {
    const uint32_t e = threadIdx.x + u * kThreads;
    if (e < total) {
      const uint32_t s = seq_fast_in ? (e & (seqs - 1)) : (e >> log2l);
      const uint32_t i = seq_fast_in ? (e >> log2seqs) : (e & (L - 1));
      const uint32_t r = log2l == 0 ? 0u : (__brev(i) >> (32u - log2l));
      buf[(s << log2l) + r] = v[u];
    }
  }
  __syncthreads();
  uint32_t lg = 1;
  for (; lg + 1 <= log2l; lg += 2) {  // stages lg and lg + 1 per barrier
    const uint32_t h = 1u << (lg - 1);
    for (uint32_t g = threadIdx.x; g < (total >> 2); g += blockDim.x) {
      const uint32_t s = g >> (log2l - 2);
      const uint32_t gg = g & ((L >> 2) - 1);
      const uint32_t j = gg & (h - 1);
      const uint32_t p = (s << log2l) + ((gg >> (lg - 1)) << (lg + 1)) + j;
      const float2 a0 = buf[p], a1 = buf[p + h], a2 = buf[p + 2 * h], a3 = buf[p + 3 * h];
      const float2 w1 = tw[j << (log2l - lg)];
      float2 t = cmul(w1, a1);
      const float2 b0 = make_float2(a0.x + t.x, a0.y + t.y), b1 = make_float2(a0.x - t.x, a0.y - t.y);
      t = cmul(w1, a3);
      const float2 b2 = make_float2(a2.x + t.x, a2.y + t.y), b3 = make_float2(a2.x - t.x, a2.y - t.y);
      t = cmul(tw[j << (log2l - lg - 1)], b2);
      buf[p] = make_float2(b0.x + t.x, b0.y + t.y);
      buf[p + 2 * h] = make_float2(b0.x - t.x, b0.y - t.y);
      t = cmul(tw[(j + h) << (log2l - lg - 1)], b3);
      buf[p + h] = make_float2(b1.x + t.x, b1.y + t.y);
      buf[p + 3 * h] = make_float2(b1.x - t.x, b1.y - t.y);
    }
    __syncthreads();
  }
  if (lg == log2l) {  // an odd stage count leaves the last stage (span L)
    const uint32_t half = L >> 1;
    for (uint32_t b = threadIdx.x; b < (total >> 1); b += blockDim.x) {
      const uint32_t p = ((b >> (log2l - 1)) << log2l) + (b & (half - 1));
      const float2 t = cmul(tw[b & (half - 1)], buf[p + half]);
      const float2 a = buf[p];
      buf[p] = make_float2(a.x + t.x, a.y + t.y);
      buf[p + half] = make_float2(a.x - t.x, a.y - t.y);
    }
    __syncthreads();
  }
  const uint32_t n = 1u << log2n;
#pragma unroll
  for (uint32_t u = 0; u < kPerThread; ++u) {
    const uint32_t e = threadIdx.x + u * kThreads;
    if (e < total) {
      const uint32_t s = seq_fast_out ? (e & (seqs - 1)) : (e >> log2l);
      const uint32_t k = seq_fast_out ? (e >> log2seqs) : (e & (L - 1));
      if (q0 + s < nseq) {
        float2 r = buf[(s << log2l) + k];
        if (post) r = cmul(root(sign, (uint32_t)((q0 + s) * k) & (n - 1), n), r);  // (q0 + s) * k < N
        dst[(q0 + s) * out_seq + (uint64_t)k * out_elem] = make_float2(r.x * scale, r.y * scale);
      }
    }
  }
}

uint32_t ilog2(uint32_t v) {
  uint32_t r = 0;
  while ((1u << r) < v) ++r;
  return r;
}

// Sequences per workgroup: as many as keep >= 512 workgroups in the grid,
// within the LDS budget.
uint32_t pick_log2seqs(uint32_t log2l, uint32_t nseq, uint32_t slices) {
  uint32_t best = 0;
  while (((1u << (best + 1)) << log2l) <= kMaxLds &&
         (uint64_t)((nseq + (2u << best) - 1) >> (best + 1)) * slices >= 512u)
    ++best;
  return best;
}

hipError_t launch_pass(const float2* in, float2* out, uint32_t log2l, uint32_t nseq, uint32_t slices,
                       uint64_t in_batch, uint64_t in_seq, uint64_t in_elem, uint64_t out_batch, uint64_t out_seq,
                       uint64_t out_elem, uint32_t log2n, int post, float sign, float scale, int fast_in,
                       int fast_out, hipStream_t stream) {
  const uint32_t log2seqs = pick_log2seqs(log2l, nseq, slices);
  const uint32_t blocks = (nseq + (1u << log2seqs) - 1) >> log2seqs;
  const size_t lds = (((size_t)1 << (log2l + log2seqs)) + ((size_t)1 << log2l) / 2) * sizeof(float2);
  hipLaunchKernelGGL(fft32_lds_kernel, dim3(blocks, slices), dim3(kThreads), lds, stream, in, out, log2l, log2seqs,
                     nseq, in_batch, in_seq, in_elem, out_batch, out_seq, out_elem, log2n, post, sign, scale, fast_in,
                     fast_out);
  return hipGetLastError();
}

}  // namespace

// x (batch b at x + b * stride) -> y (same layout); temp holds batch * n values
// when n > 4096.  Device pointers; stream-ordered.
hipError_t launch_fft32(const float2* x, float2* y, float2* temp, uint32_t n, uint32_t batch, uint32_t stride,
                        bool inverse, hipStream_t stream) {
  const uint32_t log2n = ilog2(n);
  if ((1u << log2n) != n || log2n > kMaxLog2 || batch == 0 || batch > 65535u * 256u || stride < n)
    return hipErrorInvalidValue;
  const float sign = inverse ? 1.0f : -1.0f;
  const float scale = inverse ? 1.0f / (float)n : 1.0f;
  if (n <= kMaxLds)
    return launch_pass(x, y, log2n, batch, 1, 0, stride, 1, 0, stride, 1, log2n, 0, sign, scale, 0, 0, stream);
  if (batch > 65535u || temp == nullptr) return hipErrorInvalidValue;
  const uint32_t log2n1 = (log2n + 1) / 2, log2n2 = log2n - log2n1;
  const uint64_t n1 = 1ull << log2n1, n2 = 1ull << log2n2;
  // pass 1: N2 columns of length N1 (stride N2), twiddled, to T[b*N + k1*N2 + n2]
  hipError_t e = launch_pass(x, temp, log2n1, (uint32_t)n2, batch, stride, 1, n2, n, 1, n2, log2n, 1, sign, 1.0f, 1,
                             1, stream);
  if (e != hipSuccess) return e;
  // pass 2: N1 rows of length N2 (contiguous), to X[b*stride + k1 + N1*k2]
  return launch_pass(temp, y, log2n2, (uint32_t)n1, batch, n, n2, 1, stride, 1, n1, log2n, 0, sign, scale, 0, 1,
                     stream);
}

}  // namespace prom

using namespace prom;

namespace {

PrometheusFftDiagnostics default_diag() {
  PrometheusFftDiagnostics d;
  memset(&d, 0, sizeof(d));
  d.struct_size = (uint32_t)sizeof(d);
  d.api_declared = 1u;
  d.last_failure_detail = PROM_FFT_DETAIL_UNAVAILABLE;
  d.last_validation_status = PROM_FFT_PATH_STATUS_UNAVAILABLE;
  d.executed_path_id = PROM_FFT_PATH_UNAVAILABLE;
  return d;
}

PrometheusFftDiagnostics* diag_of(Runtime* rt) {
  if (rt->fft_diag.struct_size == 0) rt->fft_diag = default_diag();
  return &rt->fft_diag;
}

// reactor_vulkan_fft.c:59-80, in its order.
int32_t validate(const PrometheusFftRequest* r, uint32_t* direction, uint64_t* physical) {
  if (r == nullptr || r->struct_size < sizeof(*r)) return PROM_FFT_DETAIL_INVALID_REQUEST;
  if (r->input == nullptr) return PROM_FFT_DETAIL_NULL_INPUT;
  if (r->output == nullptr) return PROM_FFT_DETAIL_NULL_OUTPUT;
  if (r->element_count == 0u) return PROM_FFT_DETAIL_ZERO_ELEMENT_COUNT;
  if ((r->element_count & (r->element_count - 1u)) != 0u) return PROM_FFT_DETAIL_NON_POWER_OF_TWO;
  if (r->element_count > (1u << kMaxLog2)) return PROM_FFT_DETAIL_UNSUPPORTED_SIZE;
  if (r->batch_count == 0u) return PROM_FFT_DETAIL_ZERO_BATCH_COUNT;
  if ((r->flags & PROM_FFT_FLAG_FORWARD) && (r->flags & PROM_FFT_FLAG_INVERSE))
    return PROM_FFT_DETAIL_INVALID_DIRECTION_FLAGS;
  if ((r->flags & PROM_FFT_FLAG_INVERSE_NORMALIZE) && !(r->flags & PROM_FFT_FLAG_INVERSE))
    return PROM_FFT_DETAIL_INVERSE_NORMALIZE_REQUIRES_INVERSE;
  if (r->stride_elements != 0u && r->stride_elements < r->element_count) return PROM_FFT_DETAIL_INVALID_STRIDE;
  if (r->stride_elements != 0u && r->batch_count > UINT32_MAX / r->stride_elements) return PROM_FFT_DETAIL_SIZE_OVERFLOW;
  const uint32_t stride = r->stride_elements == 0u ? r->element_count : r->stride_elements;
  *physical = (uint64_t)(r->batch_count - 1u) * stride + r->element_count;
  if (*physical * sizeof(PrometheusComplex32) > UINT32_MAX) return PROM_FFT_DETAIL_SIZE_OVERFLOW;
  if ((uint64_t)r->element_count * r->batch_count > kMaxElements) return PROM_FFT_DETAIL_UNSUPPORTED_SIZE;
  *direction = (r->flags & PROM_FFT_FLAG_INVERSE) ? kDirInverse : kDirForward;
  return 0;
}

// The radix-2 plan the reference reports (reactor_vulkan_fft.c:82-101): log2(N)
// passes of spans 2 .. N ping-ponging after the bit reversal.
void record_plan(PrometheusFftDiagnostics* d, uint32_t n, uint32_t direction) {
  const uint32_t passes = ilog2(n);
  d->plan_valid = 1u;
  d->plan_element_count = n;
  d->plan_log2_element_count = passes;
  d->plan_pass_count = passes;
  d->ping_pong_swap_count = passes;
  d->final_output_role = passes == 0 ? 2u : ((passes & 1u) ? 3u : 2u);  // ping 2, pong 3
  d->plan_first_span = passes ? 2u : 0u;
  d->plan_last_span = passes ? n : 0u;
  d->plan_radix_mask = passes ? (1u << 2) : 0u;
  d->plan_bit_reversal_required = n > 1u ? 1u : 0u;
  d->plan_first_source_role = passes ? 2u : 1u;
  d->plan_first_destination_role = passes ? 3u : 2u;
  d->plan_direction = direction;
  d->plan_twiddle_mode = 2u;
}

// Caller holds ctx().mu (the diagnostics record and the staging buffers).
int run_fft(Runtime* rt, const PrometheusFftRequest* r, uint32_t* stage, int* detail) {
  PrometheusFftDiagnostics* d = diag_of(rt);
  *d = default_diag();
  if (r != nullptr) {
    d->last_element_count = r->element_count;
    d->last_batch_count = r->batch_count;
    d->last_stride_elements = r->stride_elements;
    d->last_flags = r->flags;
    d->last_effective_stride_elements = r->stride_elements == 0u ? r->element_count : r->stride_elements;
  }
  uint32_t direction = kDirForward;
  uint64_t physical = 0;
  const int32_t invalid = validate(r, &direction, &physical);
  d->last_direction = direction;
  if (invalid != 0) {
    d->last_failure_detail = invalid;
    set_status(stage, detail, PROM_STAGE_INIT, invalid);
    return PROM_ERROR;
  }
  record_plan(d, r->element_count, direction);
  d->requested_path_id = PROM_FFT_PATH_VULKAN_RADIX2_RESERVED;
  d->requested_radix = 2u;
  if (!rt->available) {
    d->last_failure_detail = PROM_FFT_DETAIL_VULKAN_UNAVAILABLE;
    set_status(stage, detail, PROM_STAGE_INIT, PROM_FFT_DETAIL_VULKAN_UNAVAILABLE);
    return PROM_ERROR;
  }
  d->capability_reported = 1u;
  d->production_enabled = 1u;
  d->benchmark_enabled = 1u;
  d->last_validation_status = PROM_FFT_PATH_STATUS_BENCHMARK_ENABLED;
  auto fail = [&](uint32_t st, int32_t code) {
    (void)hipGetLastError();
    d->executed_path_id = PROM_FFT_PATH_UNAVAILABLE;
    d->last_failure_detail = code;
    set_status(stage, detail, st, code);
    return PROM_ERROR;
  };
  rt->requests++;
  const uint32_t n = r->element_count, batch = r->batch_count;
  const uint32_t stride = r->stride_elements == 0u ? n : r->stride_elements;
  const size_t bytes = (size_t)physical * sizeof(float2);
  DeviceContext& cx = ctx();
  float2* din = static_cast<float2*>(staging(0, bytes));
  float2* dout = static_cast<float2*>(staging(1, bytes));
  float2* dtmp = n > kMaxLds ? static_cast<float2*>(staging(3, (size_t)n * batch * sizeof(float2))) : nullptr;
  if ((rt->test_flags & PROM_TESTCFG_FAIL_BUFFER_ALLOC) != 0u || din == nullptr || dout == nullptr ||
      (n > kMaxLds && dtmp == nullptr))
    return fail(PROM_STAGE_INIT, PROM_FFT_DETAIL_ALLOCATION_FAILED);
  if ((rt->test_flags & PROM_TESTCFG_FAIL_UPLOAD) != 0u ||
      hipMemcpyAsync(din, r->input, bytes, hipMemcpyHostToDevice, cx.stream) != hipSuccess)
    return fail(PROM_STAGE_TRANSFER_IN, PROM_FFT_DETAIL_UPLOAD_FAILED);
  if ((rt->test_flags & PROM_TESTCFG_FAIL_DISPATCH) != 0u ||
      launch_fft32(din, dout, dtmp, n, batch, stride, direction == kDirInverse, cx.stream) != hipSuccess) {
    (void)hipStreamSynchronize(cx.stream);
    return fail(PROM_STAGE_SUBMIT, PROM_FFT_DETAIL_DISPATCH_FAILED);
  }
  // element_count values per batch; the caller's padding is not written
  if ((rt->test_flags & PROM_TESTCFG_FAIL_DOWNLOAD) != 0u ||
      hipMemcpy2DAsync(r->output, (size_t)stride * sizeof(float2), dout, (size_t)stride * sizeof(float2),
                       (size_t)n * sizeof(float2), batch, hipMemcpyDeviceToHost, cx.stream) != hipSuccess ||
      hipStreamSynchronize(cx.stream) != hipSuccess) {
    (void)hipStreamSynchronize(cx.stream);
    return fail(PROM_STAGE_TRANSFER_OUT, PROM_FFT_DETAIL_READBACK_FAILED);
  }
  rt->successes++;
  d->executed_path_id = PROM_FFT_PATH_VULKAN_RADIX2_RESERVED;
  d->executed_radix = 2u;
  d->last_failure_detail = 0;
  set_status(stage, detail, PROM_STAGE_TRANSFER_OUT, 0);
  return PROM_OK;
}

}  // namespace

extern "C" {

PROM_REACTOR_API int prometheus_reactor_runtime_fft(void* handle, const PrometheusFftRequest* request,
                                                    uint32_t* out_stage, int* out_detail_code) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_INVALID_HANDLE);
    return PROM_INVALID_HANDLE;
  }
  std::lock_guard<std::mutex> lock(ctx().mu);
  return run_fft(rt, request, out_stage, out_detail_code);
}

PROM_REACTOR_API int prometheus_reactor_runtime_fft_benchmark_variant(void* handle,
                                                                      const PrometheusFftRequest* request,
                                                                      uint32_t requested_variant, uint32_t* out_stage,
                                                                      int* out_detail_code) {
  if (requested_variant != PROM_FFT_BENCHMARK_VARIANT_RADIX2) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_FFT_DETAIL_PLAN_DISPATCH_DISAGREEMENT);
    return PROM_ERROR;
  }
  return prometheus_reactor_runtime_fft(handle, request, out_stage, out_detail_code);
}

PROM_REACTOR_API int prometheus_reactor_runtime_fft_diagnostics_sized(void* handle, PrometheusFftDiagnostics* out_diag,
                                                                      uint32_t out_size) {
  if (out_diag == nullptr || out_size == 0u) return PROM_ERROR;
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  if (out_size > sizeof(*out_diag)) out_size = (uint32_t)sizeof(*out_diag);
  std::lock_guard<std::mutex> lock(ctx().mu);
  memset(out_diag, 0, out_size);
  memcpy(out_diag, diag_of(rt), out_size);
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_fft_diagnostics(void* handle, PrometheusFftDiagnostics* out_diag) {
  return prometheus_reactor_runtime_fft_diagnostics_sized(handle, out_diag, (uint32_t)sizeof(*out_diag));
}

}  // extern "C"
