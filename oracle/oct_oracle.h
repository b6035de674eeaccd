/*
 * oct_oracle.h -- CPU restatement of Oct's Prometheus hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * reactor in oct_amd/.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path never links or calls it.
 *
 * Each function names the reference file:line whose behaviour it restates.
 * Pinning (what checks each function against known answers) is listed in the
 * header comment of oct_oracle.c.
 */
#ifndef OCT_ORACLE_H
#define OCT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded synthetic generators (SplitMix64 -> xoshiro256**) ---------- */
void oct_gen_uniform_f32(uint64_t seed, float* out, uint64_t count, float lo, float hi);
void oct_gen_normal_f32(uint64_t seed, float* out, uint64_t count, float mean, float stddev);
/* internal/prometheus/runtime.go:242-249 and Marionette/reactor_stub_tests.cpp:50-58 */
void oct_deterministic_matrix(float* out, uint64_t count);
/* Marionette/reactor_concept_sgemm_tests.cpp:17-21 */
void oct_concept_sgemm_matrix(float* out, uint32_t count, uint32_t seed);
/* Marionette/reactor_reduction_tests.cpp:78-87 */
void oct_reduction_deterministic_input(float* out, uint32_t rows, uint32_t width, float bias);
/* internal/prometheus/gemma4e2b_m1_rtx.go:1005-1014 */
uint16_t oct_f32_to_bf16(float value);
float oct_bf16_to_f32(uint16_t bits);
void oct_f32_to_bf16_array(const float* in, uint16_t* out, uint64_t count);
void oct_bf16_to_f32_array(const uint16_t* in, float* out, uint64_t count);

/* ---- Oct `@` ------------------------------------------------------------ */
/* internal/interpret/interpret.go:6278-6305: acc = a[r,0]*b[0,c], then
   acc = acc + a[r,k]*b[k,c] for k = 1..K-1, binary64, multiply then add.
   Rows are split across `threads`; each element's operation order is the
   sequential one, so the result is bit-identical for any thread count.
   row_begin/row_end restrict the computed rows (c is indexed by absolute row). */
void oct_matmul_f64(const double* a, const double* b, double* c,
                    uint32_t m, uint32_t n, uint32_t k,
                    uint32_t row_begin, uint32_t row_end, uint32_t threads);
/* The Prometheus strict path first rounds operands to fp32
   (internal/prometheus/runtime.go:298-306); this is oct_matmul_f64 on those
   fp32 operands widened back to binary64. */
void oct_matmul_f32in_f64(const float* a, const float* b, double* c,
                          uint32_t m, uint32_t n, uint32_t k,
                          uint32_t row_begin, uint32_t row_end, uint32_t threads);
/* Same loop on bf16 operands (widened exactly to binary64). */
void oct_matmul_bf16in_f64(const uint16_t* a, const uint16_t* b, double* c,
                           uint32_t m, uint32_t n, uint32_t k,
                           uint32_t row_begin, uint32_t row_end, uint32_t threads);
/* internal/build/emit_go_runtime.go:168-205 (__octMatMulMM): ijk, acc from 0,
   B walked column-strided, single thread.  Used as the timed CPU baseline. */
void oct_matmul_compiled_f64(const double* a, const double* b, double* c,
                             uint32_t m, uint32_t n, uint32_t k,
                             uint32_t row_begin, uint32_t row_end);
/* internal/prometheus/runtime.go:319-331 (cpuSGEMM): float32 sequential k. */
void oct_cpu_sgemm_f32(const float* a, const float* b, float* c,
                       uint32_t m, uint32_t n, uint32_t k);

typedef struct OctCorrectness {
  int32_t pass;
  int32_t failing_count;
  int64_t first_failing_index;
  double max_abs_error;
  double max_rel_error;
  float first_expected;
  float first_actual;
} OctCorrectness;
/* internal/prometheus/runtime.go:339-376 (compareAgainstOracle) with the
   abs 1e-4 / rel 1e-4 tolerances of runtime.go:12-15. */
void oct_compare_against_oracle(const float* expected, const float* actual, uint64_t count,
                                OctCorrectness* out);
/* ||actual - expected||_F / ||expected||_F in binary64 (rows restricts to a
   row range of an m x n matrix when row_end > row_begin; else the full count). */
double oct_normwise_rel_err(const float* actual, const double* expected, uint64_t count);
double oct_normwise_rel_err_f32(const float* actual, const float* expected, uint64_t count);

/* ---- row reductions ----------------------------------------------------- */
/* native/reactor_vulkan_fused_reduction.c:996-1036 (prom_reduction_cpu_reference)
   operation 1 = sum (binary64 accumulate), 2 = max (float compare),
   3 = stable softmax (float max, binary64 sum of exp).  Returns 0 or a
   PROM_REDUCTION_DETAIL_* code (non-finite input -> -6814). */
int32_t oct_reduction_cpu_reference(const float* input, float* output, uint32_t rows,
                                    uint32_t width, uint32_t operation);
typedef struct OctReductionMismatch {
  uint32_t row;
  uint32_t column;
  float expected;
  float actual;
  float absolute_error;
  float relative_error;
} OctReductionMismatch;
/* native/reactor_vulkan_fused_reduction.c:1038-1114 (prom_reduction_compare):
   returns 0 on pass, 1 on mismatch (details in *out). */
int32_t oct_reduction_compare(uint32_t rows, uint32_t width, uint32_t operation,
                              const float* expected, const float* actual,
                              OctReductionMismatch* out);

/* native/reactor_vulkan_gemma4e2b.c:286-319 (prom_m46_rmsnorm_cpu_reference):
   float sum of squares left to right, inv = 1/sqrtf(sumsq/W + eps),
   y = z*inv*w.  Returns 0, or 1 on invalid/non-finite. */
int32_t oct_rmsnorm_cpu_reference(const float* z, const float* weight, float* y, float* inv_rms,
                                  uint32_t tokens, uint32_t width, uint32_t z_row_stride,
                                  float epsilon);

/* internal/fft/fft.go:218-226 (roots): n/2 interleaved (cos, sin) pairs. */
void oct_fft64_roots(double* twiddles, uint32_t n);
/* internal/fft/fft.go:228-258 (cpuWithRoots): interleaved complex binary64,
   forward, unnormalised; input and output may not overlap. */
void oct_fft64_with_roots(const double* input, double* output, const double* twiddles, uint32_t n);
/* roots + transform; scratch_twiddles holds n doubles.  Returns 1 on an
   invalid request (NULL, zero or non-power-of-two n). */
int32_t oct_fft64(const double* input, double* output, double* scratch_twiddles, uint32_t n);
/* internal/fft/fft.go:176-192 (agrees). */
int32_t oct_fft64_agrees(const double* reference, const double* actual, uint32_t n);
/* reactor_fft_api_tests.cpp:525-553: the direct binary64 DFT of `batch`
   complex-fp32 sequences of n points `stride` apart (inverse / n), rounded to
   fp32; the padding is copied from the input. */
void oct_dft_c32(const float* input, float* output, uint32_t n, uint32_t batch, uint32_t stride, int32_t inverse);

/* Gemma-4-E2B M1 stages (oct_oracle_m1.c). */
void oct_m1_rmsnorm(const float* input, uint32_t stride, const float* weight, float* output, float* inv_rms,
                    uint32_t rows, uint32_t width, float epsilon, int32_t round_in, int32_t round_out);
void oct_m1_head_rmsnorm_go(const float* input, const float* weight, float* output, uint32_t rows, uint32_t width,
                            float epsilon);
void oct_m1_rope(const float* source, const float* cosine, const float* sine, float* output, uint32_t tokens,
                 uint32_t heads, uint32_t width);
void oct_m1_raw_scores(const float* query, const float* key, float* scores, uint32_t tokens, uint32_t query_heads,
                       uint32_t width, float scale);

#ifdef __cplusplus
}
#endif
#endif
