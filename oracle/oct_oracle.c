/*
 * oct_oracle.c -- CPU restatement of Oct's Prometheus hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP reactor.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 * It is compiled with -ffp-contract=off so that every `a*b + c` below is a
 * rounded multiply followed by a rounded add, as Go's amd64 code generation
 * does for the reference loops (no FMA contraction at GOAMD64=v1).
 *
 * How each function is pinned (tests/test_oracle.py):
 *   oct_matmul_f64 / _f32in_f64 / _compiled_f64:
 *       KAT [[1,2],[3,4]]@[[5,6],[7,8]] = [[19,22],[43,50]]
 *       (internal/prometheus/runtime_test.go:180-203); a@a[0,0] = 7
 *       (Language/Prometheus/gpu/matrix.octest:3-9); exact rational
 *       products (fractions.Fraction) on the deterministic corpora of
 *       runtime.go:83-89 and reactor_stub_tests.cpp:205-253; identity,
 *       diagonal and rank-1 closed forms; transposition identity
 *       (A@B)^T = B^T@A^T; thread-count invariance (bit-identical).
 *   oct_cpu_sgemm_f32: numpy float32 sequential-k loop on tiny shapes;
 *       Marionette 1e-4 tolerance against the binary64 product.
 *   oct_reduction_cpu_reference: FusedReductionSemantics.sdslvtest:6-95 KATs,
 *       the captured attention row M5/attention_token0_head0.octagon
 *       (1024 logits, Oct binary64 expected values), softmax invariants.
 *   oct_rmsnorm_cpu_reference: the captured Q-norm row
 *       M4/qnorm_row0_head0.octagon (eps 1e-5, 2e-6), and the constant-row
 *       closed form w*c/sqrt(c^2+eps).
 *   oct_reduction_compare: planted mismatches (abs/rel thresholds, row sum).
 */
#include "oct_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* generators                                                               */
/* ------------------------------------------------------------------------ */

static uint64_t splitmix64_next(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

typedef struct xoshiro256 {
  uint64_t s[4];
} xoshiro256;

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static void xoshiro_seed(xoshiro256* g, uint64_t seed) {
  uint64_t sm = seed;
  for (int i = 0; i < 4; ++i) g->s[i] = splitmix64_next(&sm);
}

/* xoshiro256** (Blackman & Vigna 2018). */
static uint64_t xoshiro_next(xoshiro256* g) {
  uint64_t* s = g->s;
  const uint64_t result = rotl64(s[1] * 5u, 7) * 9u;
  const uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl64(s[3], 45);
  return result;
}

/* 53-bit uniform in [0,1). */
static double xoshiro_unit(xoshiro256* g) { return (double)(xoshiro_next(g) >> 11) * 0x1.0p-53; }

/* The stream is cut into blocks of 2^20 values; block b draws from xoshiro256**
   seeded with seed ^ (b * 0x9E3779B97F4A7C15).  Blocks are generated in
   parallel, and the values do not depend on the thread count. */
#define OCT_GEN_BLOCK (1ull << 20)

typedef struct gen_job {
  uint64_t seed;
  float* out;
  uint64_t count;
  float a, b;  /* uniform: lo, hi; normal: mean, stddev */
  int normal;
  uint64_t first_block, block_stride;
} gen_job;

static void gen_block(const gen_job* j, uint64_t blk) {
  xoshiro256 g;
  xoshiro_seed(&g, j->seed ^ (blk * 0x9E3779B97F4A7C15ull));
  const uint64_t begin = blk * OCT_GEN_BLOCK;
  uint64_t end = begin + OCT_GEN_BLOCK;
  if (end > j->count) end = j->count;
  if (!j->normal) {
    const double span = (double)j->b - (double)j->a;
    for (uint64_t i = begin; i < end; ++i) j->out[i] = (float)((double)j->a + xoshiro_unit(&g) * span);
    return;
  }
  const double two_pi = 6.283185307179586476925286766559;
  uint64_t i = begin;
  while (i < end) {
    /* Box-Muller on (0,1] x [0,1). */
    const double u1 = 1.0 - xoshiro_unit(&g);
    const double u2 = xoshiro_unit(&g);
    const double r = sqrt(-2.0 * log(u1));
    j->out[i++] = (float)((double)j->a + (double)j->b * r * cos(two_pi * u2));
    if (i < end) j->out[i++] = (float)((double)j->a + (double)j->b * r * sin(two_pi * u2));
  }
}

static void* gen_worker(void* raw) {
  const gen_job* j = (const gen_job*)raw;
  const uint64_t blocks = (j->count + OCT_GEN_BLOCK - 1) / OCT_GEN_BLOCK;
  for (uint64_t b = j->first_block; b < blocks; b += j->block_stride) gen_block(j, b);
  return NULL;
}

static void gen_dispatch(uint64_t seed, float* out, uint64_t count, float a, float b, int normal) {
  const uint64_t blocks = (count + OCT_GEN_BLOCK - 1) / OCT_GEN_BLOCK;
  uint64_t threads = blocks < 16 ? blocks : 16;
  if (threads < 1) threads = 1;
  gen_job jobs[16];
  pthread_t tids[16];
  for (uint64_t t = 0; t < threads; ++t) {
    jobs[t].seed = seed;
    jobs[t].out = out;
    jobs[t].count = count;
    jobs[t].a = a;
    jobs[t].b = b;
    jobs[t].normal = normal;
    jobs[t].first_block = t;
    jobs[t].block_stride = threads;
  }
  if (threads == 1) {
    gen_worker(&jobs[0]);
    return;
  }
  for (uint64_t t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, gen_worker, &jobs[t]);
  for (uint64_t t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
}

void oct_gen_uniform_f32(uint64_t seed, float* out, uint64_t count, float lo, float hi) {
  gen_dispatch(seed, out, count, lo, hi, 0);
}

void oct_gen_normal_f32(uint64_t seed, float* out, uint64_t count, float mean, float stddev) {
  gen_dispatch(seed, out, count, mean, stddev, 1);
}

void oct_deterministic_matrix(float* out, uint64_t count) {
  for (uint64_t i = 0; i < count; ++i) {
    const int v = (int)(i % 23u) - 11;
    out[i] = (float)v / 7.0f;
  }
}

void oct_concept_sgemm_matrix(float* out, uint32_t count, uint32_t seed) {
  for (uint32_t i = 0; i < count; ++i) out[i] = (float)((int)((i * 7u + seed) % 23u) - 11) / 8.0f;
}

void oct_reduction_deterministic_input(float* out, uint32_t rows, uint32_t width, float bias) {
  for (uint32_t row = 0; row < rows; ++row) {
    for (uint32_t column = 0; column < width; ++column) {
      const int centered = (int)((row * 29u + column * 17u) % 101u) - 50;
      out[(uint64_t)row * width + column] = bias + (float)centered / 16.0f;
    }
  }
}

uint16_t oct_f32_to_bf16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof(bits));
  const uint32_t lsb = (bits >> 16) & 1u;
  const uint32_t rounded = bits + 0x7FFFu + lsb;
  return (uint16_t)(rounded >> 16);
}

float oct_bf16_to_f32(uint16_t bits) {
  const uint32_t wide = (uint32_t)bits << 16;
  float out;
  memcpy(&out, &wide, sizeof(out));
  return out;
}

void oct_f32_to_bf16_array(const float* in, uint16_t* out, uint64_t count) {
  for (uint64_t i = 0; i < count; ++i) out[i] = oct_f32_to_bf16(in[i]);
}

void oct_bf16_to_f32_array(const uint16_t* in, float* out, uint64_t count) {
  for (uint64_t i = 0; i < count; ++i) out[i] = oct_bf16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Oct `@` in binary64                                                      */
/* ------------------------------------------------------------------------ */

typedef enum { OPERAND_F64 = 0, OPERAND_F32 = 1, OPERAND_BF16 = 2 } operand_kind;

typedef struct matmul_job {
  const void* a;
  const void* b;
  double* c;
  uint32_t m, n, k;
  uint32_t row_begin, row_end;
  operand_kind kind;
} matmul_job;

static inline double load_operand(const void* base, uint64_t index, operand_kind kind) {
  switch (kind) {
    case OPERAND_F32: return (double)((const float*)base)[index];
    case OPERAND_BF16: return (double)oct_bf16_to_f32(((const uint16_t*)base)[index]);
    default: return ((const double*)base)[index];
  }
}

/* Row r of the interpreter's evalMatrixMultiply.  The loop is reordered to
   r-k-c so B is read contiguously, but every element still sees
   acc = a0*b0, then acc = acc + ak*bk for k = 1..K-1 in that order, each a
   separately rounded binary64 operation: bit-identical to the r-c-k loop. */
static void matmul_row(const matmul_job* job, uint32_t r, double* brow_scratch) {
  const uint32_t n = job->n, k = job->k;
  double* crow = job->c + (uint64_t)r * n;
  for (uint32_t kk = 0; kk < k; ++kk) {
    const double av = load_operand(job->a, (uint64_t)r * k + kk, job->kind);
    const double* brow;
    if (job->kind == OPERAND_F64) {
      brow = (const double*)job->b + (uint64_t)kk * n;
    } else {
      for (uint32_t c = 0; c < n; ++c) brow_scratch[c] = load_operand(job->b, (uint64_t)kk * n + c, job->kind);
      brow = brow_scratch;
    }
    if (kk == 0) {
      for (uint32_t c = 0; c < n; ++c) crow[c] = av * brow[c];
    } else {
      for (uint32_t c = 0; c < n; ++c) {
        const double term = av * brow[c];
        crow[c] = crow[c] + term;
      }
    }
  }
}

typedef struct matmul_thread_arg {
  const matmul_job* job;
  uint32_t first, stride;
} matmul_thread_arg;

static void* matmul_worker(void* raw) {
  matmul_thread_arg* arg = (matmul_thread_arg*)raw;
  const matmul_job* job = arg->job;
  double* scratch = NULL;
  if (job->kind != OPERAND_F64) scratch = (double*)malloc(sizeof(double) * (job->n ? job->n : 1));
  for (uint32_t r = job->row_begin + arg->first; r < job->row_end; r += arg->stride) matmul_row(job, r, scratch);
  free(scratch);
  return NULL;
}

static void matmul_dispatch(const matmul_job* job, uint32_t threads) {
  if (job->row_end <= job->row_begin || job->n == 0) return;
  if (job->k == 0) {
    /* Oct's interpreter yields the zero Value for an empty inner dimension. */
    for (uint32_t r = job->row_begin; r < job->row_end; ++r)
      memset(job->c + (uint64_t)r * job->n, 0, sizeof(double) * job->n);
    return;
  }
  if (threads < 1u) threads = 1u;
  if (threads > job->row_end - job->row_begin) threads = job->row_end - job->row_begin;
  if (threads > 256u) threads = 256u;
  pthread_t tids[256];
  matmul_thread_arg args[256];
  for (uint32_t t = 0; t < threads; ++t) {
    args[t].job = job;
    args[t].first = t;
    args[t].stride = threads;
  }
  if (threads == 1u) {
    matmul_worker(&args[0]);
    return;
  }
  for (uint32_t t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, matmul_worker, &args[t]);
  for (uint32_t t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
}

static void matmul_generic(const void* a, const void* b, double* c, uint32_t m, uint32_t n, uint32_t k,
                           uint32_t row_begin, uint32_t row_end, uint32_t threads, operand_kind kind) {
  matmul_job job;
  if (row_end == 0u || row_end > m) row_end = m;
  job.a = a;
  job.b = b;
  job.c = c;
  job.m = m;
  job.n = n;
  job.k = k;
  job.row_begin = row_begin;
  job.row_end = row_end;
  job.kind = kind;
  matmul_dispatch(&job, threads);
}

void oct_matmul_f64(const double* a, const double* b, double* c, uint32_t m, uint32_t n, uint32_t k,
                    uint32_t row_begin, uint32_t row_end, uint32_t threads) {
  matmul_generic(a, b, c, m, n, k, row_begin, row_end, threads, OPERAND_F64);
}

void oct_matmul_f32in_f64(const float* a, const float* b, double* c, uint32_t m, uint32_t n, uint32_t k,
                          uint32_t row_begin, uint32_t row_end, uint32_t threads) {
  matmul_generic(a, b, c, m, n, k, row_begin, row_end, threads, OPERAND_F32);
}

void oct_matmul_bf16in_f64(const uint16_t* a, const uint16_t* b, double* c, uint32_t m, uint32_t n, uint32_t k,
                           uint32_t row_begin, uint32_t row_end, uint32_t threads) {
  matmul_generic(a, b, c, m, n, k, row_begin, row_end, threads, OPERAND_BF16);
}

void oct_matmul_compiled_f64(const double* a, const double* b, double* c, uint32_t m, uint32_t n, uint32_t k,
                             uint32_t row_begin, uint32_t row_end) {
  if (row_end == 0u || row_end > m) row_end = m;
  for (uint32_t r = row_begin; r < row_end; ++r) {
    for (uint32_t col = 0; col < n; ++col) {
      double acc = 0.0;
      for (uint32_t kk = 0; kk < k; ++kk) {
        const double term = a[(uint64_t)r * k + kk] * b[(uint64_t)kk * n + col];
        acc = acc + term;
      }
      c[(uint64_t)r * n + col] = acc;
    }
  }
}

void oct_cpu_sgemm_f32(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k) {
  for (uint32_t row = 0; row < m; ++row) {
    for (uint32_t col = 0; col < n; ++col) {
      float sum = 0.0f;
      for (uint32_t kk = 0; kk < k; ++kk) {
        const float term = a[(uint64_t)row * k + kk] * b[(uint64_t)kk * n + col];
        sum = sum + term;
      }
      c[(uint64_t)row * n + col] = sum;
    }
  }
}

void oct_compare_against_oracle(const float* expected, const float* actual, uint64_t count, OctCorrectness* out) {
  const double abs_tol = 1e-4, rel_tol = 1e-4;
  memset(out, 0, sizeof(*out));
  out->pass = 1;
  out->first_failing_index = -1;
  for (uint64_t idx = 0; idx < count; ++idx) {
    const float e = expected[idx];
    const float a = actual[idx];
    if (!isfinite(e) || !isfinite(a)) {
      if (out->first_failing_index < 0) {
        out->first_failing_index = (int64_t)idx;
        out->first_expected = e;
        out->first_actual = a;
      }
      out->failing_count++;
      out->pass = 0;
      continue;
    }
    /* Go computes float64(e - a): the difference is a float32 subtraction. */
    const float diff = e - a;
    const double abs_err = fabs((double)diff);
    const double rel_err = e != 0.0f ? abs_err / fabs((double)e) : 0.0;
    if (abs_err > out->max_abs_error) out->max_abs_error = abs_err;
    if (rel_err > out->max_rel_error) out->max_rel_error = rel_err;
    if (abs_err > abs_tol && rel_err > rel_tol) {
      if (out->first_failing_index < 0) {
        out->first_failing_index = (int64_t)idx;
        out->first_expected = e;
        out->first_actual = a;
      }
      out->failing_count++;
      out->pass = 0;
    }
  }
}

double oct_normwise_rel_err(const float* actual, const double* expected, uint64_t count) {
  double num = 0.0, den = 0.0;
  for (uint64_t i = 0; i < count; ++i) {
    const double d = (double)actual[i] - expected[i];
    num += d * d;
    den += expected[i] * expected[i];
  }
  if (den == 0.0) return num == 0.0 ? 0.0 : INFINITY;
  return sqrt(num / den);
}

double oct_normwise_rel_err_f32(const float* actual, const float* expected, uint64_t count) {
  double num = 0.0, den = 0.0;
  for (uint64_t i = 0; i < count; ++i) {
    const double d = (double)actual[i] - (double)expected[i];
    num += d * d;
    den += (double)expected[i] * (double)expected[i];
  }
  if (den == 0.0) return num == 0.0 ? 0.0 : INFINITY;
  return sqrt(num / den);
}

/* ------------------------------------------------------------------------ */
/* reductions                                                               */
/* ------------------------------------------------------------------------ */

int32_t oct_reduction_cpu_reference(const float* input, float* output, uint32_t rows, uint32_t width,
                                    uint32_t operation) {
  if (input == NULL) return -6802;
  if (output == NULL) return -6803;
  if (rows == 0u) return -6804;
  if (width == 0u) return -6805;
  if (operation < 1u || operation > 3u) return -6806;
  const uint64_t total = (uint64_t)rows * width;
  for (uint64_t i = 0; i < total; ++i)
    if (!isfinite(input[i])) return -6814;
  for (uint32_t row = 0; row < rows; ++row) {
    const float* values = input + (uint64_t)row * width;
    if (operation == 1u) {
      double accumulator = 0.0;
      for (uint32_t column = 0; column < width; ++column) accumulator += (double)values[column];
      output[row] = (float)accumulator;
    } else if (operation == 2u) {
      float maximum = values[0];
      for (uint32_t column = 1; column < width; ++column)
        if (values[column] > maximum) maximum = values[column];
      output[row] = maximum;
    } else {
      float maximum = values[0];
      double denominator = 0.0;
      for (uint32_t column = 1; column < width; ++column)
        if (values[column] > maximum) maximum = values[column];
      for (uint32_t column = 0; column < width; ++column) denominator += exp((double)values[column] - maximum);
      for (uint32_t column = 0; column < width; ++column)
        output[(uint64_t)row * width + column] = (float)(exp((double)values[column] - maximum) / denominator);
    }
  }
  return 0;
}

static float reduction_relative_error(float expected, float actual) {
  float denominator = fabsf(expected);
  if (denominator < 1.0e-20f) denominator = 1.0f;
  return fabsf(actual - expected) / denominator;
}

int32_t oct_reduction_compare(uint32_t rows, uint32_t width, uint32_t operation, const float* expected,
                              const float* actual, OctReductionMismatch* out) {
  const int softmax = operation == 3u;
  const uint64_t count = softmax ? (uint64_t)rows * width : rows;
  const float abs_tol = softmax ? 2.0e-5f : (operation == 2u ? 0.0f : 2.0e-5f * (float)width);
  const float rel_tol = softmax ? 2.0e-4f : (operation == 2u ? 0.0f : 2.0e-5f);
  for (uint64_t i = 0; i < count; ++i) {
    const float abs_err = fabsf(actual[i] - expected[i]);
    const float rel_err = reduction_relative_error(expected[i], actual[i]);
    if (!isfinite(actual[i]) || (abs_err > abs_tol && rel_err > rel_tol)) {
      if (out != NULL) {
        out->row = softmax ? (uint32_t)(i / width) : (uint32_t)i;
        out->column = softmax ? (uint32_t)(i % width) : UINT32_MAX;
        out->expected = expected[i];
        out->actual = actual[i];
        out->absolute_error = abs_err;
        out->relative_error = rel_err;
      }
      return 1;
    }
  }
  if (softmax) {
    for (uint32_t row = 0; row < rows; ++row) {
      double row_sum = 0.0;
      for (uint32_t column = 0; column < width; ++column) {
        const float value = actual[(uint64_t)row * width + column];
        if (!isfinite(value) || value < -2.0e-7f) {
          if (out != NULL) {
            out->row = row;
            out->column = column;
            out->expected = 0.0f;
            out->actual = value;
            out->absolute_error = fabsf(value);
            out->relative_error = fabsf(value);
          }
          return 1;
        }
        row_sum += value;
      }
      if (fabs(row_sum - 1.0) > 3.0e-4) {
        if (out != NULL) {
          out->row = row;
          out->column = UINT32_MAX;
          out->expected = 1.0f;
          out->actual = (float)row_sum;
          out->absolute_error = (float)fabs(row_sum - 1.0);
          out->relative_error = out->absolute_error;
        }
        return 1;
      }
    }
  }
  return 0;
}

int32_t oct_rmsnorm_cpu_reference(const float* z, const float* weight, float* y, float* inv_rms, uint32_t tokens,
                                  uint32_t width, uint32_t z_row_stride, float epsilon) {
  if (z == NULL || weight == NULL || y == NULL || tokens == 0u || width == 0u || z_row_stride < width ||
      !isfinite(epsilon) || epsilon <= 0.0f)
    return 1;
  for (uint32_t token = 0; token < tokens; ++token) {
    float sumsq = 0.0f;
    const float* row = z + (uint64_t)token * z_row_stride;
    for (uint32_t column = 0; column < width; ++column) {
      if (!isfinite(row[column]) || !isfinite(weight[column])) return 1;
      const float sq = row[column] * row[column];
      sumsq = sumsq + sq;
    }
    const float inv = 1.0f / sqrtf(sumsq / (float)width + epsilon);
    if (!isfinite(sumsq) || !isfinite(inv)) return 1;
    if (inv_rms != NULL) inv_rms[token] = inv;
    for (uint32_t column = 0; column < width; ++column) {
      const float n = row[column] * inv * weight[column];
      if (!isfinite(n)) return 1;
      y[(uint64_t)token * width + column] = n;
    }
  }
  return 0;
}
