/* Command-line check of the C loader against a reactor library.
 *
 *   bridge_check open   [library]   open a runtime, print its caps or issue
 *   bridge_check strict [library]   strict.go's matmul of a 2x3 by a 3x2
 *   bridge_check run    [library]   the loader's whole call sequence with
 *                                   known answers (needs a GPU)
 *
 * With no library argument the loader's discovery applies
 * ($OCT_PROMETHEUS_REACTOR, then the reference's default paths).  Every
 * answer checked here is fixed by exact arithmetic or a closed form: small
 * integer operands make every fp32 product and partial sum exact whatever
 * the summation order; an impulse transforms to all ones; a complex
 * exponential e^(2 pi i f j / N) transforms to N at bin f and zero elsewhere;
 * a constant row c normalises to w * c / sqrt(c^2 + eps).
 *
 * Exit status: 0 success, 1 a check failed, 3 the loader reported an issue.
 */
#define _GNU_SOURCE
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "prom_bridge.h"

static int failures = 0;

static void report(const char* name, int ok, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
static void report(const char* name, int ok, const char* fmt, ...) {
  char msg[256] = "";
  if (fmt) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof(msg), fmt, ap);
    va_end(ap);
  }
  printf("%s %s%s%s\n", ok ? "ok" : "FAIL", name, msg[0] ? " " : "", msg);
  fflush(stdout);
  if (!ok) ++failures;
}

/* Integers in [-4, 4] from a fixed LCG. */
static void small_ints(float* x, size_t n, uint32_t seed) {
  uint32_t s = seed;
  for (size_t i = 0; i < n; ++i) {
    s = s * 1664525u + 1013904223u;
    x[i] = (float)((int)((s >> 16) % 9u) - 4);
  }
}

/* Exact product of integer-valued matrices in int64. */
static void int_matmul(const float* a, const float* b, float* c, uint32_t m, uint32_t n, uint32_t k) {
  for (uint32_t i = 0; i < m; ++i)
    for (uint32_t j = 0; j < n; ++j) {
      int64_t acc = 0;
      for (uint32_t p = 0; p < k; ++p) acc += (int64_t)a[(size_t)i * k + p] * (int64_t)b[(size_t)p * n + j];
      c[(size_t)i * n + j] = (float)acc;
    }
}

static int open_or_report(const char* path, prom_bridge** b) {
  prom_issue issue;
  if (prom_bridge_open(path, b, &issue) != 0) {
    printf("issue=%s symbol=%s abi=%u message=%s\n", prom_issue_name(issue.code), issue.symbol,
           (unsigned)issue.actual_abi, issue.message);
    fflush(stdout);
    return -1;
  }
  return 0;
}

static int cmd_open(const char* path) {
  prom_bridge* b = NULL;
  if (open_or_report(path, &b) != 0) return 3;
  const PrometheusCaps caps = prom_bridge_caps(b);
  printf("open=ok available=%u backend=%u reason=%u environment=%s\n", (unsigned)caps.available,
         (unsigned)caps.backend_type, (unsigned)caps.reason_code, prom_bridge_environment(b));
  prom_bridge_close(b);
  return 0;
}

static int cmd_strict(const char* path) {
  const double left[6] = {1, 2, 3, 4, 5, 6};
  const double right[6] = {7, 8, 9, 10, 11, 12};
  double out[4] = {0, 0, 0, 0};
  char err[640];
  if (prom_bridge_matmul_strict(path, left, right, 2, 3, 2, out, err, sizeof(err)) != 0) {
    printf("strict=error message=%s\n", err);
    return 3;
  }
  printf("strict=ok out=%g,%g,%g,%g\n", out[0], out[1], out[2], out[3]);
  return (out[0] == 58 && out[1] == 64 && out[2] == 139 && out[3] == 154) ? 0 : 1;
}

static void check_sgemm(prom_bridge* b, uint32_t m, uint32_t n, uint32_t k, uint32_t seed) {
  float* a = malloc(sizeof(float) * (size_t)m * k);
  float* bm = malloc(sizeof(float) * (size_t)k * n);
  float* c = malloc(sizeof(float) * (size_t)m * n);
  float* want = malloc(sizeof(float) * (size_t)m * n);
  char name[64];
  snprintf(name, sizeof(name), "sgemm_%ux%ux%u", (unsigned)m, (unsigned)n, (unsigned)k);
  if (!a || !bm || !c || !want) {
    report(name, 0, "host allocation failed");
  } else {
    small_ints(a, (size_t)m * k, seed);
    small_ints(bm, (size_t)k * n, seed + 1);
    int_matmul(a, bm, want, m, n, k);
    uint32_t stage = 0;
    int detail = 0;
    const int rc = prom_bridge_sgemm(b, a, bm, c, m, n, k, &stage, &detail);
    const int same = rc == PROM_OK && memcmp(c, want, sizeof(float) * (size_t)m * n) == 0;
    report(name, same, "rc=%d stage=%u detail=%d", rc, (unsigned)stage, detail);
  }
  free(a);
  free(bm);
  free(c);
  free(want);
}

static void check_sgemm_errors(prom_bridge* b) {
  float one = 1.0f, out = 0.0f;
  uint32_t stage = 0;
  int detail = 0;
  /* reactor_sgemm.cpp:4152-4191: a NULL operand is TRANSFER_IN, a zero
     dimension is INIT. */
  int rc = prom_bridge_sgemm(b, NULL, &one, &out, 1, 1, 1, &stage, &detail);
  report("sgemm_null_operand", rc == PROM_ERROR && stage == PROM_STAGE_TRANSFER_IN, "rc=%d stage=%u", rc,
         (unsigned)stage);
  rc = prom_bridge_sgemm(b, &one, &one, &out, 0, 1, 1, &stage, &detail);
  report("sgemm_zero_dimension", rc == PROM_ERROR && stage == PROM_STAGE_INIT, "rc=%d stage=%u", rc,
         (unsigned)stage);
}

static void check_strict(const char* path) {
  const double left[6] = {1, 2, 3, 4, 5, 6};
  const double right[6] = {7, 8, 9, 10, 11, 12};
  double out[4] = {0, 0, 0, 0};
  char err[640] = "";
  const int rc = prom_bridge_matmul_strict(path, left, right, 2, 3, 2, out, err, sizeof(err));
  report("strict_matmul_2x3x2", rc == 0 && out[0] == 58 && out[1] == 64 && out[2] == 139 && out[3] == 154,
         "%s", err);
  double none = 0;
  const int rc0 = prom_bridge_matmul_strict(path, left, right, 0, 3, 2, &none, err, sizeof(err));
  report("strict_matmul_empty", rc0 != 0 && strstr(err, "requires non-empty matrices") != NULL, "%s", err);
}

static void check_fft(prom_bridge* b) {
  const uint32_t n = 4096;
  double* x = calloc((size_t)2 * n, sizeof(double));
  double* y = calloc((size_t)2 * n, sizeof(double));
  if (!x || !y) {
    report("fft64", 0, "host allocation failed");
    free(x);
    free(y);
    return;
  }
  uint32_t stage = 0;
  int detail = 0;
  /* Impulse -> all ones, exactly (every output is 1 * 1 with no sums). */
  x[0] = 1.0;
  int rc = prom_bridge_fft64(b, x, y, n, &stage, &detail);
  int ok = rc == PROM_OK;
  for (uint32_t i = 0; ok && i < n; ++i) ok = y[2 * i] == 1.0 && y[2 * i + 1] == 0.0;
  report("fft64_impulse_4096", ok, "rc=%d stage=%u detail=%d", rc, (unsigned)stage, detail);

  /* e^(2 pi i f j / N) -> N at bin f, 0 elsewhere, to fft.go's 1e-12 * max|X|. */
  const uint32_t f = 37;
  for (uint32_t j = 0; j < n; ++j) {
    const double t = 2.0 * M_PI * (double)(((uint64_t)f * j) % n) / (double)n;
    x[2 * j] = cos(t);
    x[2 * j + 1] = sin(t);
  }
  rc = prom_bridge_fft64(b, x, y, n, &stage, &detail);
  double worst = 0.0;
  for (uint32_t i = 0; i < n; ++i) {
    const double re = y[2 * i] - (i == f ? (double)n : 0.0), im = y[2 * i + 1];
    const double e = fabs(re) > fabs(im) ? fabs(re) : fabs(im);
    if (e > worst) worst = e;
  }
  report("fft64_tone_4096", rc == PROM_OK && worst <= 1e-12 * n, "rc=%d max_err=%.3g", rc, worst);

  /* count 1 is the identity; count 3 is not a power of two. */
  const double one[2] = {0.25, -1.5};
  double got[2] = {0, 0};
  rc = prom_bridge_fft64(b, one, got, 1, &stage, &detail);
  report("fft64_count_1", rc == PROM_OK && got[0] == 0.25 && got[1] == -1.5, "rc=%d", rc);
  rc = prom_bridge_fft64(b, x, y, 3, &stage, &detail);
  report("fft64_rejects_count_3", rc == PROM_ERROR && stage == PROM_STAGE_INIT, "rc=%d stage=%u", rc,
         (unsigned)stage);
  free(x);
  free(y);
}

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static void check_async(prom_bridge* b) {
  const uint32_t m = 300, n = 260, k = 190;
  float* a = malloc(sizeof(float) * m * k);
  float* bm = malloc(sizeof(float) * k * n);
  float* c = malloc(sizeof(float) * m * n);
  float* want = malloc(sizeof(float) * m * n);
  if (!a || !bm || !c || !want) {
    report("async", 0, "host allocation failed");
    goto done;
  }
  small_ints(a, (size_t)m * k, 11);
  small_ints(bm, (size_t)k * n, 12);
  int_matmul(a, bm, want, m, n, k);
  int task = -1;
  uint32_t stage = 0;
  int detail = 0;
  int rc = prom_bridge_submit_async(b, a, bm, m, n, k, &task, &stage, &detail);
  report("async_submit", rc == PROM_OK && task >= 0, "rc=%d task=%d detail=%d", rc, task, detail);
  if (rc != PROM_OK) goto done;
  /* Poll until ready, for at most 30 s. */
  PrometheusAsyncStatus st;
  memset(&st, 0, sizeof(st));
  const double t0 = now_s();
  do {
    rc = prom_bridge_query_async(b, task, &st);
    if (rc != PROM_OK || st.ready || st.failed) break;
    struct timespec pause = {0, 200000};
    nanosleep(&pause, NULL);
  } while (now_s() - t0 < 30.0);
  report("async_query_ready", rc == PROM_OK && st.ready && !st.failed, "rc=%d ready=%u failed=%u", rc,
         (unsigned)st.ready, (unsigned)st.failed);
  rc = prom_bridge_consume_async(b, task, c, m * n, &stage, &detail);
  report("async_consume_exact", rc == PROM_OK && memcmp(c, want, sizeof(float) * m * n) == 0,
         "rc=%d stage=%u detail=%d", rc, (unsigned)stage, detail);
  /* A consumed task cannot be consumed again. */
  rc = prom_bridge_consume_async(b, task, c, m * n, &stage, &detail);
  report("async_consume_twice_rejected", rc != PROM_OK, "rc=%d detail=%d", rc, detail);
  /* Submit and abandon: the task table frees its slot. */
  rc = prom_bridge_submit_async(b, a, bm, m, n, k, &task, &stage, &detail);
  if (rc == PROM_OK) {
    const double t1 = now_s();
    do {
      if (prom_bridge_query_async(b, task, &st) != PROM_OK || st.ready || st.failed) break;
      struct timespec pause = {0, 200000};
      nanosleep(&pause, NULL);
    } while (now_s() - t1 < 30.0);
    rc = prom_bridge_abandon_async(b, task);
  }
  report("async_abandon", rc == PROM_OK, "rc=%d", rc);
done:
  free(a);
  free(bm);
  free(c);
  free(want);
}

static void fill_rms(PrometheusGemma4E2BM1InputRmsNormRequest* r, const float* x, const float* w, float* y,
                     float* inv, uint32_t rows, uint32_t width, uint64_t gen) {
  memset(r, 0, sizeof(*r));
  r->struct_size = (uint32_t)sizeof(*r);
  r->input = x;
  r->weight = w;
  r->output = y;
  r->inv_rms_output = inv;
  r->input_element_count = (uint64_t)rows * width;
  r->weight_element_count = width;
  r->output_element_count = (uint64_t)rows * width;
  r->inv_rms_output_element_count = rows;
  r->tokens = rows;
  r->model_width = width;
  r->input_row_stride = width;
  r->epsilon = 1e-6f;
  r->input_generation = 1;
  r->weight_generation = gen;
  r->exact_source_hash = 0x52A1;
}

static void check_rmsnorm(prom_bridge* b) {
  enum { kRows = 3, kWidth = 1536 };
  static float x[kRows * kWidth], w[kWidth], y[kRows * kWidth], y2[kRows * kWidth], inv[kRows];
  const float row_value[kRows] = {0.5f, -2.0f, 3.0f};
  for (int r = 0; r < kRows; ++r)
    for (int i = 0; i < kWidth; ++i) x[r * kWidth + i] = row_value[r];
  for (int i = 0; i < kWidth; ++i) w[i] = 0.75f + (float)(i % 7) / 64.0f;
  PrometheusGemma4E2BM1InputRmsNormRequest req;
  PrometheusGemma4E2BM1InputRmsNormResult res;
  fill_rms(&req, x, w, y, inv, kRows, kWidth, 1);
  memset(&res, 0, sizeof(res));
  res.struct_size = (uint32_t)sizeof(res);
  int rc = prom_bridge_gemma_input_rmsnorm(b, &req, &res);
  double err_y = 0.0, err_inv = 0.0;
  for (int r = 0; r < kRows; ++r) {
    const double c = row_value[r], s = 1.0 / sqrt(c * c + 1e-6);
    err_inv = fmax(err_inv, fabs(inv[r] - s));
    for (int i = 0; i < kWidth; ++i) err_y = fmax(err_y, fabs(y[r * kWidth + i] - c * s * w[i]));
  }
  /* The reference's bars: output within 1e-4, inverse RMS within 1e-5. */
  report("gemma_input_rmsnorm_constant_rows", rc == PROM_OK && err_y < 1e-4 && err_inv < 1e-5,
         "rc=%d stage=%u detail=%d err_y=%.3g err_inv=%.3g", rc, (unsigned)res.stage, (int)res.detail_code, err_y,
         err_inv);
  /* The same weight generation again is stale and writes nothing. */
  for (int i = 0; i < kRows * kWidth; ++i) y2[i] = -7.0f;
  fill_rms(&req, x, w, y2, inv, kRows, kWidth, 1);
  rc = prom_bridge_gemma_input_rmsnorm(b, &req, &res);
  int untouched = 1;
  for (int i = 0; i < kRows * kWidth; ++i) untouched &= y2[i] == -7.0f;
  report("gemma_input_rmsnorm_stale_generation", rc == PROM_ERROR && res.stage == PROM_STAGE_TRANSFER_IN && untouched,
         "rc=%d stage=%u", rc, (unsigned)res.stage);
}

static int cmd_run(const char* path) {
  prom_bridge* b = NULL;
  if (open_or_report(path, &b) != 0) return 3;
  char why[256];
  if (prom_bridge_require_hardware_gpu(b, why, sizeof(why)) != 0) {
    printf("issue=hardware_gpu message=%s\n", why);
    prom_bridge_close(b);
    return 3;
  }
  static const char* const optional[] = {
      "prometheus_reactor_runtime_fft64", "prometheus_reactor_runtime_sgemm_submit_async",
      "prometheus_reactor_runtime_sgemm_query_async", "prometheus_reactor_runtime_sgemm_consume_async",
      "prometheus_reactor_runtime_sgemm_abandon_async", "prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm"};
  int all = 1;
  for (size_t i = 0; i < sizeof(optional) / sizeof(optional[0]); ++i) all &= prom_bridge_has(b, optional[i]);
  report("optional_entries_resolved", all, NULL);
  report("environment", strcmp(prom_bridge_environment(b), "hardware_gpu_hip") == 0, "%s",
         prom_bridge_environment(b));

  /* Three shapes: the reference's own 2x3x2, a ragged one, and a square one
     large enough for the MFMA tiles and split-K. */
  {
    const float a[6] = {1, 2, 3, 4, 5, 6}, bm[6] = {7, 8, 9, 10, 11, 12};
    float c[4] = {0, 0, 0, 0};
    uint32_t stage = 0;
    int detail = 0;
    const int rc = prom_bridge_sgemm(b, a, bm, c, 2, 2, 3, &stage, &detail);
    report("sgemm_2x2x3_known_answer", rc == PROM_OK && c[0] == 58 && c[1] == 64 && c[2] == 139 && c[3] == 154,
           "rc=%d", rc);
  }
  check_sgemm(b, 67, 129, 95, 1);
  check_sgemm(b, 1024, 1024, 2048, 5);
  check_sgemm_errors(b);
  check_fft(b);
  check_async(b);
  check_rmsnorm(b);
  prom_bridge_close(b);
  /* strict.go opens a runtime of its own per call. */
  check_strict(path);
  printf("%s failures=%d\n", failures ? "FAILED" : "PASSED", failures);
  return failures ? 1 : 0;
}

int main(int argc, char** argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: %s open|strict|run [library]\n", argv[0]);
    return 2;
  }
  const char* path = argc > 2 ? argv[2] : NULL;
  if (!strcmp(argv[1], "open")) return cmd_open(path);
  if (!strcmp(argv[1], "strict")) return cmd_strict(path);
  if (!strcmp(argv[1], "run")) return cmd_run(path);
  fprintf(stderr, "unknown command %s\n", argv[1]);
  return 2;
}
