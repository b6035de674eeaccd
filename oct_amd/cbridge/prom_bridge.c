/* C loader and call layer for libprometheus_reactor.so; the contract of
 * each function is in prom_bridge.h.  The call sequence follows
 * internal/prometheus/bridge.go:242-394 and the trampolines
 * bridge_dlopen_linux.go:56-67, 305-327, 395-448. */
#define _GNU_SOURCE
#include "prom_bridge.h"

#include <dlfcn.h>
#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

typedef uint32_t (*abi_fn)(void);
typedef int (*create_fn)(void*, void**);
typedef int (*destroy_fn)(void*);
typedef int (*probe_fn)(void*, PrometheusCaps*);
typedef int (*sgemm_fn)(void*, const float*, const float*, float*, uint32_t, uint32_t, uint32_t, uint32_t*, int*);
typedef int (*fft64_fn)(void*, const double*, double*, uint32_t, uint32_t*, int*);
typedef int (*submit_fn)(void*, const float*, const float*, uint32_t, uint32_t, uint32_t, int*, uint32_t*, int*);
typedef int (*query_fn)(void*, int, PrometheusAsyncStatus*);
typedef int (*consume_fn)(void*, int, float*, uint32_t, uint32_t*, int*);
typedef int (*abandon_fn)(void*, int);
typedef int (*rmsnorm_fn)(void*, const PrometheusGemma4E2BM1InputRmsNormRequest*,
                          PrometheusGemma4E2BM1InputRmsNormResult*);

struct prom_bridge {
  void* lib;
  void* handle;
  PrometheusCaps caps;
  char path[512];
  destroy_fn destroy;
  sgemm_fn sgemm;
  fft64_fn fft64;
  submit_fn submit;
  query_fn query;
  consume_fn consume;
  abandon_fn abandon;
  rmsnorm_fn input_rmsnorm;
};

static const char* const kSymAbi = "prometheus_reactor_abi_version";
static const char* const kSymCreate = "prometheus_reactor_runtime_create";
static const char* const kSymDestroy = "prometheus_reactor_runtime_destroy";
static const char* const kSymProbe = "prometheus_reactor_runtime_probe";
static const char* const kSymSgemm = "prometheus_reactor_runtime_sgemm";
static const char* const kSymFft64 = "prometheus_reactor_runtime_fft64";
static const char* const kSymSubmit = "prometheus_reactor_runtime_sgemm_submit_async";
static const char* const kSymQuery = "prometheus_reactor_runtime_sgemm_query_async";
static const char* const kSymConsume = "prometheus_reactor_runtime_sgemm_consume_async";
static const char* const kSymAbandon = "prometheus_reactor_runtime_sgemm_abandon_async";
static const char* const kSymInputRms = "prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm";

const char* prom_issue_name(prom_issue_code code) {
  switch (code) {
    case PROM_ISSUE_NONE: return "none";
    case PROM_ISSUE_NOT_FOUND: return "reactor_not_found";
    case PROM_ISSUE_LOAD_FAILED: return "reactor_load_failed";
    case PROM_ISSUE_SYMBOL_MISSING: return "symbol_missing";
    case PROM_ISSUE_ABI_MISMATCH: return "abi_mismatch";
    case PROM_ISSUE_CREATE_FAILED: return "runtime_create_failed";
    case PROM_ISSUE_PROBE_UNAVAILABLE: return "runtime_probe_unavailable";
    case PROM_ISSUE_SGEMM_FAILED: return "runtime_sgemm_failed";
  }
  return "unknown";
}

/* Truncating copy; dst always ends in a NUL. */
static void copy_str(char* dst, size_t cap, const char* src) {
  if (cap == 0) return;
  const size_t n = src ? strnlen(src, cap - 1) : 0;
  if (n) memcpy(dst, src, n);
  dst[n] = '\0';
}

/* Fills *issue (when given) with bridge.go:54-71's text for the code,
   followed by ": detail" when a detail is given. */
static int fail(prom_issue* issue, prom_issue_code code, const char* path, const char* symbol, const char* fmt, ...) {
  if (!issue) return -1;
  memset(issue, 0, sizeof(*issue));
  issue->code = code;
  issue->expected_abi = PROM_REACTOR_ABI_V1;
  copy_str(issue->path, sizeof(issue->path), path);
  copy_str(issue->symbol, sizeof(issue->symbol), symbol);
  char detail[384] = "";
  if (fmt) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(detail, sizeof(detail), fmt, ap);
    va_end(ap);
  }
  const char* head;
  switch (code) {
    case PROM_ISSUE_NOT_FOUND: head = "prometheus reactor not found"; break;
    case PROM_ISSUE_SYMBOL_MISSING: head = "prometheus reactor missing symbol"; break;
    case PROM_ISSUE_ABI_MISMATCH: head = "prometheus reactor ABI mismatch"; break;
    case PROM_ISSUE_CREATE_FAILED: head = "prometheus reactor runtime creation failed"; break;
    case PROM_ISSUE_PROBE_UNAVAILABLE: head = "prometheus reactor runtime probe failed"; break;
    case PROM_ISSUE_SGEMM_FAILED: head = "prometheus reactor runtime sgemm failed"; break;
    default: head = "prometheus reactor load failed"; break;
  }
  if (code == PROM_ISSUE_SYMBOL_MISSING)
    snprintf(issue->message, sizeof(issue->message), "%s \"%s\"%s%s", head, symbol ? symbol : "",
             detail[0] ? ": " : "", detail);
  else
    snprintf(issue->message, sizeof(issue->message), "%s%s%s", head, detail[0] ? ": " : "", detail);
  return -1;
}

/* dlsym's object pointer, moved into a function pointer without the cast
   ISO C leaves undefined. */
static int resolve(void* lib, const char* name, void* fn_out, size_t fn_size) {
  dlerror();
  void* sym = dlsym(lib, name);
  if (!sym || fn_size != sizeof(sym)) return -1;
  memcpy(fn_out, &sym, fn_size);
  return 0;
}
#define RESOLVE(lib, name, fn) resolve((lib), (name), &(fn), sizeof(fn))

static int exists(const char* path) {
  struct stat st;
  return stat(path, &st) == 0;
}

static uint32_t test_flags_from_env(void) {
  const char* v = getenv(PROM_BRIDGE_ENV_TEST_FLAGS);
  if (!v || !*v) return 0;
  char* end = NULL;
  errno = 0;
  const unsigned long long x = strtoull(v, &end, 0);
  if (errno || end == v || *end || x > 0xffffffffull) return 0;
  return (uint32_t)x;
}

/* bridge.go:276-394 on one opened library.  On failure the library stays
   open; the caller closes it. */
static int runtime_from_library(const char* path, void* lib, prom_bridge** out, prom_issue* issue) {
  abi_fn abi = NULL;
  create_fn create = NULL;
  destroy_fn destroy = NULL;
  probe_fn probe = NULL;
  if (RESOLVE(lib, kSymAbi, abi)) return fail(issue, PROM_ISSUE_SYMBOL_MISSING, path, kSymAbi, NULL);
  const uint32_t actual = abi();
  if (actual != PROM_REACTOR_ABI_V1) {
    fail(issue, PROM_ISSUE_ABI_MISMATCH, path, NULL, "expected=%u actual=%u", (unsigned)PROM_REACTOR_ABI_V1,
         (unsigned)actual);
    if (issue) issue->actual_abi = actual;
    return -1;
  }
  if (RESOLVE(lib, kSymCreate, create)) return fail(issue, PROM_ISSUE_SYMBOL_MISSING, path, kSymCreate, NULL);
  if (RESOLVE(lib, kSymDestroy, destroy)) return fail(issue, PROM_ISSUE_SYMBOL_MISSING, path, kSymDestroy, NULL);
  if (RESOLVE(lib, kSymProbe, probe)) return fail(issue, PROM_ISSUE_SYMBOL_MISSING, path, kSymProbe, NULL);

  /* bridge.go:315-319; no shader package applies to this library. */
  PrometheusReactorConfig cfg;
  memset(&cfg, 0, sizeof(cfg));
  cfg.struct_size = (uint32_t)sizeof(cfg);
  cfg.test_flags = test_flags_from_env();
  cfg.reduction_ring_depth = 3;
  void* handle = NULL;
  int rc = create(&cfg, &handle);
  if (rc != PROM_OK || !handle) return fail(issue, PROM_ISSUE_CREATE_FAILED, path, NULL, "status %d", rc);

  PrometheusCaps caps;
  memset(&caps, 0, sizeof(caps));
  rc = probe(handle, &caps);
  if (rc != PROM_OK || !caps.available) {
    destroy(handle);
    return fail(issue, PROM_ISSUE_PROBE_UNAVAILABLE, path, NULL, "status %d available=%u backend=%u reason=%u", rc,
                (unsigned)caps.available, (unsigned)caps.backend_type, (unsigned)caps.reason_code);
  }

  prom_bridge* b = (prom_bridge*)calloc(1, sizeof(*b));
  if (!b) {
    destroy(handle);
    return fail(issue, PROM_ISSUE_LOAD_FAILED, path, NULL, "out of host memory");
  }
  if (RESOLVE(lib, kSymSgemm, b->sgemm)) {
    destroy(handle);
    free(b);
    return fail(issue, PROM_ISSUE_SYMBOL_MISSING, path, kSymSgemm, NULL);
  }
  /* Optional entries (bridge.go:346-391). */
  (void)RESOLVE(lib, kSymFft64, b->fft64);
  (void)RESOLVE(lib, kSymSubmit, b->submit);
  (void)RESOLVE(lib, kSymQuery, b->query);
  (void)RESOLVE(lib, kSymConsume, b->consume);
  (void)RESOLVE(lib, kSymAbandon, b->abandon);
  (void)RESOLVE(lib, kSymInputRms, b->input_rmsnorm);
  b->lib = lib;
  b->handle = handle;
  b->caps = caps;
  b->destroy = destroy;
  copy_str(b->path, sizeof(b->path), path);
  *out = b;
  return 0;
}

static int open_one(const char* path, prom_bridge** out, prom_issue* issue, int* loaded) {
  *loaded = 0;
  dlerror();
  void* lib = dlopen(path, RTLD_NOW | RTLD_LOCAL);
  if (!lib) {
    const char* why = dlerror();
    return fail(issue, PROM_ISSUE_LOAD_FAILED, path, NULL, "%s", why ? why : "dlopen failed");
  }
  *loaded = 1;
  if (runtime_from_library(path, lib, out, issue) != 0) {
    dlclose(lib);
    return -1;
  }
  return 0;
}

int prom_bridge_open(const char* path, prom_bridge** out, prom_issue* issue) {
  prom_issue local;
  if (!issue) issue = &local;
  if (!out) return fail(issue, PROM_ISSUE_LOAD_FAILED, path, NULL, "no output handle");
  *out = NULL;

  /* bridge.go:552-582 */
  char cand[4][512];
  int n = 0;
  const char* env = getenv(PROM_BRIDGE_ENV_LIBRARY);
  if (path && *path) {
    copy_str(cand[n++], sizeof(cand[0]), path);
  } else if (env && *env) {
    copy_str(cand[n++], sizeof(cand[0]), env);
  } else {
    snprintf(cand[n++], sizeof(cand[0]), "internal/prometheus/reactor/%s", PROM_BRIDGE_LIBRARY_BASENAME);
    snprintf(cand[n++], sizeof(cand[0]), "out/prometheus/native/%s", PROM_BRIDGE_LIBRARY_BASENAME);
    char exe[400];
    const ssize_t len = readlink("/proc/self/exe", exe, sizeof(exe) - 1);
    if (len > 0) {
      exe[len] = '\0';
      char* slash = strrchr(exe, '/');
      if (slash) {
        *slash = '\0';
        snprintf(cand[n++], sizeof(cand[0]), "%s/%s", exe, PROM_BRIDGE_LIBRARY_BASENAME);
      }
    }
  }

  /* bridge.go:253-272: a missing candidate is skipped, a failed load is
     remembered, and the first library that loads decides the outcome. */
  prom_issue last;
  int have_last = 0;
  for (int i = 0; i < n; ++i) {
    if (!exists(cand[i])) continue;
    int loaded = 0;
    if (open_one(cand[i], out, &last, &loaded) == 0) {
      memset(issue, 0, sizeof(*issue));
      return 0;
    }
    if (loaded) {
      *issue = last;
      return -1;
    }
    have_last = 1;
  }
  if (have_last) {
    *issue = last;
    return -1;
  }
  return fail(issue, PROM_ISSUE_NOT_FOUND, n ? cand[0] : "", NULL, NULL);
}

void prom_bridge_close(prom_bridge* b) {
  if (!b) return;
  if (b->destroy && b->handle) b->destroy(b->handle);
  if (b->lib) dlclose(b->lib);
  free(b);
}

PrometheusCaps prom_bridge_caps(const prom_bridge* b) {
  PrometheusCaps none;
  memset(&none, 0, sizeof(none));
  return b ? b->caps : none;
}

const char* prom_bridge_path(const prom_bridge* b) { return b ? b->path : ""; }

const char* prom_bridge_environment(const prom_bridge* b) {
  if (!b) return "unknown";
  switch (b->caps.backend_type) {
    case PROM_BACKEND_HARDWARE_GPU: return "hardware_gpu_hip";
    case PROM_BACKEND_VULKAN_SOFTWARE: return "software_vulkan_llvmpipe_or_cpu";
    default: return "unknown";
  }
}

int prom_bridge_require_hardware_gpu(const prom_bridge* b, char* err, size_t err_len) {
  if (b && b->caps.available && b->caps.backend_type == PROM_BACKEND_HARDWARE_GPU) return 0;
  if (err && err_len)
    snprintf(err, err_len, "GPU execution requires a hardware device; backend is %s", prom_bridge_environment(b));
  return -1;
}

int prom_bridge_has(const prom_bridge* b, const char* symbol) {
  if (!b || !symbol) return 0;
  if (!strcmp(symbol, kSymSgemm)) return b->sgemm != NULL;
  if (!strcmp(symbol, kSymFft64)) return b->fft64 != NULL;
  if (!strcmp(symbol, kSymSubmit)) return b->submit != NULL;
  if (!strcmp(symbol, kSymQuery)) return b->query != NULL;
  if (!strcmp(symbol, kSymConsume)) return b->consume != NULL;
  if (!strcmp(symbol, kSymAbandon)) return b->abandon != NULL;
  if (!strcmp(symbol, kSymInputRms)) return b->input_rmsnorm != NULL;
  return 0;
}

static int unavailable(uint32_t* stage, int* detail) {
  if (stage) *stage = PROM_STAGE_INIT;
  if (detail) *detail = PROM_BRIDGE_DETAIL_ENTRY_UNAVAILABLE;
  return PROM_ERROR;
}

int prom_bridge_sgemm(prom_bridge* b, const float* a, const float* bm, float* c, uint32_t m, uint32_t n, uint32_t k,
                      uint32_t* stage, int* detail) {
  if (!b || !b->sgemm) return unavailable(stage, detail);
  return b->sgemm(b->handle, a, bm, c, m, n, k, stage, detail);
}

int prom_bridge_fft64(prom_bridge* b, const double* input, double* output, uint32_t count, uint32_t* stage,
                      int* detail) {
  if (!b || !b->fft64) return unavailable(stage, detail);
  return b->fft64(b->handle, input, output, count, stage, detail);
}

int prom_bridge_submit_async(prom_bridge* b, const float* a, const float* bm, uint32_t m, uint32_t n, uint32_t k,
                             int* task_id, uint32_t* stage, int* detail) {
  if (!b || !b->submit) return unavailable(stage, detail);
  return b->submit(b->handle, a, bm, m, n, k, task_id, stage, detail);
}

int prom_bridge_query_async(prom_bridge* b, int task_id, PrometheusAsyncStatus* status) {
  if (!b || !b->query) return PROM_ERROR;
  return b->query(b->handle, task_id, status);
}

int prom_bridge_consume_async(prom_bridge* b, int task_id, float* c, uint32_t c_len, uint32_t* stage, int* detail) {
  if (!b || !b->consume) return unavailable(stage, detail);
  return b->consume(b->handle, task_id, c, c_len, stage, detail);
}

int prom_bridge_abandon_async(prom_bridge* b, int task_id) {
  if (!b || !b->abandon) return PROM_ERROR;
  return b->abandon(b->handle, task_id);
}

int prom_bridge_gemma_input_rmsnorm(prom_bridge* b, const PrometheusGemma4E2BM1InputRmsNormRequest* request,
                                    PrometheusGemma4E2BM1InputRmsNormResult* result) {
  if (!b || !b->input_rmsnorm) return PROM_ERROR;
  return b->input_rmsnorm(b->handle, request, result);
}

int prom_bridge_matmul_strict(const char* path, const double* left, const double* right, uint32_t rows,
                              uint32_t inner, uint32_t cols, double* out, char* err, size_t err_len) {
  static const char kPrefix[] = "PROMETHEUS requires GPU matrix execution: ";
  char tmp[8];
  if (!err || err_len == 0) {
    err = tmp;
    err_len = sizeof(tmp);
  }
  err[0] = '\0';
  /* runtime.go:259-279 */
  if (rows == 0 || inner == 0 || cols == 0 || !left || !right || !out) {
    snprintf(err, err_len, "%s",
             rows == 0 ? "compiled Prometheus matmul requires non-empty matrices"
                       : "compiled Prometheus matmul requires matrices with at least one column");
    return -1;
  }
  prom_issue issue;
  prom_bridge* b = NULL;
  if (prom_bridge_open(path, &b, &issue) != 0) {
    snprintf(err, err_len, "%s%s", kPrefix, issue.message);
    return -1;
  }
  char why[256];
  if (prom_bridge_require_hardware_gpu(b, why, sizeof(why)) != 0) {
    snprintf(err, err_len, "%s%s", kPrefix, why);
    prom_bridge_close(b);
    return -1;
  }
  const size_t na = (size_t)rows * inner, nb = (size_t)inner * cols, nc = (size_t)rows * cols;
  float* a32 = (float*)malloc(na * sizeof(float));
  float* b32 = (float*)malloc(nb * sizeof(float));
  float* c32 = (float*)malloc(nc * sizeof(float));
  int result = -1;
  if (!a32 || !b32 || !c32) {
    snprintf(err, err_len, "%sout of host memory", kPrefix);
  } else {
    for (size_t i = 0; i < na; ++i) a32[i] = (float)left[i];
    for (size_t i = 0; i < nb; ++i) b32[i] = (float)right[i];
    uint32_t stage = 0;
    int detail = 0;
    const int rc = prom_bridge_sgemm(b, a32, b32, c32, rows, cols, inner, &stage, &detail);
    if (rc != PROM_OK) {
      snprintf(err, err_len, "%s%s: status %d stage %u detail %d", kPrefix, prom_issue_name(PROM_ISSUE_SGEMM_FAILED),
               rc, (unsigned)stage, detail);
    } else {
      for (size_t i = 0; i < nc; ++i) out[i] = (double)c32[i];
      result = 0;
    }
  }
  free(a32);
  free(b32);
  free(c32);
  prom_bridge_close(b);
  return result;
}
