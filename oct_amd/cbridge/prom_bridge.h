/* C loader and call layer for libprometheus_reactor.so.
 *
 * Oct's Go package binds the reactor through cgo: a C preamble of dlopen,
 * dlsym and one small trampoline per entry point
 * (internal/prometheus/bridge_dlopen_linux.go:5-192, 211-237, 305-327), and
 * Go code that checks the ABI, creates and probes a runtime and maps
 * failures to ReactorIssue codes (internal/prometheus/bridge.go:36-71,
 * 242-394, 552-594).  This file is that C half written as a compiled,
 * tested library: a cgo preamble includes this header and links
 * prom_bridge.c, and the Go methods become one-line calls.  It is also
 * usable from any C or C++ host.
 *
 * Every entry returns the reactor's own status (PROM_OK, PROM_ERROR, ...)
 * and passes its stage and detail codes through unchanged.
 */
#ifndef OCT_PROM_BRIDGE_H
#define OCT_PROM_BRIDGE_H

#include <stddef.h>
#include <stdint.h>

#include "prometheus_reactor.h"

#ifdef __cplusplus
extern "C" {
#endif

/* bridge.go:36-42 -- the ReactorIssue codes. */
typedef enum {
  PROM_ISSUE_NONE = 0,
  PROM_ISSUE_NOT_FOUND,         /* "reactor_not_found" */
  PROM_ISSUE_LOAD_FAILED,       /* "reactor_load_failed" */
  PROM_ISSUE_SYMBOL_MISSING,    /* "symbol_missing" */
  PROM_ISSUE_ABI_MISMATCH,      /* "abi_mismatch" */
  PROM_ISSUE_CREATE_FAILED,     /* "runtime_create_failed" */
  PROM_ISSUE_PROBE_UNAVAILABLE, /* "runtime_probe_unavailable" */
  PROM_ISSUE_SGEMM_FAILED       /* "runtime_sgemm_failed" */
} prom_issue_code;

typedef struct {
  prom_issue_code code;
  uint32_t expected_abi;
  uint32_t actual_abi;
  char path[512];
  char symbol[128];
  char message[512]; /* bridge.go:54-71's text, then the loader's own detail */
} prom_issue;

/* Environment variables read by prom_bridge_open (bridge.go:552-594). */
#define PROM_BRIDGE_ENV_LIBRARY "OCT_PROMETHEUS_REACTOR"
#define PROM_BRIDGE_ENV_TEST_FLAGS "OCT_PROMETHEUS_REACTOR_TEST_FLAGS"
#define PROM_BRIDGE_LIBRARY_BASENAME "libprometheus_reactor.so"

/* Returned as detail code, with stage PROM_STAGE_INIT, when an optional
   entry point is absent from the loaded library (runtime.go's -3). */
#define PROM_BRIDGE_DETAIL_ENTRY_UNAVAILABLE (-3)

typedef struct prom_bridge prom_bridge;

/* The ReactorIssue code's name ("reactor_not_found", ...). */
const char* prom_issue_name(prom_issue_code code);

/* Loads the reactor and opens a runtime (bridge.go:242-394).
 *
 * path == NULL follows bridge.go:552-582: $OCT_PROMETHEUS_REACTOR if set,
 * else internal/prometheus/reactor/ and out/prometheus/native/ under the
 * working directory, then the executable's directory.  A candidate that does
 * not exist is skipped; one that fails to load is remembered and reported if
 * no later candidate loads.  The library is opened with RTLD_NOW |
 * RTLD_LOCAL.  Then: abi_version must be 1; create, destroy and probe must
 * resolve; create gets test_flags from $OCT_PROMETHEUS_REACTOR_TEST_FLAGS
 * (strtoul base 0; unparsable -> 0) and reduction_ring_depth 3; probe must
 * report available; sgemm must resolve.  The async and Gemma entries are
 * optional.  Returns 0 and *out on success, else -1 with *issue filled
 * (issue may be NULL). */
int prom_bridge_open(const char* path, prom_bridge** out, prom_issue* issue);

/* Destroys the runtime and closes the library (bridge.go:396-408).
   NULL is allowed. */
void prom_bridge_close(prom_bridge* bridge);

PrometheusCaps prom_bridge_caps(const prom_bridge* bridge);
const char* prom_bridge_path(const prom_bridge* bridge);

/* bridge.go:518-532: "hardware_gpu_hip" for backend 2 (the reference says
   "hardware_vulkan"), "software_vulkan_llvmpipe_or_cpu" for 3, else
   "unknown". */
const char* prom_bridge_environment(const prom_bridge* bridge);

/* fft.go:50-55: 0 when the runtime is available on a hardware device, else
   -1 with a message in err. */
int prom_bridge_require_hardware_gpu(const prom_bridge* bridge, char* err, size_t err_len);

/* 1 if the loaded library exports the named optional entry point. */
int prom_bridge_has(const prom_bridge* bridge, const char* symbol);

/* Trampolines (bridge_dlopen_linux.go:56-67, 305-327, 395-448). */
int prom_bridge_sgemm(prom_bridge* bridge, const float* a, const float* b, float* c, uint32_t m, uint32_t n,
                      uint32_t k, uint32_t* stage, int* detail);
int prom_bridge_fft64(prom_bridge* bridge, const double* input, double* output, uint32_t count,
                      uint32_t* stage, int* detail);
int prom_bridge_submit_async(prom_bridge* bridge, const float* a, const float* b, uint32_t m, uint32_t n,
                             uint32_t k, int* task_id, uint32_t* stage, int* detail);
int prom_bridge_query_async(prom_bridge* bridge, int task_id, PrometheusAsyncStatus* status);
int prom_bridge_consume_async(prom_bridge* bridge, int task_id, float* c, uint32_t c_len, uint32_t* stage,
                              int* detail);
int prom_bridge_abandon_async(prom_bridge* bridge, int task_id);
int prom_bridge_gemma_input_rmsnorm(prom_bridge* bridge, const PrometheusGemma4E2BM1InputRmsNormRequest* request,
                                    PrometheusGemma4E2BM1InputRmsNormResult* result);

/* strict.go:11-32 on flat row-major binary64 operands: left is rows x inner,
 * right is inner x cols, out receives rows x cols.  Opens a runtime (path as
 * in prom_bridge_open), requires a hardware device, runs SGEMM in fp32 and
 * widens the result.  Never computes a CPU substitute: any failure returns -1
 * with err starting "PROMETHEUS requires GPU matrix execution: " (a failed
 * SGEMM call included, as strict.go:24-27 wraps it), or, for an empty shape,
 * "compiled Prometheus matmul requires ..." as runtime.go:259-279 words it. */
int prom_bridge_matmul_strict(const char* path, const double* left, const double* right, uint32_t rows,
                              uint32_t inner, uint32_t cols, double* out, char* err, size_t err_len);

#ifdef __cplusplus
}
#endif

#endif /* OCT_PROM_BRIDGE_H */
