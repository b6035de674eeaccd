/*
 * prometheus_reactor.h -- C ABI of the MI355X (gfx950) Prometheus reactor.
 *
 * A drop-in for the subset of Oct's `libprometheus_reactor.so` that the
 * north-star hot path uses: runtime lifecycle, FP32 SGEMM (the `@` operator
 * inside PROMETHEUS { }), row reductions (sum / max / stable softmax) and
 * RMSNorm.  Struct layouts, enum values and status conventions of those entry
 * points are kept identical to the reference so an unmodified Go loader binds
 * this library.  Entry points the reference does not have (bf16 GEMM,
 * generic RMSNorm, device-resident variants, transformer blocks) follow the
 * same conventions and are marked NEW.
 *
 * Conventions (reference: internal/prometheus/native/reactor_api.h:55-83,227-324):
 *   return PROM_OK / PROM_ERROR / PROM_INVALID_HANDLE / PROM_INTERNAL_ERROR;
 *   out_stage reports the phase reached (TRANSFER_OUT on success);
 *   out_detail is a positive path code on success, negative on failure.
 *   Host-pointer entry points are synchronous: inputs are copied in, the
 *   result copied out before return; outputs are written only on success.
 */
#ifndef OCT_AMD_PROMETHEUS_REACTOR_H
#define OCT_AMD_PROMETHEUS_REACTOR_H

#include <stdint.h>

#if defined(__GNUC__)
#define PROM_REACTOR_API __attribute__((visibility("default")))
#else
#define PROM_REACTOR_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* reactor_api.h:22-25 */
enum { PROM_REACTOR_ABI_V1 = 1u };

/* reactor_api.h:55-60 */
enum { PROM_OK = 0, PROM_ERROR = 1, PROM_INVALID_HANDLE = 2, PROM_INTERNAL_ERROR = 3 };

/* reactor_api.h:62-67.  Value 2 is "hardware GPU" to the Go loader
   (internal/prometheus/fft.go:50-55 requires it); this library reports 2 on a
   HIP device and exposes the real device via ..._hip_device_diagnostics. */
enum {
  PROM_BACKEND_UNKNOWN = 0,
  PROM_BACKEND_STUB = 1,
  PROM_BACKEND_VULKAN = 2,
  PROM_BACKEND_HARDWARE_GPU = 2,
  PROM_BACKEND_VULKAN_SOFTWARE = 3,
};

/* reactor_api.h:69-73 */
enum { PROM_REASON_NONE = 0, PROM_REASON_STUB_UNAVAILABLE = 1, PROM_REASON_VULKAN_UNAVAILABLE = 2 };

/* reactor_api.h:76-83 */
enum {
  PROM_STAGE_NONE = 0,
  PROM_STAGE_INIT = 1,
  PROM_STAGE_TRANSFER_IN = 2,
  PROM_STAGE_SUBMIT = 3,
  PROM_STAGE_TRANSFER_OUT = 4,
  PROM_STAGE_CLEANUP = 5,
};

/* reactor_api.h:131-166 (the fault-injection bits this library honours). */
enum {
  PROM_TESTCFG_FAIL_DEVICE_CREATE = 1u << 0,
  PROM_TESTCFG_FAIL_BUFFER_ALLOC = 1u << 2,
  PROM_TESTCFG_FAIL_UPLOAD = 1u << 3,
  PROM_TESTCFG_FAIL_DISPATCH = 1u << 4,
  PROM_TESTCFG_FAIL_DOWNLOAD = 1u << 5,
  PROM_TESTCFG_SKIP_VULKAN_INIT = 1u << 7,
  /* An async query observes a failure for every submitted task. */
  PROM_TESTCFG_FAIL_ASYNC_POLL = 1u << 15,
  /* The recorded work fails to end / to be submitted: the synchronous SGEMM
     fails at stage SUBMIT with detail -4 (reactor_sgemm.cpp:5071-5078), the
     binary64 FFT with PROM_FFT_DETAIL_DISPATCH_FAILED
     (PrometheusFft.concept:171, reactor_concept_fft.cpp:63-70); nothing is
     queued and no output is written. */
  PROM_TESTCFG_FAIL_COMMAND_END = 1u << 20,
  PROM_TESTCFG_FAIL_QUEUE_SUBMIT = 1u << 22,
};

/* reactor_api.h:227-324 (subset) */
enum {
  PROM_DETAIL_INJECTED_UPLOAD_FAILURE = -6001,
  PROM_DETAIL_INJECTED_DISPATCH_FAILURE = -6002,
  PROM_DETAIL_INJECTED_DOWNLOAD_FAILURE = -6003,
  PROM_DETAIL_SIZE_OVERFLOW = -6004,
  PROM_DETAIL_PATH_DIRECT = 6101,
  /* NEW success path codes (no Vulkan counterpart). */
  PROM_DETAIL_PATH_HIP_MFMA_F32 = 6120,
  PROM_DETAIL_PATH_HIP_GEMV_F32 = 6121,
  PROM_DETAIL_PATH_HIP_MFMA_BF16 = 6122,
  PROM_DETAIL_PATH_HIP_SIMT_F32 = 6123,
  /* NEW failure detail codes. */
  PROM_DETAIL_HIP_ALLOC_FAILED = -6901,
  PROM_DETAIL_HIP_COPY_FAILED = -6902,
  PROM_DETAIL_HIP_LAUNCH_FAILED = -6903,
  PROM_DETAIL_HIP_SYNC_FAILED = -6904,
  PROM_DETAIL_HIP_UNAVAILABLE = -6905,
  PROM_DETAIL_INVALID_ARGUMENT = -6906,
  /* ..._sgemm_device_noalloc: the plan's split-K partials exceed the static
     scratch array, or the array's device address could not be obtained. */
  PROM_DETAIL_SCRATCH_LIMIT = -6930,
  PROM_DETAIL_SCRATCH_UNAVAILABLE = -6931,
};

/* reactor_api.h:386-390 */
enum {
  PROM_REDUCTION_OPERATION_SUM = 1u,
  PROM_REDUCTION_OPERATION_MAX = 2u,
  PROM_REDUCTION_OPERATION_SOFTMAX = 3u,
};
/* reactor_api.h:392-395 */
enum { PROM_REDUCTION_FINALIZATION_NONE = 0u, PROM_REDUCTION_FINALIZATION_STABLE_SOFTMAX = 1u };
/* reactor_api.h:397-402 */
enum {
  PROM_REDUCTION_STRATEGY_AUTO = 0u,
  PROM_REDUCTION_STRATEGY_FUSED_SINGLE_WORKGROUP = 1u,
  PROM_REDUCTION_STRATEGY_COMPOSED = 2u,
  PROM_REDUCTION_STRATEGY_PACKED_SHORT_ROWS = 3u,
};
/* reactor_api.h:404-412 */
enum {
  PROM_REDUCTION_STAGE_ROW_SUM = 1u,
  PROM_REDUCTION_STAGE_ROW_MAX = 2u,
  PROM_REDUCTION_STAGE_SOFTMAX_EXP_SUM = 3u,
  PROM_REDUCTION_STAGE_SOFTMAX_NORMALIZE = 4u,
  PROM_REDUCTION_STAGE_SOFTMAX_FUSED = 5u,
  PROM_REDUCTION_STAGE_ROW_SUM_PACKED_SHORT = 6u,
  PROM_REDUCTION_STAGE_SOFTMAX_PACKED_SHORT = 7u,
};
/* reactor_api.h:414-419 */
enum {
  PROM_REDUCTION_TEMPORARY_NONE = 0u,
  PROM_REDUCTION_TEMPORARY_PARTIALS = 1u,
  PROM_REDUCTION_TEMPORARY_ROW_MAX = 2u,
  PROM_REDUCTION_TEMPORARY_ROW_SUM = 3u,
};
/* reactor_api.h:421-424 */
enum { PROM_REDUCTION_FLAG_FORCE_FUSED = 1u << 0u, PROM_REDUCTION_FLAG_FORCE_COMPOSED = 1u << 1u };

/* reactor_api.h:426-452 */
enum {
  PROM_REDUCTION_DETAIL_INVALID_REQUEST = -6801,
  PROM_REDUCTION_DETAIL_NULL_INPUT = -6802,
  PROM_REDUCTION_DETAIL_NULL_OUTPUT = -6803,
  PROM_REDUCTION_DETAIL_ZERO_ROW_COUNT = -6804,
  PROM_REDUCTION_DETAIL_ZERO_ROW_WIDTH = -6805,
  PROM_REDUCTION_DETAIL_UNSUPPORTED_OPERATION = -6806,
  PROM_REDUCTION_DETAIL_INVALID_FINALIZATION = -6807,
  PROM_REDUCTION_DETAIL_SIZE_OVERFLOW = -6808,
  PROM_REDUCTION_DETAIL_INPUT_SIZE_MISMATCH = -6809,
  PROM_REDUCTION_DETAIL_OUTPUT_SIZE_MISMATCH = -6810,
  PROM_REDUCTION_DETAIL_ROW_LIMIT = -6811,
  PROM_REDUCTION_DETAIL_WIDTH_LIMIT = -6812,
  PROM_REDUCTION_DETAIL_ELEMENT_LIMIT = -6813,
  PROM_REDUCTION_DETAIL_NONFINITE_INPUT = -6814,
  PROM_REDUCTION_DETAIL_UNSUPPORTED_STRATEGY = -6815,
  PROM_REDUCTION_DETAIL_MALFORMED_PLAN = -6816,
  PROM_REDUCTION_DETAIL_TEMPORARY_UNDERSIZED = -6817,
  PROM_REDUCTION_DETAIL_RESOURCE_CREATE_FAILED = -6818,
  PROM_REDUCTION_DETAIL_PIPELINE_CREATE_FAILED = -6819,
  PROM_REDUCTION_DETAIL_COMMAND_RECORD_FAILED = -6820,
  PROM_REDUCTION_DETAIL_QUEUE_SUBMIT_FAILED = -6821,
  PROM_REDUCTION_DETAIL_COMPLETION_UNCERTAIN = -6822,
  PROM_REDUCTION_DETAIL_QUERY_FAILED = -6823,
  PROM_REDUCTION_DETAIL_READBACK_FAILED = -6824,
  PROM_REDUCTION_DETAIL_RUNTIME_UNAVAILABLE = -6825,
};

/* reactor_api.h:456-470 */
enum {
  PROM_SOFTMAX_DETAIL_INVALID_REQUEST = -6851,
  PROM_SOFTMAX_DETAIL_NULL_INPUT = -6852,
  PROM_SOFTMAX_DETAIL_NULL_OUTPUT = -6853,
  PROM_SOFTMAX_DETAIL_COUNT_MISMATCH = -6854,
  PROM_SOFTMAX_DETAIL_SIZE_OVERFLOW = -6855,
  PROM_SOFTMAX_DETAIL_ROW_LIMIT = -6856,
  PROM_SOFTMAX_DETAIL_WIDTH_LIMIT = -6857,
  PROM_SOFTMAX_DETAIL_ELEMENT_LIMIT = -6858,
  PROM_SOFTMAX_DETAIL_PARTIAL_ALIAS = -6859,
  PROM_SOFTMAX_DETAIL_NONFINITE_INPUT = -6860,
  PROM_SOFTMAX_DETAIL_RUNTIME_UNAVAILABLE = -6861,
  PROM_SOFTMAX_DETAIL_SUBGROUP_UNSUPPORTED = -6862,
  PROM_SOFTMAX_DETAIL_TOPOLOGY_UNSUPPORTED = -6863,
};

/* reactor_api.h:472-490 (plan vocabulary; kept so plans serialise identically) */
enum {
  PROM_REDUCTION_SHADER_ROW_SUM = 16u,
  PROM_REDUCTION_SHADER_ROW_MAX = 17u,
  PROM_REDUCTION_SHADER_SOFTMAX_EXP_SUM = 18u,
  PROM_REDUCTION_SHADER_SOFTMAX_NORMALIZE = 19u,
  PROM_REDUCTION_SHADER_SOFTMAX_FUSED = 20u,
  PROM_REDUCTION_SHADER_ROW_SUM_PACKED_SHORT = 21u,
  PROM_REDUCTION_SHADER_SOFTMAX_PACKED_SHORT = 22u,
};
enum {
  PROM_REDUCTION_IMPLEMENTATION_ROW_SUM = 1001u,
  PROM_REDUCTION_IMPLEMENTATION_ROW_MAX = 1002u,
  PROM_REDUCTION_IMPLEMENTATION_SOFTMAX_EXP_SUM = 1003u,
  PROM_REDUCTION_IMPLEMENTATION_SOFTMAX_NORMALIZE = 1004u,
  PROM_REDUCTION_IMPLEMENTATION_SOFTMAX_FUSED = 1005u,
  PROM_REDUCTION_IMPLEMENTATION_ROW_SUM_PACKED_SHORT = 1006u,
  PROM_REDUCTION_IMPLEMENTATION_SOFTMAX_PACKED_SHORT = 1007u,
};

/* reactor_api.h:492-510 -- the reference admission envelope.  The reference
   entry points (..._reduction, ..._reduction_plan, ..._row_wise_softmax) keep
   it unchanged; the NEW ..._reduction_v2 admits the lifted envelope below. */
#define PROM_REDUCTION_MAX_STAGES 8u
#define PROM_REDUCTION_MAX_ROWS 1024u
#define PROM_REDUCTION_MAX_ELEMENTS_PER_ROW 1048576u
#define PROM_REDUCTION_MAX_TOTAL_ELEMENTS 16777216u
#define PROM_REDUCTION_LOCAL_SIZE 256u
#define PROM_REDUCTION_ELEMENTS_PER_PARTIAL 1024u
#define PROM_REDUCTION_SINGLE_STAGE_THRESHOLD 1024u
#define PROM_REDUCTION_FORCE_FUSED_MAX_ELEMENTS_PER_ROW 1056u
#define PROM_REDUCTION_PACKED_SHORT_WIDTH_MAX 128u
#define PROM_REDUCTION_PACKED_SHORT_SUM_MIN_ROWS 512u
#define PROM_REDUCTION_PACKED_SHORT_SUM_WIDE_MIN_ROWS 1024u
#define PROM_REDUCTION_PACKED_SHORT_ROWS_PER_GROUP 8u
#define PROM_REDUCTION_PACKED_SHORT_LANES_PER_ROW 32u
#define PROM_ROW_WISE_SOFTMAX_MAX_ROWS PROM_REDUCTION_MAX_ROWS
#define PROM_ROW_WISE_SOFTMAX_MAX_ELEMENTS_PER_ROW PROM_REDUCTION_FORCE_FUSED_MAX_ELEMENTS_PER_ROW
#define PROM_ROW_WISE_SOFTMAX_MAX_TOTAL_ELEMENTS PROM_REDUCTION_MAX_TOTAL_ELEMENTS

/* NEW: lifted envelope of ..._reduction_v2 (rows fit uint32; 4 Gi elements = 16 GiB
   of fp32, well inside one MI355X's 288 GB). */
#define PROM_REDUCTION_V2_MAX_ROWS 0xFFFFFFFFu
#define PROM_REDUCTION_V2_MAX_ELEMENTS_PER_ROW 1048576u
#define PROM_REDUCTION_V2_MAX_TOTAL_ELEMENTS 4294967296ull

/* reactor_api.h:512-539 */
typedef struct PrometheusRowWiseSoftmaxRequest {
  uint32_t struct_size;
  const float* input;
  float* output;
  uint32_t row_count;
  uint32_t elements_per_row;
  uint64_t input_element_count;
  uint64_t output_element_count;
} PrometheusRowWiseSoftmaxRequest;

typedef struct PrometheusRowWiseSoftmaxResult {
  uint32_t struct_size;
  uint32_t stage;
  int32_t detail_code;
  uint32_t output_written;
  uint32_t physical_dispatch_count;
  uint32_t physical_submission_count;
  uint32_t gpu_timestamp_valid;
  uint64_t gpu_duration_ns;
  uint64_t end_to_end_ns;
  uint64_t first_nonfinite_index;
} PrometheusRowWiseSoftmaxResult;

/* reactor_api.h:541-552 */
typedef struct PrometheusReductionRequest {
  uint32_t struct_size;
  const float* input;
  float* output;
  uint32_t row_count;
  uint32_t elements_per_row;
  uint64_t input_element_count;
  uint64_t output_element_count;
  uint32_t operation;
  uint32_t finalization;
  uint32_t flags;
} PrometheusReductionRequest;

/* reactor_api.h:554-565 */
typedef struct PrometheusReductionStageDispatch {
  uint32_t stage_role;
  uint32_t shader_id;
  uint32_t implementation_id;
  uint32_t groups_x;
  uint32_t groups_y;
  uint32_t groups_z;
  uint32_t input_elements_per_row;
  uint32_t output_partials_per_row;
  uint32_t temporary_role;
  uint64_t temporary_bytes_written;
} PrometheusReductionStageDispatch;

/* reactor_api.h:567-581 */
typedef struct PrometheusReductionPlan {
  uint32_t struct_size;
  uint32_t operation;
  uint32_t row_count;
  uint32_t elements_per_row;
  uint32_t strategy;
  uint32_t local_size;
  uint32_t elements_per_partial;
  uint32_t partial_count;
  uint32_t stage_count;
  uint32_t temporary_alignment_bytes;
  uint64_t temporary_bytes;
  uint64_t replay_id;
  PrometheusReductionStageDispatch stages[PROM_REDUCTION_MAX_STAGES];
} PrometheusReductionPlan;

/* reactor_api.h:583-598 */
typedef struct PrometheusReductionExecutionResult {
  uint32_t struct_size;
  uint32_t stage;
  int32_t detail_code;
  uint64_t logical_request_id;
  uint32_t physical_slot_id;
  uint32_t physical_slot_generation;
  uint32_t physical_slot_recyclable;
  uint32_t gpu_timestamp_valid;
  uint64_t gpu_duration_ns;
  uint64_t end_to_end_ns;
  uint64_t first_nonfinite_index;
  uint32_t validation_error_count_before;
  uint32_t validation_error_count_after;
  PrometheusReductionPlan plan;
} PrometheusReductionExecutionResult;

/* reactor_api.h:600-664.  Diagnostics of the runtime's row reductions, and
   the benchmark request/result: warmup + measured executions of one
   reduction, timing percentiles and a correctness verdict. */
typedef struct PrometheusReductionDiagnostics {
  uint32_t struct_size;
  uint32_t initialized;
  uint32_t production_enabled;
  uint32_t experimental_enabled;
  uint32_t configured_ring_depth;
  uint32_t physical_slot_count;
  uint32_t acquire_cursor;
  uint32_t outstanding_slots;
  uint32_t quarantined_slots;
  uint64_t next_logical_request_id;
  uint64_t total_requests;
  uint64_t successful_requests;
  uint64_t logical_failure_count;
  uint64_t physical_recycle_count;
  uint64_t quarantine_count;
  uint64_t reap_count;
  uint64_t pipeline_create_count;
  uint64_t descriptor_update_count;
  uint64_t command_record_count;
  uint64_t queue_submit_count;
  uint64_t buffer_allocation_count;
  uint64_t buffer_reuse_count;
  uint64_t temporary_capacity_bytes;
  uint64_t last_replay_id;
  uint64_t last_gpu_duration_ns;
  uint64_t last_end_to_end_ns;
  uint32_t last_stage_count;
  uint32_t last_physical_slot_id;
  uint32_t last_physical_slot_generation;
  int32_t last_detail_code;
  uint32_t validation_enabled;
  uint32_t validation_error_count;
} PrometheusReductionDiagnostics;

typedef struct PrometheusReductionBenchmarkRequest {
  uint32_t struct_size;
  PrometheusReductionRequest reduction;
  uint32_t warmup_iterations;
  uint32_t measured_iterations;
} PrometheusReductionBenchmarkRequest;

typedef struct PrometheusReductionBenchmarkResult {
  uint32_t struct_size;
  uint32_t completed_iterations;
  uint32_t correctness_passed;
  uint32_t validation_passed;
  uint32_t device_lost;
  uint32_t stage_count;
  uint64_t temporary_bytes;
  uint64_t replay_id;
  uint64_t gpu_min_ns;
  uint64_t gpu_median_ns;
  uint64_t gpu_max_ns;
  uint64_t end_to_end_min_ns;
  uint64_t end_to_end_median_ns;
  uint64_t end_to_end_max_ns;
  uint32_t first_mismatch_row;
  uint32_t first_mismatch_column;
  float first_expected;
  float first_actual;
  float first_absolute_error;
  float first_relative_error;
  int32_t detail_code;
} PrometheusReductionBenchmarkResult;

/* reactor_api.h:1582-1586 */
typedef struct PrometheusCaps {
  uint32_t available;
  uint32_t backend_type;
  uint32_t reason_code;
} PrometheusCaps;

/* reactor_api.h:1596-1606 (filled from the HIP device; api_version = HIP runtime version). */
typedef struct PrometheusVulkanDeviceDiagnostics {
  char device_name[256];
  uint32_t vendor_id;
  uint32_t device_id;
  uint32_t device_type;
  uint32_t driver_version;
  uint32_t api_version;
  uint32_t software_vulkan;
  uint32_t compute_queue_family;
  uint32_t transfer_queue_family;
} PrometheusVulkanDeviceDiagnostics;

/* reactor_api.h:1751-1769.  struct_size gates the tail field. */
typedef struct PrometheusReactorConfig {
  uint32_t struct_size;
  uint32_t test_flags;
  uint32_t p15_shadow_disabled;
  uint32_t async_test_flags;
  uint32_t batch_ring_depth;
  uint32_t reduction_test_flags;
  uint32_t reduction_ring_depth;
  const char* shader_package_root;
} PrometheusReactorConfig;

/* reactor_api.h:1781-1825 */
typedef struct PrometheusGemma4E2BM1InputRmsNormRequest {
  uint32_t struct_size;
  const float* input;
  const float* weight;
  float* output;
  float* inv_rms_output;
  uint64_t input_element_count;
  uint64_t weight_element_count;
  uint64_t output_element_count;
  uint64_t inv_rms_output_element_count;
  uint32_t tokens;
  uint32_t model_width;
  uint32_t input_row_stride;
  float epsilon;
  uint64_t input_generation;
  uint64_t weight_generation;
  uint64_t exact_source_hash;
} PrometheusGemma4E2BM1InputRmsNormRequest;

typedef struct PrometheusGemma4E2BM1InputRmsNormResult {
  uint32_t struct_size;
  uint32_t stage;
  int32_t detail_code;
  uint32_t output_written;
  uint32_t matched_input;
  uint64_t input_hash;
  uint64_t weight_hash;
  uint64_t output_hash;
  uint64_t inv_rms_hash;
  uint32_t submit_count;
  uint32_t final_readback_count;
  uint32_t no_product_intermediate_readback_change;
  uint32_t reserved0;
  uint64_t retained_bytes;
  uint64_t buffer_allocation_count;
  uint64_t buffer_reuse_count;
  uint64_t descriptor_update_count;
  uint64_t pipeline_create_count;
  uint64_t command_buffer_reuse_count;
  uint64_t reduction_gpu_ns;
  uint64_t final_reduction_gpu_ns;
  uint64_t inv_rms_gpu_ns;
  uint64_t apply_gpu_ns;
  uint64_t end_to_end_ns;
} PrometheusGemma4E2BM1InputRmsNormResult;

/* RMSNorm detail codes: internal/prometheus/native/reactor_vulkan.h:1870-1888 (subset).
   The Gemma entry keeps the reference's admission envelope
   (tokens <= 1024, width <= 4096: reactor_vulkan.h:10-11); the generic
   ..._rmsnorm entry lifts it. */
enum {
  PROM_M46_DETAIL_INVALID_REQUEST = -7401,
  PROM_M46_DETAIL_SHAPE = -7403,
  PROM_M46_DETAIL_STRIDE = -7404,
  PROM_M46_DETAIL_STALE_WEIGHT_GENERATION = -7406,
  PROM_M46_DETAIL_EPSILON = -7407,
  PROM_M46_DETAIL_SIZE_OVERFLOW = -7409,
  PROM_M46_DETAIL_RESOURCE = -7411,
  PROM_M46_DETAIL_READBACK = -7416,
  PROM_M46_DETAIL_NONFINITE_INPUT = -7418,
};
#define PROM_M42_MAX_TOKENS 1024u
#define PROM_M42_MAX_MODEL_WIDTH 4096u

/* NEW: generic RMSNorm request (no generation/hash bookkeeping). */
typedef struct PrometheusRmsNormRequest {
  uint32_t struct_size;
  const float* input;     /* [tokens, input_row_stride] */
  const float* weight;    /* [width] */
  float* output;          /* [tokens, width] */
  float* inv_rms_output;  /* [tokens], may be NULL */
  uint32_t tokens;
  uint32_t width;
  uint32_t input_row_stride;
  float epsilon;
} PrometheusRmsNormRequest;

typedef struct PrometheusRmsNormResult {
  uint32_t struct_size;
  uint32_t stage;
  int32_t detail_code;
  uint32_t output_written;
  uint64_t gpu_duration_ns;
  uint64_t end_to_end_ns;
} PrometheusRmsNormResult;

/* ------------------------------------------------------------------------ */
/* Reference entry points (reactor_api.h:2557-2699)                          */
/* ------------------------------------------------------------------------ */

/* reactor_api.h:2557 -- returns PROM_REACTOR_ABI_V1. */
PROM_REACTOR_API uint32_t prometheus_reactor_abi_version(void);
/* reactor_api.h:2558 -- config may be NULL (defaults). */
PROM_REACTOR_API int prometheus_reactor_runtime_create(void* config, void** out_handle);
/* reactor_api.h:2559 -- second destroy of a handle returns PROM_INVALID_HANDLE. */
PROM_REACTOR_API int prometheus_reactor_runtime_destroy(void* handle);
/* reactor_api.h:2560 -- available=1, backend 2 on a HIP device; else
   available=0, backend UNKNOWN, reason VULKAN_UNAVAILABLE (no device). */
PROM_REACTOR_API int prometheus_reactor_runtime_probe(void* handle, PrometheusCaps* out_caps);
/* reactor_api.h:2822-2825; reactor_api.c:801-812 -- backward-compatible
   aliases of create / destroy / probe from the reference's earlier contract
   drafts; each behaves exactly as the entry it names. */
PROM_REACTOR_API int prometheus_runtime_create(void* config, void** out_handle);
PROM_REACTOR_API int prometheus_runtime_destroy(void* handle);
PROM_REACTOR_API int prometheus_runtime_probe(void* handle, PrometheusCaps* out_caps);
/* reactor_api.h:2561-2562 */
PROM_REACTOR_API int prometheus_reactor_runtime_vulkan_device_diagnostics(void* handle,
                                                                           PrometheusVulkanDeviceDiagnostics* out_diag);
/* reactor_api.h:2587-2595 -- C[m,n] = A[m,k] @ B[k,n], row-major fp32,
   synchronous, host pointers.  Validation order and codes follow
   reactor_sgemm.cpp:4152-4191 (invalid handle -> INIT/PROM_INVALID_HANDLE;
   NULL operand -> TRANSFER_IN/PROM_ERROR; zero dimension -> INIT/PROM_ERROR;
   no device -> INIT).  The reference rejects m*n*k >= 2^32 with
   PROM_DETAIL_SIZE_OVERFLOW, which excludes 4096^3; here the limit is that
   each of m*k, k*n and m*n is below 2^32 elements (16 GiB of fp32). */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm(void* handle, const float* a, const float* b, float* c,
                                                      uint32_t m, uint32_t n, uint32_t k, uint32_t* out_stage,
                                                      int* out_detail_code);
/* reactor_api.h:2671-2672 -- reference planner, reference envelope. */
PROM_REACTOR_API int prometheus_reactor_reduction_plan(const PrometheusReductionRequest* request,
                                                        PrometheusReductionPlan* out_plan);
/* reactor_api.h:2673-2675 -- reference envelope (rows <= 1024, total <= 2^24). */
PROM_REACTOR_API int prometheus_reactor_runtime_reduction(void* handle, const PrometheusReductionRequest* request,
                                                          PrometheusReductionExecutionResult* out_result);
/* reactor_api.h:2676-2677.  Counts the reduction, reduction_v2 and
   row_wise_softmax calls of this runtime (one stream: ring depth and slot
   count 1); out_diag NULL -> PROM_ERROR, unknown handle -> PROM_INVALID_HANDLE. */
PROM_REACTOR_API int prometheus_reactor_runtime_reduction_diagnostics(void* handle,
                                                                      PrometheusReductionDiagnostics* out_diag);
/* reactor_api.h:2678-2681; reactor_vulkan_fused_reduction.c:1122-1201.
   measured_iterations in 1..10000 (else INVALID_REQUEST); runs warmup +
   measured executions of `reduction` (reference envelope), reports the
   min/median/max GPU and end-to-end times, and checks the last output
   against a binary64 evaluation of the same reduction on the device with the
   reference's tolerances (softmax abs 2e-5 or rel 2e-4, values >= -2e-7 and
   row sums within 3e-4; sum abs 2e-5 * width or rel 2e-5; max exact); a
   mismatch reports its first position and READBACK_FAILED. */
PROM_REACTOR_API int prometheus_reactor_runtime_reduction_benchmark(void* handle,
                                                                    const PrometheusReductionBenchmarkRequest* request,
                                                                    PrometheusReductionBenchmarkResult* out_result);
/* reactor_api.h:2682-2685 -- rows <= 1024, width <= 1056, exact in-place allowed. */
PROM_REACTOR_API int prometheus_reactor_runtime_row_wise_softmax(void* handle,
                                                                 const PrometheusRowWiseSoftmaxRequest* request,
                                                                 PrometheusRowWiseSoftmaxResult* out_result);
/* reactor_api.h:2686-2689; reactor_api.c:250-359.  Gemma-4-E2B M1 family
   (this and the five entries below) follows the reference's call chain:
   request validation (INIT / -7401) -> weight commit, which requires a
   weight_generation strictly greater than the runtime's last committed one
   (PrometheusRmsNorm.concept:199-213; stale -> TRANSFER_IN / -7406) -> shape,
   epsilon and finiteness checks (-7401 / -7418) -> execution.  Success reports
   stage 0 and detail 0, as reactor_concept_rmsnorm.cpp:110-146 leaves them.
   RMSNorm: y = x * inv * w, inv = 1/sqrt(sum(x^2)/W + eps) (sum in binary64). */
PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm(
    void* handle, const PrometheusGemma4E2BM1InputRmsNormRequest* request,
    PrometheusGemma4E2BM1InputRmsNormResult* out_result);

/* ------------------------------------------------------------------------ */
/* NEW entry points (same conventions; no reference counterpart)             */
/* ------------------------------------------------------------------------ */

/* HIP device identity: name, gfx arch, CU count, clock, HBM bytes. */
typedef struct PrometheusHipDeviceDiagnostics {
  uint32_t struct_size;
  char device_name[256];
  char gcn_arch_name[64];
  uint32_t compute_units;
  uint32_t clock_khz;
  uint32_t memory_clock_khz;
  uint32_t memory_bus_width;
  uint64_t total_global_mem;
  uint32_t lds_bytes_per_workgroup;
  uint32_t wavefront_size;
  int32_t hip_runtime_version;
  int32_t device_ordinal;
  /* Device allocations made so far by the library's grow-only staging
     buffers (operand staging, block workspaces, split-K partials, padded
     copies), and the bytes they hold now.  Written only when struct_size
     covers them (a caller's struct that ends at device_ordinal is accepted). */
  uint64_t staging_allocations;
  uint64_t staging_bytes;
} PrometheusHipDeviceDiagnostics;
PROM_REACTOR_API int prometheus_reactor_runtime_hip_device_diagnostics(void* handle,
                                                                        PrometheusHipDeviceDiagnostics* out_diag);

/* The reduction entry of the reference with the admission envelope lifted to
   PROM_REDUCTION_V2_* (C3's [8192, 4096] does not fit the reference's). */
PROM_REACTOR_API int prometheus_reactor_runtime_reduction_v2(void* handle, const PrometheusReductionRequest* request,
                                                             PrometheusReductionExecutionResult* out_result);
/* Generic RMSNorm: y = x * rsqrt(mean(x^2) + eps) * w, inv_rms optional. */
PROM_REACTOR_API int prometheus_reactor_runtime_rmsnorm(void* handle, const PrometheusRmsNormRequest* request,
                                                        PrometheusRmsNormResult* out_result);
/* bf16 GEMM: A[m,k], B[k,n] as bf16 bit patterns (uint16), C fp32, row-major,
   fp32 accumulate; synchronous, host pointers. */
PROM_REACTOR_API int prometheus_reactor_runtime_gemm_bf16(void* handle, const uint16_t* a, const uint16_t* b, float* c,
                                                          uint32_t m, uint32_t n, uint32_t k, uint32_t* out_stage,
                                                          int* out_detail_code);

/* Device-resident operation.  Buffers come from ..._device_alloc (or any
   device pointer of the same HIP device); work is queued on the runtime's
   single stream and these calls return without waiting. */
PROM_REACTOR_API int prometheus_reactor_runtime_device_alloc(void* handle, uint64_t bytes, void** out_device_ptr);
PROM_REACTOR_API int prometheus_reactor_runtime_device_free(void* handle, void* device_ptr);
PROM_REACTOR_API int prometheus_reactor_runtime_device_upload(void* handle, void* device_dst, const void* host_src,
                                                              uint64_t bytes);
PROM_REACTOR_API int prometheus_reactor_runtime_device_download(void* handle, void* host_dst, const void* device_src,
                                                                uint64_t bytes);
PROM_REACTOR_API int prometheus_reactor_runtime_synchronize(void* handle);
/* Event timing on the runtime stream: record into one of 64 slots; elapsed
   waits for the end event. */
PROM_REACTOR_API int prometheus_reactor_runtime_event_record(void* handle, uint32_t slot);
PROM_REACTOR_API int prometheus_reactor_runtime_event_elapsed_ms(void* handle, uint32_t start_slot, uint32_t end_slot,
                                                                 float* out_ms);

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_device(void* handle, const float* a, const float* b, float* c,
                                                             uint32_t m, uint32_t n, uint32_t k, uint32_t* out_stage,
                                                             int* out_detail_code);
/* No counterpart in the reference.  For callers that cannot allocate device
   memory (tight serving loops, harnesses that forbid hipMalloc): the product
   of ..._sgemm_device, with the same plan and bit-identical results, that
   allocates nothing.  The scratch the plan needs beyond A, B and C (the
   split-K partial slices, rounded up to 256 bytes, followed by the
   zero-padded copies of A and B when the plan repacks unaligned operands)
   goes to a static device array of PROM_SGEMM_NOALLOC_SCRATCH_BYTES (64 MiB,
   one per GPU, held until the process ends) instead of runtime-allocated
   staging.  A plan whose PrometheusSgemmPlanInfo.scratch_bytes (exactly that
   sum) exceeds the array is rejected before anything is queued: PROM_ERROR,
   stage TRANSFER_IN, PROM_DETAIL_SCRATCH_LIMIT, C untouched.  The work is
   queued on the library's own stream, like every entry here, so a HIP graph
   capture that a caller runs on a stream of its own does not record it.
   Every call on a GPU shares that GPU's array and leaves the last call's
   contents in it (nothing in it needs to start at zero: each slice and copy
   overwrites its part); calls are ordered on that one stream, and two
   processes, or two library copies, running this entry on one GPU race on
   the array. */
#define PROM_SGEMM_NOALLOC_SCRATCH_BYTES (64ull << 20)
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_device_noalloc(void* handle, const float* a, const float* b,
                                                                     float* c, uint32_t m, uint32_t n, uint32_t k,
                                                                     uint32_t* out_stage, int* out_detail_code);
/* No counterpart in the reference: ..._sgemm_device with a caller-chosen
   kernel variant instead of the plan model's, for tuning and per-variant
   tests.  tile: 0 = 128x256, 1 = 128x128, 2 = 64x128 (register-staged
   loads), 3 = 128x256, 4 = 128x128 (HBM -> LDS loads, K tile 16: k and each
   K slice multiples of 16), 5 = 64x64 with K tile 32, 6 = 64x64 with K tile
   64 (HBM -> LDS loads, the K tile split between two wave groups of the
   workgroup; any k).  Tiles 3-6 need k and n multiples of 4 and 16-byte
   aligned operands; k_slices 1..16 (split-K with a reduce launch when > 1).
   A variant that cannot run the shape returns PROM_ERROR, stage INIT,
   PROM_DETAIL_INVALID_ARGUMENT; otherwise the device entry's statuses. */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_device_variant(void* handle, const float* a, const float* b,
                                                                     float* c, uint32_t m, uint32_t n, uint32_t k,
                                                                     uint32_t tile, uint32_t k_slices,
                                                                     uint32_t* out_stage, int* out_detail_code);
/* No counterpart in the reference (its attention exists only inside the
   Z-Image block shaders, main_transformer_joint_attention_streaming.sdslv):
   the bf16 flash attention of the DiT block on device pointers, for its own
   parity tests and tuning.  O = softmax(Q K^T / sqrt(128)) V per head, full
   attention; q, k, v, o are bf16 [tokens, ld] with head h at column 128 h,
   16-byte aligned, ld a multiple of 8, >= 128 * heads and < 2^24, tokens *
   ld * 2 < 2^31.  variant 0 = the block's kernel (DMA-fed), 1 = the
   register-staged kernel.  Invalid arguments: PROM_ERROR, stage INIT,
   PROM_DETAIL_INVALID_ARGUMENT.  Queued on the runtime's stream. */
PROM_REACTOR_API int prometheus_reactor_runtime_attention_bf16_device(void* handle, const uint16_t* q,
                                                                      const uint16_t* k, const uint16_t* v,
                                                                      uint16_t* o, uint32_t tokens, uint32_t heads,
                                                                      uint32_t ld, uint32_t variant,
                                                                      uint32_t* out_stage, int* out_detail_code);
/* The SGEMM launch plan that ..._sgemm and ..._sgemm_device queue for a
   contiguous row-major product with 16-byte-aligned operands.  It is a pure
   function of the shape and needs neither a runtime nor a device.  The
   reference reports its own choice (occupancy variant, geometry) through its
   judgment engine, reactor_judgment_engine.c:895-948.
   Admission is the device entries' rule: any dimension above 2^31 - 1, or
   m*k, k*n or m*n at or above 2^32, returns PROM_ERROR with detail_code
   PROM_DETAIL_SIZE_OVERFLOW; a zero dimension returns PROM_ERROR with detail
   PROM_ERROR.  On success detail_code is the path detail the device entry
   reports (PROM_DETAIL_PATH_HIP_MFMA_F32 or _GEMV_F32).  products is 0 for
   the GEMV, else 1, or 2 when the rows past the last full 128-row tile row
   (rows head_rows..m-1) run as a second product. */
typedef struct PrometheusSgemmPlanInfo {
  uint32_t struct_size;
  int32_t detail_code;
  uint32_t products;
  uint32_t head_rows;
  uint32_t tile_m[2];       /* macro tile of each product */
  uint32_t tile_n[2];
  uint32_t direct_to_lds[2]; /* 1: tiles go HBM -> LDS by buffer_load ... lds */
  uint32_t k_slices[2];     /* split-K slices (1: no split) */
  uint32_t k_slice_len[2];
  uint32_t launches;        /* kernel launches queued (padding copies, GEMMs, split-K reduces) */
  uint32_t repacked;        /* 1: A and B are first copied to zero-padded buffers with 16-byte rows */
  uint64_t partial_bytes;   /* split-K partial buffer the plan writes */
  double estimated_us;      /* the plan model's estimate */
  uint64_t repack_bytes;    /* the padded copies of A and B */
  /* Scratch of ..._sgemm_device_noalloc: partial_bytes rounded up to 256,
     plus repack_bytes.  Written only when struct_size covers it (a caller's
     struct that ends at repack_bytes is still accepted). */
  uint64_t scratch_bytes;
} PrometheusSgemmPlanInfo;
PROM_REACTOR_API int prometheus_reactor_sgemm_plan(uint32_t m, uint32_t n, uint32_t k,
                                                   PrometheusSgemmPlanInfo* out_plan);
PROM_REACTOR_API int prometheus_reactor_runtime_gemm_bf16_device(void* handle, const uint16_t* a, const uint16_t* b,
                                                                 float* c, uint32_t m, uint32_t n, uint32_t k,
                                                                 uint32_t* out_stage, int* out_detail_code);
/* operation as PrometheusReductionRequest; softmax writes rows*width, sum/max rows. */
PROM_REACTOR_API int prometheus_reactor_runtime_reduction_device(void* handle, const float* input, float* output,
                                                                 uint32_t rows, uint32_t width, uint32_t operation,
                                                                 uint32_t* out_stage, int* out_detail_code);
PROM_REACTOR_API int prometheus_reactor_runtime_rmsnorm_device(void* handle, const float* input, const float* weight,
                                                               float* output, float* inv_rms, uint32_t tokens,
                                                               uint32_t width, uint32_t input_row_stride, float epsilon,
                                                               uint32_t* out_stage, int* out_detail_code);

/* ------------------------------------------------------------------------ */
/* NEW: transformer-block dispatch.  The reference's block ABI is closed and   */
/* shape-locked (Z-Image main transformer, reactor_api.h:800-1244, 2713-2821); */
/* these entries carry explicit shape fields instead.  Weights are [in, out]   */
/* row-major as canonicalLinear (zimage/canonical_reference.go:156-175).       */
/* ------------------------------------------------------------------------ */

enum {
  PROM_BLOCK_DETAIL_INVALID_REQUEST = -7501,
  PROM_BLOCK_DETAIL_SHAPE = -7502,
  PROM_BLOCK_DETAIL_UNSUPPORTED = -7503,
};

/* Gemma-style decoder layer in fp32:
     n1 = RMSNorm(x; attn_norm_weight, eps)          y = x * rsqrt(mean(x^2)+eps) * w
     q,k,v = n1 @ w_qkv   (columns: q_heads*head_dim | head_dim | head_dim)
     rotate-half RoPE on q and k at positions position_offset + t, base rope_base
     attention: softmax(q k^T / sqrt(head_dim)) v, causal, every query head on KV head 0
     h = x + attn @ w_o
     n2 = RMSNorm(h; ffn_norm_weight, eps)
     g|u = n2 @ w_gate_up (columns: ffn_hidden gate | ffn_hidden up)
     out = h + (gelu_tanh(g) * u) @ w_down
   kv_heads must be 1 (multi-query attention, as Gemma-2B). */
typedef struct PrometheusDecoderLayerF32Request {
  uint32_t struct_size;
  uint32_t tokens;
  uint32_t hidden;
  uint32_t q_heads;
  uint32_t kv_heads;
  uint32_t head_dim;
  uint32_t ffn_hidden;
  uint32_t position_offset;
  float rms_epsilon;
  float rope_base;
  const float* input;            /* [tokens, hidden] */
  const float* attn_norm_weight; /* [hidden] */
  const float* w_qkv;            /* [hidden, (q_heads + 2*kv_heads) * head_dim] */
  const float* w_o;              /* [q_heads * head_dim, hidden] */
  const float* ffn_norm_weight;  /* [hidden] */
  const float* w_gate_up;        /* [hidden, 2 * ffn_hidden] */
  const float* w_down;           /* [ffn_hidden, hidden] */
  float* output;                 /* [tokens, hidden] */
} PrometheusDecoderLayerF32Request;

/* Z-Image-style single-stream DiT block in bf16;
   the per-stage definition follows zimage/canonical_reference.go:315-480 and
   tools/python/zimage/zimage_main_transformer_canonical.py:178-277:
     m = condition @ w_adaln + b_adaln  -> scaleA = 1+m0, gateA = tanh(m1),
                                          scaleM = 1+m2, gateM = tanh(m3)
     a = RMSNorm(x; attn_norm1) * scaleA          (eps rms_epsilon)
     q|k|v = a @ w_qkv;  q,k = per-head RMSNorm(q_norm / k_norm)
     3-axis interleaved-pair RoPE on q,k (axes rope_axes, theta rope_theta,
     per-token coordinates [frame,row,col])
     o = softmax(q k^T / sqrt(head_dim)) v  (full attention, per head)
     r = x + gateA * RMSNorm(o @ w_out; attn_norm2)
     f = RMSNorm(r; ffn_norm1) * scaleM
     out = r + gateM * RMSNorm((silu(f @ w1) * (f @ w3)) @ w2; ffn_norm2)
   GEMM operands are bf16 (weights as given; activations rounded to nearest
   even), accumulation and norms fp32; x and out are fp32. */
typedef struct PrometheusDitBlockBf16Request {
  uint32_t struct_size;
  uint32_t tokens;
  uint32_t hidden;
  uint32_t heads;
  uint32_t head_dim;
  uint32_t ffn_hidden;
  uint32_t cond_dim;
  uint32_t rope_axes[3];
  float rope_theta;
  float rms_epsilon;
  const float* input;        /* [tokens, hidden] fp32 */
  const float* coordinates;  /* [tokens, 3] fp32 */
  const float* condition;    /* [cond_dim] fp32 */
  const uint16_t* w_adaln;   /* bf16 [cond_dim, 4*hidden] */
  const float* b_adaln;      /* [4*hidden] */
  const float* attn_norm1;   /* [hidden] */
  const float* attn_norm2;   /* [hidden] */
  const float* ffn_norm1;    /* [hidden] */
  const float* ffn_norm2;    /* [hidden] */
  const float* q_norm;       /* [head_dim] */
  const float* k_norm;       /* [head_dim] */
  const uint16_t* w_qkv;     /* bf16 [hidden, 3*hidden] */
  const uint16_t* w_out;     /* bf16 [hidden, hidden] */
  const uint16_t* w_13;      /* bf16 [hidden, 2*ffn_hidden]: w1 columns then w3 columns */
  const uint16_t* w_2;       /* bf16 [ffn_hidden, hidden] */
  float* output;             /* [tokens, hidden] fp32 */
} PrometheusDitBlockBf16Request;

typedef struct PrometheusBlockResult {
  uint32_t struct_size;
  uint32_t stage;
  int32_t detail_code;
  uint32_t output_written;
  uint32_t kernel_launches;
  uint32_t reserved0;
  uint64_t gpu_duration_ns;
  uint64_t end_to_end_ns;
  uint64_t workspace_bytes;
} PrometheusBlockResult;

/* Host-pointer forms copy weights and activations in and the output out
   (synchronous).  _device forms take device pointers for every array, enqueue
   on the runtime stream and return; the workspace is owned by the runtime's
   device context (grow-only, reused across calls). */
PROM_REACTOR_API int prometheus_reactor_runtime_decoder_layer_f32(void* handle,
                                                                  const PrometheusDecoderLayerF32Request* request,
                                                                  PrometheusBlockResult* out_result);
PROM_REACTOR_API int prometheus_reactor_runtime_decoder_layer_f32_device(
    void* handle, const PrometheusDecoderLayerF32Request* request, PrometheusBlockResult* out_result);
PROM_REACTOR_API int prometheus_reactor_runtime_dit_block_bf16(void* handle, const PrometheusDitBlockBf16Request* request,
                                                               PrometheusBlockResult* out_result);
PROM_REACTOR_API int prometheus_reactor_runtime_dit_block_bf16_device(void* handle,
                                                                      const PrometheusDitBlockBf16Request* request,
                                                                      PrometheusBlockResult* out_result);

/* ------------------------------------------------------------------------ */
/* Asynchronous and batched SGEMM (reference lifecycle, HIP execution)       */
/* ------------------------------------------------------------------------ */

/* reactor_api.h:84-114 */
enum {
  PROM_ASYNC_STATE_IDLE = 0,
  PROM_ASYNC_STATE_SUBMITTED = 1,
  PROM_ASYNC_STATE_READY = 2,
  PROM_ASYNC_STATE_FAILED = 3,
  PROM_ASYNC_STATE_CONSUMED = 4,
};

enum {
  PROM_ASYNC_FAILURE_NONE = 0,
  PROM_ASYNC_FAILURE_PRE_SUBMIT = 1,
  PROM_ASYNC_FAILURE_OBSERVATION = 2,
  PROM_ASYNC_FAILURE_QUERY = 3,
  PROM_ASYNC_FAILURE_SUBMISSION = 4,
  PROM_ASYNC_FAILURE_DEVICE_LOST = 5,
};

enum {
  PROM_ASYNC_PHYSICAL_EMPTY = 0,
  PROM_ASYNC_PHYSICAL_PREPARING = 1,
  PROM_ASYNC_PHYSICAL_RECORDED = 2,
  PROM_ASYNC_PHYSICAL_SUBMITTED = 3,
  PROM_ASYNC_PHYSICAL_COMPLETE = 4,
  PROM_ASYNC_PHYSICAL_READY = 5,
  PROM_ASYNC_PHYSICAL_FAILED = 6,
  PROM_ASYNC_PHYSICAL_QUARANTINED = 7,
  PROM_ASYNC_PHYSICAL_FAILED_FATAL = 8,
};

/* reactor_api.h:250-260, 282-295 */
enum {
  PROM_DETAIL_ASYNC_NOT_READY = -6108,
  PROM_DETAIL_ASYNC_NO_TASK = -6109,
  PROM_DETAIL_ASYNC_ALREADY_CONSUMED = -6110,
  PROM_DETAIL_ASYNC_INVALID_TASK = -6111,
  PROM_DETAIL_ASYNC_SUBMIT_REJECTED = -6112,
  PROM_DETAIL_ASYNC_SOFTWARE_SUPPRESSED = -6113,
  PROM_DETAIL_ASYNC_FAILED = -6114,
  PROM_DETAIL_ASYNC_UNCONSUMED = -6115,
  PROM_DETAIL_INJECTED_ASYNC_POLL_FAILURE = -6116,
  PROM_DETAIL_ASYNC_QUEUE_FULL = -6117,
  PROM_DETAIL_BATCH_ZERO_WORKERS = -6601,
  PROM_DETAIL_BATCH_PLAN_INVALID = -6602,
  PROM_DETAIL_BATCH_EVENT_RING_OVERFLOW = -6603,
  PROM_DETAIL_BATCH_EXECUTION_FAILED = -6604,
  PROM_DETAIL_BATCH_RESOURCE_OWNERSHIP_VIOLATION = -6605,
  PROM_DETAIL_BATCH_COMMAND_RESOURCE_CREATE_FAILED = -6606,
  PROM_DETAIL_BATCH_COMMAND_RECORD_FAILED = -6607,
  PROM_DETAIL_BATCH_FENCE_RESET_FAILED = -6608,
  PROM_DETAIL_BATCH_FENCE_WAIT_FAILED = -6609,
  PROM_DETAIL_BATCH_QUEUE_SUBMIT_FAILED = -6610,
  PROM_DETAIL_BATCH_DEVICE_LOST = -6611,
  PROM_DETAIL_BATCH_DRAIN_TIMEOUT = -6612,
  PROM_DETAIL_BATCH_UNSUPPORTED_OPTION = -6613,
};

/* reactor_api.h:1448-1474.  Bits 0..7 of the batch flags are the requested
   logical width (0 means 1); PARTITION_CONTIGUOUS selects the contiguous lane
   map.  The other bits are test seams that only ..._sgemm_batch_m31_test
   accepts; the public entry rejects them with BATCH_UNSUPPORTED_OPTION. */
enum {
  PROM_BATCH_FLAG_PARTITION_CONTIGUOUS = 1u << 8,
  PROM_BATCH_FLAG_FAIL_AFTER_FIRST_SUBMIT = 1u << 9,
  PROM_BATCH_FLAG_TEST_HW_CAP_SHIFT = 10u,
  PROM_BATCH_FLAG_TEST_HW_CAP_MASK = 0xFu << 10u,
  PROM_BATCH_FLAG_TEST_SEPARATE_COMPUTE_FAMILY = 1u << 10u,
  PROM_BATCH_FLAG_TEST_ARENA_SCALE_SHIFT = 14u,
  PROM_BATCH_FLAG_TEST_ARENA_SCALE_MASK = 0x3u << 14u,
  PROM_BATCH_FLAG_TEST_EVENT_CAPACITY_SHIFT = 16u,
  PROM_BATCH_FLAG_TEST_EVENT_CAPACITY_MASK = 0x3Fu << 16u,
  PROM_BATCH_FLAG_TEST_DUAL_FAIL_FIRST_TWO = 1u << 22,
  PROM_BATCH_FLAG_TEST_DELAY_ENTRY0 = 1u << 23,
  PROM_BATCH_FLAG_TEST_FAIL_ENTRY_SHIFT = 24u,
};
/* Above INT_MAX, so a macro: ISO C limits enumerators to int. */
#define PROM_BATCH_FLAG_TEST_FAIL_ENTRY_MASK 0xFF000000u

/* reactor_api.h:1476-1545 (the values this library reports) */
enum { PROM_BATCH_PARTITION_ROUND_ROBIN = 1u, PROM_BATCH_PARTITION_CONTIGUOUS = 2u };
enum {
  PROM_BATCH_STATE_PENDING = 1u,
  PROM_BATCH_STATE_RUNNING = 2u,
  PROM_BATCH_STATE_FAILING = 3u,
  PROM_BATCH_STATE_DRAINING = 4u,
  PROM_BATCH_STATE_FAILED = 5u,
  PROM_BATCH_STATE_SUCCEEDED = 6u,
};
enum { PROM_BATCH_EXECUTION_SINGLE_WORKER = 1u };
enum { PROM_BATCH_WORKER_RESOURCE_SHARED = 2u };
enum { PROM_BATCH_QUEUE_TOPOLOGY_SINGLE_QUEUE = 1u };
enum { PROM_BATCH_QUEUE_MAPPING_SINGLE_QUEUE_SERIALIZED = 1u };

/* reactor_api.h:1771-1779 */
typedef struct PrometheusAsyncStatus {
  uint32_t lifecycle_state;
  uint32_t stage;
  int detail_code;
  uint32_t ready;
  uint32_t failed;
  uint32_t consumed;
  uint32_t outstanding_tasks;
} PrometheusAsyncStatus;

/* reactor_api.h:1307-1314 */
typedef struct PrometheusSgemmBatchEntry {
  const float* a;
  const float* b;
  float* c;
  uint32_t m;
  uint32_t n;
  uint32_t k;
} PrometheusSgemmBatchEntry;

/* reactor_api.h:1316-1447.  Field order and sizes are the reference's so a
   caller compiled against it reads the same bytes.  This library fills the
   plan, state, failure, lane, ring and per-entry (m31_*) fields; fields that
   describe Vulkan worker threads, command pools, fences and slot leases have no
   HIP counterpart and stay zero. */
typedef struct PrometheusSgemmBatchDiagnostics {
  uint32_t last_batch_entry_count;
  uint32_t requested_workers;
  uint32_t effective_workers;
  uint32_t hardware_queue_cap;
  uint32_t memory_worker_cap;
  uint32_t worker_cap_reason;
  uint32_t partition_policy;
  uint32_t batch_state;
  uint32_t failed_entry_id;
  uint32_t failed_worker_id;
  uint32_t failure_stage;
  int32_t failure_detail;
  uint32_t failure_count;
  uint32_t first_failure_stable;
  uint32_t event_overflow_count;
  uint32_t event_drain_count;
  uint32_t output_committed;
  uint32_t plan_generation;
  uint32_t worker_judgment_count;
  uint32_t execution_mode;
  uint32_t worker_resource_mode;
  uint32_t queue_topology_classification;
  uint32_t queue_mapping_mode;
  uint32_t lane_worker_count;
  uint32_t real_worker_thread_count;
  uint32_t serialized_vulkan;
  uint32_t serialized_bridge_enter_count;
  uint32_t serialized_execution_count;
  uint32_t serialized_wait_count;
  uint32_t max_concurrent_serialized_entries;
  uint32_t hardware_parallelism_claimed;
  uint32_t resource_ownership_violation_count;
  uint32_t resource_creation_failure_count;
  uint32_t worker_active_mask;
  uint32_t worker_assigned_count[8];
  uint32_t worker_completed_count[8];
  uint32_t worker_event_count[8];
  uint32_t worker_queue_index[8];
  uint32_t worker_submit_count[8];
  uint32_t worker_wait_count[8];
  uint32_t worker_in_flight[8];
  uint32_t worker_slot_id[8];
  uint32_t worker_output_staging_id[8];
  uint32_t worker_arena_bank_id[8];
  uint32_t worker_command_pool_id[8];
  uint32_t worker_command_buffer_id[8];
  uint32_t worker_fence_id[8];
  uint32_t worker_command_pool_valid[8];
  uint32_t worker_command_buffer_valid[8];
  uint32_t worker_fence_valid[8];
  uint32_t worker_reset_count[8];
  uint32_t worker_record_count[8];
  uint32_t worker_failure_stage[8];
  int32_t worker_failure_detail[8];
  uint32_t reported_compute_queue_count;
  uint32_t independent_compute_queue_count;
  uint32_t true_multi_queue_selected;
  uint32_t hardware_parallelism_eligible;
  uint32_t serialized_fallback_reason;
  uint32_t per_worker_queue_family[8];
  uint32_t per_worker_fence_state[8];
  uint32_t queue_drain_count;
  uint32_t drain_timeout_count;
  uint32_t queue_family_ownership_handoff_count;
  uint32_t transfer_compute_sync_wait_count;
  uint32_t unsafe_to_reuse;
  uint32_t slots_per_worker_target;
  uint32_t effective_slots_per_worker;
  uint32_t total_slot_count;
  uint32_t slot_cap_reason;
  uint32_t slot_refill_count;
  uint32_t slot_full_scan_poll_count;
  uint32_t slot_attention_poll_count;
  uint32_t slot_polling_avoided_count;
  uint32_t slot_failure_count;
  uint32_t slot_drain_count;
  uint32_t slot_boundary_generation;
  uint32_t slot_dirty_mask;
  uint32_t slot_ready_mask;
  uint32_t slot_failed_mask;
  uint32_t slot_invalidated_mask;
  uint32_t slot_attention_mask;
  uint32_t slot_owner_worker_id[16];
  uint32_t slot_state[16];
  uint32_t slot_generation[16];
  uint32_t slot_entry_id[16];
  uint32_t slot_queue_id[16];
  uint32_t slot_command_resource_id[16];
  uint32_t slot_arena_id[16];
  uint32_t slot_output_staging_id[16];
  uint32_t slot_in_flight[16];
  uint32_t slot_ready[16];
  uint32_t slot_invalidated[16];
  uint32_t slot_failure_stage[16];
  int32_t slot_failure_detail[16];
  uint64_t p13_m10_lease_request_count;
  uint64_t p13_m10_lease_grant_count;
  uint64_t p13_m10_lease_deny_count;
  uint64_t p13_m10_lease_yield_count;
  uint32_t p13_m10_lease_last_state;
  uint32_t p13_m10_lease_last_deny_reason;
  uint32_t p13_m10_lookahead_requested;
  uint32_t p13_m10_lookahead_allowed;
  uint32_t p13_m10_lookahead_blocked_reason;
  uint32_t p13_m10_selected_recipe_variant;
  uint32_t physical_ring_depth_configured;
  uint32_t physical_ring_depth_effective;
  uint32_t current_in_flight;
  uint32_t max_in_flight;
  uint64_t total_submits;
  uint64_t total_polls;
  uint64_t total_forced_waits;
  uint64_t ring_full_count;
  uint64_t refill_count;
  uint64_t query_harvest_count;
  uint64_t quarantine_count;
  uint64_t reap_count;
  uint64_t feedback_committed_count;
  uint64_t feedback_skipped_count;
  uint32_t m31_completion_count;
  uint32_t m31_commit_count;
  uint64_t m31_submission_sequence[64];
  uint32_t m31_physical_slot_id[64];
  uint32_t m31_completion_status[64];
  uint64_t m31_gpu_duration_ns[64];
  uint32_t m31_completion_order[64];
  uint32_t m31_commit_order[64];
} PrometheusSgemmBatchDiagnostics;

/* reactor_api.h:1987-2006 */
typedef struct PrometheusSgemmAsyncTaskDiagnostics {
  int32_t task_id;
  uint32_t generation;
  uint32_t lifecycle_state;
  uint32_t physical_slot_id;
  uint32_t physical_slot_generation;
  uint64_t submission_sequence;
  uint32_t timing_valid;
  uint64_t gpu_duration_ns;
  uint32_t feedback_pending;
  uint32_t feedback_committed;
  int32_t failure_detail;
  uint32_t failure_class;
  uint32_t abandoned;
  uint32_t physical_slot_state;
  uint32_t quarantined;
  uint32_t physical_completion_confirmed;
  uint32_t reap_pending;
  uint32_t reap_completed;
} PrometheusSgemmAsyncTaskDiagnostics;

/* reactor_api.h:2008-2032 */
typedef struct PrometheusSgemmAsyncDiagnostics {
  uint32_t task_capacity;
  uint32_t active_task_count;
  uint32_t submitted_count;
  uint32_t ready_count;
  uint32_t failed_count;
  uint32_t consumed_count;
  uint32_t abandoned_count;
  uint64_t queue_full_count;
  uint64_t stale_id_rejection_count;
  uint32_t max_in_flight;
  uint32_t feedback_pending_count;
  uint64_t feedback_committed_count;
  uint64_t feedback_skipped_count;
  uint64_t next_feedback_sequence;
  uint32_t quarantined_slot_count;
  uint64_t quarantine_event_count;
  uint64_t reap_poll_count;
  uint64_t reap_success_count;
  uint64_t reap_wait_count;
  uint64_t reap_failure_count;
  uint32_t max_quarantine_depth;
  uint32_t runtime_unsafe_to_reuse;
  PrometheusSgemmAsyncTaskDiagnostics tasks[4];
} PrometheusSgemmAsyncDiagnostics;

/* reactor_api.h:2610-2615; reactor_sgemm.cpp:5984-6009, reactor_batch.c:244-560.
   Runs every entry C_i = A_i @ B_i (host pointers, row-major fp32) and commits
   all outputs in entry order only when every entry succeeded; a failure leaves
   every caller output untouched.  Entries are validated before any work is
   enqueued (BATCH_PLAN_INVALID names the first bad entry in the diagnostics).
   Any number of entries; the device arena is reused across calls. */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_batch(void* handle, const PrometheusSgemmBatchEntry* entries,
                                                            uint32_t entry_count, uint32_t flags, uint32_t* out_stage,
                                                            int* out_detail_code);
/* reactor_api.h:2617-2622 -- the same with the test seams of the flag word
   enabled (FAIL_AFTER_FIRST_SUBMIT, TEST_FAIL_ENTRY, TEST_DUAL_FAIL_FIRST_TWO). */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_batch_m31_test(void* handle,
                                                                     const PrometheusSgemmBatchEntry* entries,
                                                                     uint32_t entry_count, uint32_t flags,
                                                                     uint32_t* out_stage, int* out_detail_code);
/* reactor_api.h:2649-2650 -- the last batch's diagnostics. */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_batch_diagnostics(void* handle,
                                                                        PrometheusSgemmBatchDiagnostics* out_diag);
/* reactor_api.h:2623-2631; reactor_sgemm.cpp:6298-6342.  Copies A and B into
   pinned staging, enqueues upload, SGEMM and download on the runtime stream
   and returns a task id (4-entry task table, ids carry a generation; two
   submission slots, so a third unconsumed task is QUEUE_FULL).  While any task
   is unconsumed the synchronous ..._sgemm is rejected with ASYNC_UNCONSUMED. */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_submit_async(void* handle, const float* a, const float* b,
                                                                   uint32_t m, uint32_t n, uint32_t k,
                                                                   int* out_task_id, uint32_t* out_stage,
                                                                   int* out_detail_code);
/* reactor_api.h:2632-2634; reactor_sgemm.cpp:6344-6364 -- non-blocking. */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_query_async(void* handle, int task_id,
                                                                  PrometheusAsyncStatus* out_status);
/* reactor_api.h:2635-2636; reactor_sgemm.cpp:6366-6416 */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_async_diagnostics(void* handle,
                                                                         PrometheusSgemmAsyncDiagnostics* out_diag);
/* reactor_api.h:2637-2642; reactor_sgemm.cpp:6418-6471 -- c_len >= m*n. */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_consume_async(void* handle, int task_id, float* c,
                                                                    uint32_t c_len, uint32_t* out_stage,
                                                                    int* out_detail_code);
/* reactor_api.h:2643; reactor_sgemm.cpp:6473-6502 -- rejected while running. */
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_abandon_async(void* handle, int task_id);

/* ------------------------------------------------------------------------ */
/* Binary64 FFT                                                              */
/* ------------------------------------------------------------------------ */

/* reactor_api.h:329-380 */
typedef struct PrometheusComplex32 {
  float real;
  float imag;
} PrometheusComplex32;

enum {
  PROM_FFT_FLAG_FORWARD = 1u << 0,
  PROM_FFT_FLAG_INVERSE = 1u << 1,
  PROM_FFT_FLAG_INVERSE_NORMALIZE = 1u << 2,
  PROM_FFT_FLAG_BENCHMARK_ALLOW_NON_PRODUCTION_PATH = 1u << 3,
};

enum {
  PROM_FFT_PATH_NONE = 0,
  PROM_FFT_PATH_UNAVAILABLE = 1,
  PROM_FFT_PATH_CPU_ORACLE_RESERVED = 2,
  PROM_FFT_PATH_VULKAN_RADIX2_RESERVED = 3,
};

enum {
  PROM_FFT_PATH_STATUS_UNAVAILABLE = 0,
  PROM_FFT_PATH_STATUS_REGISTERED = 1,
  PROM_FFT_PATH_STATUS_BENCHMARK_ENABLED = 2,
  PROM_FFT_PATH_STATUS_PRODUCTION_ENABLED = 3,
};

enum {
  PROM_FFT_BENCHMARK_VARIANT_NONE = 0,
  PROM_FFT_BENCHMARK_VARIANT_RADIX2 = 2,
};

enum {
  PROM_FFT_DETAIL_UNAVAILABLE = -6701,
  PROM_FFT_DETAIL_INVALID_REQUEST = -6702,
  PROM_FFT_DETAIL_NULL_INPUT = -6703,
  PROM_FFT_DETAIL_NULL_OUTPUT = -6704,
  PROM_FFT_DETAIL_ZERO_ELEMENT_COUNT = -6705,
  PROM_FFT_DETAIL_NON_POWER_OF_TWO = -6706,
  PROM_FFT_DETAIL_INVALID_DIRECTION_FLAGS = -6707,
  PROM_FFT_DETAIL_INVALID_STRIDE = -6708,
  PROM_FFT_DETAIL_SIZE_OVERFLOW = -6709,
  PROM_FFT_DETAIL_ZERO_BATCH_COUNT = -6710,
  PROM_FFT_DETAIL_INVERSE_NORMALIZE_REQUIRES_INVERSE = -6711,
  PROM_FFT_DETAIL_VULKAN_UNAVAILABLE = -6712,
  PROM_FFT_DETAIL_UNSUPPORTED_SIZE = -6713,
  PROM_FFT_DETAIL_ALLOCATION_FAILED = -6714,
  PROM_FFT_DETAIL_UPLOAD_FAILED = -6715,
  PROM_FFT_DETAIL_DISPATCH_FAILED = -6716,
  PROM_FFT_DETAIL_READBACK_FAILED = -6717,
  PROM_FFT_DETAIL_SHADER_UNAVAILABLE = -6718,
  PROM_FFT_DETAIL_PLAN_DISPATCH_DISAGREEMENT = -6719,
  PROM_FFT_DETAIL_FLOAT64_UNAVAILABLE = -6720,
};

/* reactor_api.h:1251-1305 */
typedef struct PrometheusFftRequest {
  uint32_t struct_size;
  const PrometheusComplex32* input;
  PrometheusComplex32* output;
  uint32_t element_count;
  uint32_t batch_count;
  uint32_t stride_elements;
  uint32_t flags;
} PrometheusFftRequest;

typedef struct PrometheusFftDiagnostics {
  uint32_t struct_size;
  uint32_t api_declared;
  uint32_t capability_reported;
  uint32_t production_enabled;
  uint32_t benchmark_enabled;
  uint32_t last_element_count;
  uint32_t last_batch_count;
  uint32_t last_stride_elements;
  uint32_t last_effective_stride_elements;
  uint32_t last_flags;
  uint32_t last_direction;
  uint32_t last_validation_status;
  int32_t last_failure_detail;
  uint32_t requested_path_id;
  uint32_t executed_path_id;
  uint32_t requested_radix;
  uint32_t executed_radix;
  uint32_t fallback_reason;
  uint32_t plan_pass_count;
  uint32_t ping_pong_swap_count;
  uint32_t final_output_role;
  uint64_t ping_arena_reuse_count;
  uint64_t ping_arena_grow_count;
  uint64_t pong_arena_reuse_count;
  uint64_t pong_arena_grow_count;
  uint64_t twiddle_arena_reuse_count;
  uint64_t twiddle_arena_grow_count;
  uint32_t selector_cache_valid;
  uint32_t plan_valid;
  uint32_t plan_element_count;
  uint32_t plan_log2_element_count;
  uint32_t plan_first_span;
  uint32_t plan_last_span;
  uint32_t plan_radix_mask;
  uint32_t plan_bit_reversal_required;
  uint32_t plan_first_source_role;
  uint32_t plan_first_destination_role;
  uint32_t plan_direction;
  uint32_t plan_twiddle_mode;
  uint64_t selector_cache_reuse_count;
  uint64_t selector_cache_recompute_count;
  uint64_t selector_cache_invalidation_count;
  uint64_t selector_cache_last_dependency_mask;
} PrometheusFftDiagnostics;

/* reactor_api.h:2652-2655; reactor_concept_fft.cpp:97-104.  Interleaved
   binary64 complex pairs, forward, unnormalised, count a power of two in
   [1, 2^20]; input and output each hold count pairs and may be the same
   array.  Invalid requests -> INIT / PROM_FFT_DETAIL_INVALID_REQUEST; no
   device -> INIT / PROM_FFT_DETAIL_VULKAN_UNAVAILABLE (no CPU fallback);
   success -> TRANSFER_OUT / 0.  Result agrees with internal/fft/fft.go's CPU
   transform within 1e-12 * max|X| per component (fft.go:176-192) and is
   bit-identical to it for count <= 4096 given the same twiddle table. */
PROM_REACTOR_API int prometheus_reactor_runtime_fft64(void* handle, const double* input, double* output,
                                                      uint32_t count, uint32_t* stage, int* detail);
/* NEW: the same transform on device pointers, enqueued on the runtime stream
   (success -> SUBMIT / 0; synchronise before reading output). */
PROM_REACTOR_API int prometheus_reactor_runtime_fft64_device(void* handle, const double* input, double* output,
                                                             uint32_t count, uint32_t* stage, int* detail);

/* reactor_api.h:2656-2670; reactor_vulkan_fft.c:59-128; PrometheusFft.concept:98-176.
   Batched complex-fp32 FFT of element_count = 2^k <= 2^20 points per batch,
   batch b at input/output + b * stride (stride_elements 0 = element_count);
   element_count * batch_count <= 65535 * 256.  Forward unless
   PROM_FFT_FLAG_INVERSE; the inverse is always scaled by 1/element_count
   (INVERSE_NORMALIZE is accepted with INVERSE only).  Output padding between
   batches is left untouched.  Validation failures report INIT and their
   -67xx detail; success TRANSFER_OUT / 0.  The diagnostics record the last
   call; the route identifiers are the reference's (requested and executed
   path 3, radix 2) so callers that check them keep working. */
PROM_REACTOR_API int prometheus_reactor_runtime_fft(void* handle, const PrometheusFftRequest* request,
                                                    uint32_t* out_stage, int* out_detail_code);
/* Variant PROM_FFT_BENCHMARK_VARIANT_RADIX2 runs prometheus_reactor_runtime_fft;
   any other is INIT / PROM_FFT_DETAIL_PLAN_DISPATCH_DISAGREEMENT. */
PROM_REACTOR_API int prometheus_reactor_runtime_fft_benchmark_variant(void* handle,
                                                                      const PrometheusFftRequest* request,
                                                                      uint32_t requested_variant, uint32_t* out_stage,
                                                                      int* out_detail_code);
PROM_REACTOR_API int prometheus_reactor_runtime_fft_diagnostics(void* handle, PrometheusFftDiagnostics* out_diag);
PROM_REACTOR_API int prometheus_reactor_runtime_fft_diagnostics_sized(void* handle, PrometheusFftDiagnostics* out_diag,
                                                                      uint32_t out_size);

/* ------------------------------------------------------------------------ */
/* Gemma-4-E2B M1 positional and score entries (reactor_api.h:1826-1985)     */
/* ------------------------------------------------------------------------ */

typedef PrometheusGemma4E2BM1InputRmsNormRequest PrometheusGemma4E2BM1HeadRmsNormRequest;
typedef PrometheusGemma4E2BM1InputRmsNormResult PrometheusGemma4E2BM1HeadRmsNormResult;

/* reactor_api.h:1837-1852 */
typedef struct PrometheusGemma4E2BM1RopeRequest {
  uint32_t struct_size;
  const float* source;
  const float* cosine;
  const float* sine;
  float* output;
  uint64_t source_element_count;
  uint64_t cosine_element_count;
  uint64_t sine_element_count;
  uint64_t output_element_count;
  uint32_t tokens;
  uint32_t heads;
  uint32_t head_width;
  uint32_t reserved0;
  uint64_t source_generation;
  uint64_t table_generation;
} PrometheusGemma4E2BM1RopeRequest;

/* reactor_api.h:1854-1869 */
typedef struct PrometheusGemma4E2BM1RopeResult {
  uint32_t struct_size;
  uint32_t stage;
  int32_t detail_code;
  uint32_t output_written;
  uint32_t dispatch_count;
  uint64_t source_hash;
  uint64_t cosine_hash;
  uint64_t sine_hash;
  uint64_t output_hash;
  uint64_t buffer_allocation_count;
  uint64_t buffer_reuse_count;
  uint64_t descriptor_update_count;
  uint64_t pipeline_create_count;
  uint64_t command_buffer_reuse_count;
} PrometheusGemma4E2BM1RopeResult;

/* reactor_api.h:1875-1897 */
typedef struct PrometheusGemma4E2BM1HeadRmsNormRopeRequest {
  uint32_t struct_size;
  const float* input;
  const float* weight;
  const float* cosine;
  const float* sine;
  float* output;
  uint64_t input_element_count;
  uint64_t weight_element_count;
  uint64_t cosine_element_count;
  uint64_t sine_element_count;
  uint64_t output_element_count;
  uint32_t tokens;
  uint32_t heads;
  uint32_t head_width;
  uint32_t reserved0;
  float epsilon;
  uint64_t input_generation;
  uint64_t weight_generation;
  uint64_t table_generation;
  uint64_t exact_source_hash;
} PrometheusGemma4E2BM1HeadRmsNormRopeRequest;

/* reactor_api.h:1899-1921 */
typedef struct PrometheusGemma4E2BM1HeadRmsNormRopeResult {
  uint32_t struct_size;
  uint32_t stage;
  int32_t detail_code;
  uint32_t output_written;
  uint32_t dispatch_count;
  uint32_t resident_source_bound;
  uint32_t normalized_readback_count;
  uint64_t source_byte_offset;
  uint64_t source_byte_range;
  uint64_t destination_byte_offset;
  uint64_t destination_byte_range;
  uint64_t input_hash;
  uint64_t weight_hash;
  uint64_t output_hash;
  uint64_t buffer_allocation_count;
  uint64_t buffer_reuse_count;
  uint64_t descriptor_update_count;
  uint64_t pipeline_create_count;
  uint64_t command_buffer_reuse_count;
  uint64_t observed_weight_generation;
  uint64_t requested_weight_generation;
} PrometheusGemma4E2BM1HeadRmsNormRopeResult;

/* reactor_api.h:1926-1959 */
typedef struct PrometheusGemma4E2BM1AttentionScoresRequest {
  uint32_t struct_size;
  const float* query_input;
  const float* key_input;
  const float* query_weight;
  const float* key_weight;
  const float* cosine;
  const float* sine;
  float* scores;
  uint64_t query_input_element_count;
  uint64_t key_input_element_count;
  uint64_t query_weight_element_count;
  uint64_t key_weight_element_count;
  uint64_t cosine_element_count;
  uint64_t sine_element_count;
  uint64_t score_element_count;
  uint32_t tokens;
  uint32_t query_heads;
  uint32_t key_heads;
  uint32_t head_width;
  float epsilon;
  float scale;
  uint32_t preparation_order; /* 0: query then key; 1: key then query */
  uint64_t query_input_generation;
  uint64_t key_input_generation;
  uint64_t query_weight_generation;
  uint64_t key_weight_generation;
  uint64_t table_generation;
  uint64_t query_exact_source_hash;
  uint64_t key_exact_source_hash;
} PrometheusGemma4E2BM1AttentionScoresRequest;

/* reactor_api.h:1961-1985 */
typedef struct PrometheusGemma4E2BM1AttentionScoresResult {
  uint32_t struct_size;
  uint32_t stage;
  int32_t detail_code;
  uint32_t score_written;
  uint32_t positional_dispatch_count;
  uint32_t score_dispatch_count;
  uint32_t score_readback_count;
  uint32_t host_detour_count;
  uint32_t query_slot_id;
  uint32_t query_slot_generation;
  uint32_t key_slot_id;
  uint32_t key_slot_generation;
  uint32_t score_slot_id;
  uint32_t score_slot_generation;
  uint64_t query_byte_range;
  uint64_t key_byte_range;
  uint64_t score_byte_range;
  uint64_t score_hash;
  uint64_t buffer_allocation_count;
  uint64_t buffer_reuse_count;
  uint64_t descriptor_update_count;
  uint64_t pipeline_create_count;
  uint64_t observed_weight_generation;
  uint64_t requested_weight_generation;
} PrometheusGemma4E2BM1AttentionScoresResult;

/* reactor_api.h:2690-2695; reactor_api.c:362-368 -- the input RMSNorm with the
   output rounded to BF16 (round to nearest even) and re-expanded: the storage
   boundary of the Q/K/V projection inputs. */
PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_projection_activation_rmsnorm(
    void* handle, const PrometheusGemma4E2BM1InputRmsNormRequest* request,
    PrometheusGemma4E2BM1InputRmsNormResult* out_result);
/* reactor_api.h:2696-2699; reactor_api.c:370-395 -- per-head RMSNorm of
   [token, head] rows of 256 channels (tokens field = rows <= 120, stride 256,
   epsilon exactly 1e-6), input and output BF16-rounded. */
PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm(
    void* handle, const PrometheusGemma4E2BM1HeadRmsNormRequest* request,
    PrometheusGemma4E2BM1HeadRmsNormResult* out_result);
/* reactor_api.h:2700-2703; reactor_concept_rmsnorm.cpp:157-189 and
   gemma4e2b/rope_half_split.sdslv -- half-split RoPE of [15, heads (1 or 8),
   256] with [15, 256] cosine/sine tables: each product, then the
   difference (first half) or sum (second half), rounded to BF16. */
PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_rope(void* handle,
                                                                  const PrometheusGemma4E2BM1RopeRequest* request,
                                                                  PrometheusGemma4E2BM1RopeResult* out_result);
/* reactor_api.h:2704-2707; reactor_api.c:404-505 -- head RMSNorm (BF16 in and
   out) followed by the RoPE above in one submission; output may be NULL with
   output_element_count 0. */
PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm_rope(
    void* handle, const PrometheusGemma4E2BM1HeadRmsNormRopeRequest* request,
    PrometheusGemma4E2BM1HeadRmsNormRopeResult* out_result);
/* reactor_api.h:2708-2711; reactor_api.c:507-587 and
   gemma4e2b/attention_scores.sdslv -- both positional preparations (query
   weight and key weight committed in preparation_order), then raw pre-mask
   scores[h][i][j] = (sum_c Q[i,h,c] * K[j,0,c]) * 0.0625 in fp32 (1800 scores). */
PROM_REACTOR_API int prometheus_reactor_runtime_gemma4e2b_m1_attention_scores(
    void* handle, const PrometheusGemma4E2BM1AttentionScoresRequest* request,
    PrometheusGemma4E2BM1AttentionScoresResult* out_result);

/* ------------------------------------------------------------------------ */
/* Resident model blocks and the compiled Z-Image session                   */
/* (reactor_api.h:25-45, 666-1249, 2713-2821)                               */
/* ------------------------------------------------------------------------ */

/* reactor_api.h:198-202: one-shot faults taken from the runtime config's
   reduction_test_flags; the resident model block consumes them in phase order. */
enum {
  PROM_REDUCTION_TESTCFG_FAIL_COMMAND_RECORD = 1u << 0,
  PROM_REDUCTION_TESTCFG_FAIL_QUEUE_SUBMIT = 1u << 1,
  PROM_REDUCTION_TESTCFG_FAIL_COMPLETION_OBSERVATION = 1u << 2,
};

enum {
  PROM_MODEL_EXECUTION_PROFILE_MINIMUM_MEMORY = 1u,
  PROM_MODEL_EXECUTION_PROFILE_PREFETCH = 2u,
};
enum {
  PROM_MAIN_ATTENTION_ROUTE_AUTO = 1u,
  PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL = 2u,
  PROM_MAIN_ATTENTION_ROUTE_SUBGROUP_OWNED32 = 3u,
};
/* reactor_api.h:43-53 */
enum {
  PROM_MAIN_ATTENTION_FALLBACK_NONE = 0u,
  PROM_MAIN_ATTENTION_FALLBACK_RUNTIME_CONTRACT = 1u,
  PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_COMPUTE = 2u,
  PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_SIZE = 3u,
  PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_ARITHMETIC = 4u,
  PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_BASIC = 5u,
  PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_SHUFFLE = 6u,
  PROM_MAIN_ATTENTION_FALLBACK_TOPOLOGY_PROOF = 7u,
  PROM_MAIN_ATTENTION_FALLBACK_SHAPE = 8u,
};

#define PROM_MODEL_BLOCK_MAX_WEIGHTS 13u
#define PROM_MODEL_BLOCK_MAX_STEPS 7u
#define PROM_MODEL_BLOCK_MAX_AUDIT_POINTS 1u
#define PROM_MODEL_BLOCK_M1B_PIPELINE_COUNT 6u
#define PROM_MODEL_BLOCK_MAIN_STAGE_COUNT 13u

enum {
  PROM_MODEL_BLOCK_STEP_BIND_PIPELINE = 1u,
  PROM_MODEL_BLOCK_STEP_BIND_RESOURCES = 2u,
  PROM_MODEL_BLOCK_STEP_PUSH_CONSTANTS = 3u,
  PROM_MODEL_BLOCK_STEP_DISPATCH = 4u,
  PROM_MODEL_BLOCK_STEP_BARRIER = 5u,
  PROM_MODEL_BLOCK_STEP_AUDIT_COPY = 6u,
  PROM_MODEL_BLOCK_STEP_OUTPUT_COPY = 7u,
};

enum {
  PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST = -6901,
  PROM_MODEL_BLOCK_DETAIL_NOT_FOUND = -6902,
  PROM_MODEL_BLOCK_DETAIL_ALREADY_CREATED = -6903,
  PROM_MODEL_BLOCK_DETAIL_WEIGHT_MISMATCH = -6904,
  PROM_MODEL_BLOCK_DETAIL_RESOURCE_CREATE_FAILED = -6905,
  PROM_MODEL_BLOCK_DETAIL_PIPELINE_CREATE_FAILED = -6906,
  PROM_MODEL_BLOCK_DETAIL_UPLOAD_FAILED = -6907,
  PROM_MODEL_BLOCK_DETAIL_COMMAND_RECORD_FAILED = -6908,
  PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED = -6909,
  PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN = -6910,
  PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED = -6911,
  PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT = -6912,
  PROM_MODEL_BLOCK_DETAIL_INGRESS_PIPELINE_CREATE_FAILED = -6913,
  PROM_MODEL_BLOCK_DETAIL_INGRESS_DISPATCH_FAILED = -6914,
  PROM_MODEL_BLOCK_DETAIL_INGRESS_AUDIT_MISMATCH = -6915,
  PROM_MODEL_BLOCK_DETAIL_INGRESS_INPUT_SIZE_MISMATCH = -6916,
  PROM_MODEL_BLOCK_DETAIL_INGRESS_TIMESTEP_SIZE_MISMATCH = -6917,
  PROM_MODEL_BLOCK_DETAIL_M1C_SOFTMAX_INVALID = -6918,
  PROM_MODEL_BLOCK_DETAIL_M1D_NONFINITE = -6919,
  PROM_MODEL_BLOCK_DETAIL_PARAMETER_SET_MISMATCH = -6920,
  PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED = -6921,
  PROM_MODEL_BLOCK_DETAIL_DESCRIPTOR_UPDATE_FAILED = -6922,
  PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST = -6923,
  PROM_MODEL_SESSION_DETAIL_STALE_STREAM = -6924,
  PROM_MODEL_SESSION_DETAIL_STREAM_MISMATCH = -6925,
  PROM_MODEL_SESSION_DETAIL_COMPLETION_UNCERTAIN = -6926,
  PROM_MODEL_SESSION_DETAIL_MAIN_ATTENTION_ROUTE_REJECTED = -6927,
};

enum {
  PROM_ZIMAGE_STREAM_PREPARED_IMAGE = 1u,
  PROM_ZIMAGE_STREAM_PREPARED_CONTEXT = 2u,
  PROM_ZIMAGE_STREAM_JOINT_WORKING = 3u,
  PROM_ZIMAGE_STREAM_MAIN_IMAGE_OUTPUT = 4u,
  PROM_ZIMAGE_STREAM_MAIN_CONTEXT_OUTPUT = 5u,
  PROM_ZIMAGE_STREAM_SLOT_COUNT = 5u,
};

enum {
  PROM_NOISE_REFINER_FAMILY_Z_IMAGE_TURBO = 1u,
  PROM_NOISE_REFINER_PARAMETER_SET_0 = 1u,
  PROM_NOISE_REFINER_PARAMETER_SET_1 = 2u,
  PROM_CONTEXT_REFINER_FAMILY_Z_IMAGE_TURBO = 2u,
  PROM_CONTEXT_REFINER_PARAMETER_SET_0 = 1u,
  PROM_CONTEXT_REFINER_PARAMETER_SET_1 = 2u,
  PROM_MAIN_TRANSFORMER_FAMILY_Z_IMAGE_TURBO = 3u,
  PROM_MAIN_TRANSFORMER_PARAMETER_SET_0 = 1u,
};

enum {
  PROM_NOISE_REFINER_BINDING_BOUND = 1u,
  PROM_NOISE_REFINER_BINDING_VALIDATING = 2u,
  PROM_NOISE_REFINER_BINDING_UPLOADING = 3u,
  PROM_NOISE_REFINER_BINDING_UPDATING_DESCRIPTORS = 4u,
  PROM_NOISE_REFINER_BINDING_READY_TO_COMMIT = 5u,
  PROM_NOISE_REFINER_BINDING_COMMITTED = 6u,
  PROM_NOISE_REFINER_BINDING_FAILED_BEFORE_COMMIT = 7u,
  PROM_NOISE_REFINER_BINDING_COMPLETION_UNCERTAIN = 8u,
  PROM_NOISE_REFINER_BINDING_QUARANTINED = 9u,
};

enum {
  PROM_MODEL_WEIGHT_WINDOW_EMPTY = 0u,
  PROM_MODEL_WEIGHT_WINDOW_HOST_PREPARED = 1u,
  PROM_MODEL_WEIGHT_WINDOW_UPLOAD_SUBMITTED = 2u,
  PROM_MODEL_WEIGHT_WINDOW_DEVICE_READY = 3u,
  PROM_MODEL_WEIGHT_WINDOW_ACTIVE = 4u,
  PROM_MODEL_WEIGHT_WINDOW_UNCERTAIN = 5u,
  PROM_MODEL_WEIGHT_WINDOW_QUARANTINED = 6u,
};

enum {
  PROM_NOISE_REFINER_AUDIT_NONE = 0u,
  PROM_NOISE_REFINER_AUDIT_M1B = 1u,
  PROM_NOISE_REFINER_AUDIT_M1C = 2u,
  PROM_NOISE_REFINER_AUDIT_M1D = 3u,
};

/* The model lock of the Z-Image Turbo compiled model (the reference's
   generated models/zimage-turbo/resolved_descriptor.h). */
#define PROM_ZIMAGE_TURBO_LOCK_ID 0x71ef202b4e34b562ull
#define PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES 47186176u
/* The lock's static-audit arenas (generated
   models/zimage-turbo/resolved_audit_schedule.h:5-10, 67-70): the
   NoiseRefiner arena holds nine full adaLN vectors (bytes 0..184319), twenty
   256-byte summary records (184320..189439) and the 64-float attention
   witness (189440); the ContextRefiner arena sixteen records and the witness
   at 4096.  Bytes past the required ones are zero. */
#define PROM_ZIMAGE_TURBO_AUDIT_LOCK_ID PROM_ZIMAGE_TURBO_LOCK_ID
#define PROM_ZIMAGE_TURBO_AUDIT_REQUIRED_BYTES 189696u
#define PROM_ZIMAGE_TURBO_AUDIT_TRANSIENT_ATTENTION_OFFSET 189440u
#define PROM_ZIMAGE_TURBO_AUDIT_STAGE_COUNT 29u
#define PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_ARENA_BYTES 1048576u
#define PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_REQUIRED_BYTES 4352u
#define PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_TRANSIENT_ATTENTION_OFFSET 4096u
#define PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_STAGE_COUNT 16u
#define PROM_ZIMAGE_TURBO_AUDIT_TRANSIENT_ATTENTION_BYTES 256u

/* reactor_api.h:775-798: the NoiseRefiner pre-attention (M1B) audit stages. */
enum {
  PROM_MODEL_BLOCK_M1B_AUDIT_NONE = 0u,
  PROM_MODEL_BLOCK_M1B_AUDIT_INGRESS_INPUT = 1u,
  PROM_MODEL_BLOCK_M1B_AUDIT_INGRESS_TIMESTEP = 2u,
  PROM_MODEL_BLOCK_M1B_AUDIT_ADALN_PROJECTION = 3u,
  PROM_MODEL_BLOCK_M1B_AUDIT_ATTENTION_SCALE_RAW = 4u,
  PROM_MODEL_BLOCK_M1B_AUDIT_ATTENTION_SCALE_ADJUSTED = 5u,
  PROM_MODEL_BLOCK_M1B_AUDIT_ATTENTION_GATE_RAW = 6u,
  PROM_MODEL_BLOCK_M1B_AUDIT_ATTENTION_GATE_TANH = 7u,
  PROM_MODEL_BLOCK_M1B_AUDIT_MLP_SCALE_RAW = 8u,
  PROM_MODEL_BLOCK_M1B_AUDIT_MLP_SCALE_ADJUSTED = 9u,
  PROM_MODEL_BLOCK_M1B_AUDIT_MLP_GATE_RAW = 10u,
  PROM_MODEL_BLOCK_M1B_AUDIT_MLP_GATE_TANH = 11u,
  PROM_MODEL_BLOCK_M1B_AUDIT_ATTENTION_NORM = 12u,
  PROM_MODEL_BLOCK_M1B_AUDIT_ATTENTION_MODULATED = 13u,
  PROM_MODEL_BLOCK_M1B_AUDIT_FUSED_QKV = 14u,
  PROM_MODEL_BLOCK_M1B_AUDIT_Q = 15u,
  PROM_MODEL_BLOCK_M1B_AUDIT_K = 16u,
  PROM_MODEL_BLOCK_M1B_AUDIT_V = 17u,
  PROM_MODEL_BLOCK_M1B_AUDIT_Q_NORM = 18u,
  PROM_MODEL_BLOCK_M1B_AUDIT_K_NORM = 19u,
  PROM_MODEL_BLOCK_M1B_AUDIT_POSITIONED_Q = 20u,
  PROM_MODEL_BLOCK_M1B_AUDIT_POSITIONED_K = 21u,
};

/* reactor_api.h:989-995, 1095-1103: attention (M1C) and FFN (M1D) stages. */
enum {
  PROM_MODEL_BLOCK_M1C_AUDIT_ATTENTION = 1u,
  PROM_MODEL_BLOCK_M1C_AUDIT_PROJECTION = 2u,
  PROM_MODEL_BLOCK_M1C_AUDIT_RESIDUAL = 3u,
};
#define PROM_MODEL_BLOCK_M1C_TRANSIENT_AUDIT_FLOATS 64u
enum {
  PROM_MODEL_BLOCK_M1D_AUDIT_FFN_NORM = 1u,
  PROM_MODEL_BLOCK_M1D_AUDIT_FFN_MODULATED = 2u,
  PROM_MODEL_BLOCK_M1D_AUDIT_W1 = 3u,
  PROM_MODEL_BLOCK_M1D_AUDIT_W3 = 4u,
  PROM_MODEL_BLOCK_M1D_AUDIT_GATED_HIDDEN = 5u,
  PROM_MODEL_BLOCK_M1D_AUDIT_W2 = 6u,
  PROM_MODEL_BLOCK_M1D_AUDIT_FINAL_OUTPUT = 7u,
};

typedef struct PrometheusModelBlockWeightDeclaration {
  uint64_t content_identity;
  uint64_t layout_identity;
  uint64_t byte_count;
} PrometheusModelBlockWeightDeclaration;

typedef struct PrometheusModelBlockCreateRequest {
  uint32_t struct_size;
  uint32_t assembly_family;
  uint32_t parameter_set;
  uint64_t parameter_set_aggregate_identity;
  uint64_t model_contract_identity;
  uint64_t weight_identity;
  uint64_t shader_portfolio_identity;
  uint64_t precision_policy_identity;
  uint64_t capability_route_identity;
  uint64_t memory_ceiling_bytes;
  uint64_t external_input_bytes;
  uint64_t external_output_bytes;
  uint64_t audit_bytes;
  uint32_t shader_id;
  uint32_t weight_count;
  PrometheusModelBlockWeightDeclaration weights[PROM_MODEL_BLOCK_MAX_WEIGHTS];
  uint32_t step_count;
  uint32_t steps[PROM_MODEL_BLOCK_MAX_STEPS];
} PrometheusModelBlockCreateRequest;

typedef struct PrometheusModelBlockWeightUpload {
  uint32_t binding_index;
  const void* bytes;
  uint64_t byte_count;
  uint64_t content_identity;
  uint64_t layout_identity;
} PrometheusModelBlockWeightUpload;

typedef struct PrometheusNoiseRefinerRebindRequest {
  uint32_t struct_size;
  uint32_t model_local_block_id;
  uint64_t lock_identity;
  uint32_t upload_count;
  const PrometheusModelBlockWeightUpload* uploads;
} PrometheusNoiseRefinerRebindRequest;

typedef struct PrometheusContextRefinerCreateRequest {
  uint32_t struct_size;
  uint32_t model_local_block_id;
  uint64_t lock_identity;
  uint32_t upload_count;
  const PrometheusModelBlockWeightUpload* uploads;
} PrometheusContextRefinerCreateRequest;

typedef PrometheusContextRefinerCreateRequest PrometheusContextRefinerRebindRequest;
typedef PrometheusContextRefinerCreateRequest PrometheusMainTransformerCreateRequest;
typedef PrometheusContextRefinerCreateRequest PrometheusMainTransformerRebindRequest;

typedef struct PrometheusMainTransformerExecuteRequest {
  uint32_t struct_size;
  uint64_t session_identity;
  uint64_t lock_identity;
  uint32_t model_local_block_id;
  uint32_t audit_enabled;
  uint32_t resident_chain_mode;
  uint32_t reserved0;
  uint64_t required_image_generation;
  uint64_t required_context_generation;
  uint64_t required_joint_generation;
  const void* timestep_bf16;
  uint64_t timestep_bytes;
  uint64_t timestep_identity;
  uint64_t output_identity;
} PrometheusMainTransformerExecuteRequest;

typedef struct PrometheusModelBlockExecuteRequest {
  uint32_t struct_size;
  const float* input;
  float* output;
  uint64_t element_count;
  uint64_t input_identity;
  uint32_t audit_enabled;
  float* audit_output;
  uint64_t audit_element_capacity;
} PrometheusModelBlockExecuteRequest;

typedef struct PrometheusNoiseRefiner0ExecuteRequest {
  uint32_t struct_size;
  const void* model_input_bf16;
  const void* timestep_bf16;
  uint64_t model_input_bytes;
  uint64_t timestep_bytes;
  uint64_t input_identity;
  uint64_t timestep_identity;
  uint64_t output_identity;
  uint32_t audit_enabled;
} PrometheusNoiseRefiner0ExecuteRequest;

typedef PrometheusNoiseRefiner0ExecuteRequest PrometheusNoiseRefiner1ExecuteRequest;

typedef struct PrometheusNoiseRefinerResidentExecuteRequest {
  uint32_t struct_size;
  uint64_t input_generation;
  uint64_t output_identity;
  uint32_t audit_enabled;
  uint32_t audit_family;
  uint32_t audit_stage;
  float* audit_output;
  uint64_t audit_element_capacity;
} PrometheusNoiseRefinerResidentExecuteRequest;

typedef struct PrometheusContextRefiner0ExecuteRequest {
  uint32_t struct_size;
  const float* context_input;
  uint64_t context_input_bytes;
  uint64_t input_identity;
  uint64_t output_identity;
  uint32_t audit_enabled;
} PrometheusContextRefiner0ExecuteRequest;

typedef struct PrometheusContextRefinerResidentExecuteRequest {
  uint32_t struct_size;
  uint64_t input_generation;
  uint64_t output_identity;
  uint32_t audit_enabled;
} PrometheusContextRefinerResidentExecuteRequest;

typedef struct PrometheusNoiseRefinerFinalAuditRequest {
  uint32_t struct_size;
  uint64_t required_output_generation;
  uint64_t output_identity;
  float* output;
  uint64_t output_element_capacity;
} PrometheusNoiseRefinerFinalAuditRequest;

typedef PrometheusNoiseRefinerFinalAuditRequest PrometheusContextRefinerFinalAuditRequest;
typedef PrometheusNoiseRefinerFinalAuditRequest PrometheusMainTransformerFinalAuditRequest;

/* reactor_api.h:957-1007: the stage-split NoiseRefiner.  M1B takes the BF16
   model input and timestep and runs adaLN through the Q/K/V split (audit
   stage optional); M1C runs the attention, projection and gated residual of
   the matching M1B prefix and returns one of its stages plus the 64-float
   witness; M1D runs the FFN of the matching M1C and returns one stage. */
typedef struct PrometheusModelBlockM1BExecuteRequest {
  uint32_t struct_size;
  const void* model_input_bf16;
  const void* timestep_bf16;
  uint64_t model_input_bytes;
  uint64_t timestep_bytes;
  uint64_t input_identity;
  uint64_t timestep_identity;
  uint32_t audit_enabled;
  uint32_t audit_stage;
  float* audit_output;
  uint64_t audit_element_capacity;
} PrometheusModelBlockM1BExecuteRequest;

typedef struct PrometheusModelBlockM1CExecuteRequest {
  uint32_t struct_size;
  uint64_t m1b_prefix_replay_identity;
  uint64_t output_identity;
  float* output;
  uint64_t output_element_capacity;
  uint32_t audit_stage;
  float* transient_audit;
  uint64_t transient_audit_element_capacity;
} PrometheusModelBlockM1CExecuteRequest;

typedef struct PrometheusModelBlockM1DExecuteRequest {
  uint32_t struct_size;
  uint64_t m1c_prefix_replay_identity;
  uint64_t output_identity;
  float* output;
  uint64_t output_element_capacity;
  uint32_t audit_stage;
} PrometheusModelBlockM1DExecuteRequest;

/* reactor_api.h:1070-1093: one audited execution into the caller's arena. */
typedef struct PrometheusNoiseRefinerStaticAuditRequest {
  uint32_t struct_size;
  uint64_t lock_identity;
  uint64_t input_generation;
  uint64_t output_identity;
  void* audit_arena;
  uint64_t audit_arena_capacity_bytes;
} PrometheusNoiseRefinerStaticAuditRequest;

typedef PrometheusNoiseRefinerStaticAuditRequest PrometheusContextRefinerStaticAuditRequest;

typedef struct PrometheusMainTransformerStaticAuditRequest {
  uint32_t struct_size;
  uint64_t session_identity;
  uint64_t lock_identity;
  uint32_t model_local_block_id;
  uint64_t required_image_generation;
  uint64_t required_context_generation;
  uint64_t required_joint_generation;
  uint64_t output_identity;
  void* audit_arena;
  uint64_t audit_arena_capacity_bytes;
} PrometheusMainTransformerStaticAuditRequest;

typedef struct PrometheusModelBlockEvidence {
  uint32_t struct_size;
  int32_t detail_code;
  uint32_t created;
  uint32_t weights_uploaded;
  uint32_t quarantined;
  uint32_t output_valid;
  uint32_t audit_valid;
  uint32_t fixed_step_count;
  uint32_t weight_count;
  uint64_t persistent_bytes;
  uint64_t reusable_bytes;
  uint64_t audit_bytes;
  uint64_t external_bytes;
  uint64_t total_committed_bytes;
  uint64_t peak_plan_bytes;
  uint64_t cold_buffer_allocation_count;
  uint64_t warm_buffer_allocation_count;
  uint64_t pipeline_create_count;
  uint64_t descriptor_set_count;
  uint64_t weight_upload_count;
  uint64_t execution_count;
  uint64_t last_execution_ns;
  uint64_t execution_plan_identity;
  uint64_t replay_identity;
  uint32_t assembly_family;
  uint32_t parameter_set;
  uint32_t binding_state;
  uint32_t active_weight_window;
  uint64_t parameter_set_aggregate_identity;
  uint64_t binding_generation;
  uint64_t output_generation;
  uint64_t descriptor_generation;
  uint64_t m1b_boundary_gpu_ns[PROM_MODEL_BLOCK_M1B_PIPELINE_COUNT];
  uint64_t gpu_total_begin_tick;
  uint64_t gpu_total_end_tick;
  uint64_t gpu_total_ns;
  uint64_t gpu_compute_begin_tick;
  uint64_t gpu_compute_end_tick;
  uint64_t gpu_compute_ns;
  uint64_t gpu_ingress_transfer_ns;
  uint64_t gpu_joint_copy_ns;
  uint64_t gpu_readback_ns;
  uint64_t main_stage_gpu_begin_tick[PROM_MODEL_BLOCK_MAIN_STAGE_COUNT];
  uint64_t main_stage_gpu_end_tick[PROM_MODEL_BLOCK_MAIN_STAGE_COUNT];
  uint64_t main_stage_gpu_ns[PROM_MODEL_BLOCK_MAIN_STAGE_COUNT];
  uint64_t last_active_target_validation_ns;
  uint64_t last_command_reset_ns;
  uint64_t last_command_begin_ns;
  uint64_t last_command_record_ns;
  uint64_t last_command_end_ns;
  uint64_t last_queue_submit_ns;
  uint64_t last_fence_wait_ns;
  uint64_t last_descriptor_update_ns;
  uint64_t last_staging_memcpy_ns;
  uint64_t last_output_readback_ns;
  /* The reference's Vulkan object counters; this library creates no Vulkan
     objects and reports them as 0. */
  uint64_t vk_create_buffer_count;
  uint64_t vk_destroy_buffer_count;
  uint64_t vk_allocate_memory_count;
  uint64_t vk_free_memory_count;
  uint64_t vk_create_shader_module_count;
  uint64_t vk_destroy_shader_module_count;
  uint64_t vk_create_compute_pipelines_count;
  uint64_t vk_allocate_descriptor_sets_count;
  uint64_t vk_update_descriptor_sets_count;
  uint64_t vk_create_command_pool_count;
  uint64_t vk_allocate_command_buffers_count;
  uint64_t vk_reset_command_buffer_count;
  uint64_t vk_queue_submit_count;
  uint64_t vk_fence_wait_count;
  uint64_t vk_timeline_wait_count;
  uint64_t vk_map_memory_count;
  uint64_t vk_unmap_memory_count;
  uint64_t vk_flush_count;
  uint64_t vk_invalidate_count;
  uint64_t m6a_activation_pack_gpu_ns;
  uint64_t m6a_cooperative_execute_gpu_ns;
  uint64_t m6a_w3_segment_repack_gpu_ns;
} PrometheusModelBlockEvidence;

typedef struct PrometheusCompiledModelSessionCreateRequest {
  uint32_t struct_size;
  uint64_t lock_identity;
  uint32_t execution_profile;
  uint32_t main_attention_route_policy;
} PrometheusCompiledModelSessionCreateRequest;

typedef struct PrometheusCompiledModelSessionCaptureRequest {
  uint32_t struct_size;
  uint64_t source_output_generation;
} PrometheusCompiledModelSessionCaptureRequest;

typedef struct PrometheusCompiledModelSessionComposeRequest {
  uint32_t struct_size;
  uint64_t required_image_generation;
  uint64_t required_context_generation;
} PrometheusCompiledModelSessionComposeRequest;

typedef struct PrometheusCompiledModelSessionEvidence {
  uint32_t struct_size;
  int32_t detail_code;
  uint32_t created;
  uint32_t quarantined;
  uint64_t session_identity;
  uint64_t lock_identity;
  uint64_t active_block_id;
  uint64_t binding_generation;
  uint64_t replay_identity;
  uint64_t prepared_image_generation;
  uint64_t prepared_context_generation;
  uint64_t joint_generation;
  uint64_t joint_image_generation;
  uint64_t joint_context_generation;
  uint64_t prepared_image_bytes;
  uint64_t prepared_context_bytes;
  uint64_t joint_bytes;
  uint64_t cold_buffer_allocation_count;
  uint64_t warm_buffer_allocation_count;
  uint64_t composition_count;
  uint32_t requested_execution_profile;
  uint32_t selected_execution_profile;
  uint32_t profile_fallback_reason;
  uint32_t requested_main_attention_route;
  uint32_t selected_main_attention_route;
  uint32_t main_attention_fallback_reason;
  uint32_t main_attention_shader_id;
} PrometheusCompiledModelSessionEvidence;

/* reactor_api.h:1237-1249 */
typedef struct PrometheusCompiledModelRetargetRequest {
  uint32_t struct_size;
  uint64_t session_identity;
  uint64_t lock_identity;
  uint32_t model_local_block_id;
  uint32_t upload_count;
  const PrometheusModelBlockWeightUpload* uploads;
} PrometheusCompiledModelRetargetRequest;

typedef PrometheusCompiledModelRetargetRequest PrometheusCompiledModelPrefetchRequest;

/* reactor_api.h:2713-2733: the closed resident program.  One model block per
   runtime; ids are never reused.  Family 0 (shader 23, the seven fixed steps)
   is the resident proof: output = input, audit = the first audit_bytes/4
   input floats.  Family 1 (shader 24) is the NoiseRefiner. */
PROM_REACTOR_API int prometheus_reactor_runtime_model_block_create(void* handle,
                                                                   const PrometheusModelBlockCreateRequest* request,
                                                                   uint64_t* out_block_id,
                                                                   PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_model_block_upload_weights(
    void* handle, uint64_t block_id, const PrometheusModelBlockWeightUpload* uploads, uint32_t upload_count,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_model_block_execute(void* handle, uint64_t block_id,
                                                                    const PrometheusModelBlockExecuteRequest* request,
                                                                    PrometheusModelBlockEvidence* out_evidence);
/* reactor_api.h:2722-2730: the stage-split NoiseRefiner on a shader-24
   block (NoiseRefiner family, bound weights); M1C and M1D need a declared
   audit size of at least the stage they return. */
PROM_REACTOR_API int prometheus_reactor_runtime_model_block_execute_m1b(
    void* handle, uint64_t block_id, const PrometheusModelBlockM1BExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_model_block_execute_m1c(
    void* handle, uint64_t block_id, const PrometheusModelBlockM1CExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_model_block_execute_m1d(
    void* handle, uint64_t block_id, const PrometheusModelBlockM1DExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
/* reactor_api.h:2734-2758: NoiseRefiner (1024 image tokens, width 3840):
   BF16 model input and timestep widened on the device, the fp32 block on the
   resident weights, output kept resident (output_generation advances). */
PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner0_execute(
    void* handle, uint64_t block_id, const PrometheusNoiseRefiner0ExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner1_execute(
    void* handle, uint64_t block_id, const PrometheusNoiseRefiner1ExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner_rebind(void* handle, uint64_t block_id,
                                                                     const PrometheusNoiseRefinerRebindRequest* request,
                                                                     PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner_execute_resident(
    void* handle, uint64_t block_id, const PrometheusNoiseRefinerResidentExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
/* reactor_api.h:2743-2745: one resident NoiseRefiner 1 execution that also
   fills the lock's audit arena (output_generation advances). */
PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner_execute_static_audit(
    void* handle, uint64_t block_id, const PrometheusNoiseRefinerStaticAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner_audit_final(
    void* handle, uint64_t block_id, const PrometheusNoiseRefinerFinalAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
/* reactor_api.h:2759-2776: ContextRefiner (32 context tokens, no adaLN). */
PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_create(
    void* handle, const PrometheusContextRefinerCreateRequest* request, uint64_t* out_block_id,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_rebind(
    void* handle, uint64_t block_id, const PrometheusContextRefinerRebindRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner0_execute(
    void* handle, uint64_t block_id, const PrometheusContextRefiner0ExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_execute_resident(
    void* handle, uint64_t block_id, const PrometheusContextRefinerResidentExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
/* reactor_api.h:2761-2763: parameter set 0 re-runs its external input,
   set 1 its resident boundary, filling the ContextRefiner audit arena. */
PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_execute_static_audit(
    void* handle, uint64_t block_id, const PrometheusContextRefinerStaticAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_audit_final(
    void* handle, uint64_t block_id, const PrometheusContextRefinerFinalAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
/* reactor_api.h:2777-2791: MainTransformer layer i of 30 over the session's
   1056-token JointWorking stream (image then context). */
PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_create(
    void* handle, const PrometheusMainTransformerCreateRequest* request, uint64_t* out_block_id,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_rebind(
    void* handle, uint64_t block_id, const PrometheusMainTransformerRebindRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_execute(
    void* handle, uint64_t block_id, const PrometheusMainTransformerExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
/* reactor_api.h:2776-2778: layer 0 re-run on the session's JointWorking
   stream (the session is not advanced); the arena receives its output. */
PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_execute_static_audit(
    void* handle, uint64_t block_id, const PrometheusMainTransformerStaticAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_audit_final(
    void* handle, uint64_t block_id, const PrometheusMainTransformerFinalAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence);
/* reactor_api.h:2792-2794 */
PROM_REACTOR_API int prometheus_reactor_runtime_model_block_get_evidence(void* handle, uint64_t block_id,
                                                                         PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_model_block_destroy(void* handle, uint64_t block_id);
/* reactor_api.h:2795-2808: the session owns the PreparedImage (1024 x 3840),
   PreparedContext (32 x 3840) and JointWorking (1056 x 3840) fp32 streams. */
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_create(
    void* handle, const PrometheusCompiledModelSessionCreateRequest* request, uint64_t* out_session_id,
    PrometheusCompiledModelSessionEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_capture_completed(
    void* handle, uint64_t session_id, uint64_t completed_block_id,
    const PrometheusCompiledModelSessionCaptureRequest* request, PrometheusCompiledModelSessionEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_compose_joint(
    void* handle, uint64_t session_id, const PrometheusCompiledModelSessionComposeRequest* request,
    PrometheusCompiledModelSessionEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_get_evidence(
    void* handle, uint64_t session_id, PrometheusCompiledModelSessionEvidence* out_evidence);
/* reactor_api.h:2798-2802: records the route the next MainTransformer
   create decides; rejected while a model block exists.  The subgroup-owned
   route needs 32-lane subgroups: on 64-lane wavefronts AUTO selects the
   serial-canonical route (fallback SUBGROUP_SIZE) and an explicit
   SUBGROUP_OWNED32 makes that create fail. */
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_set_main_attention_route(
    void* handle, uint64_t session_id, uint32_t main_attention_route_policy,
    PrometheusCompiledModelSessionEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_destroy(void* handle, uint64_t session_id);
/* reactor_api.h:2809-2821: the compiled-model owner the Z-Image bridge drives
   (tools/prometheus_zimage_bridge/reactor_windows.go:86-115): one block,
   created bound to NoiseRefiner 0 for an existing session, retargeted in
   place through NoiseRefiner 1, ContextRefiner 0/1 and MainTransformer 0..29
   (the session's position names the next block), reset for a new evaluation.
   A session that requests PREFETCH selects it (fallback reason 0: a second
   HIP stream is always an independent transfer queue) and its owner holds a
   second weight window: prefetch uploads the next block into it on that
   stream, from a caller thread other than the one executing, and
   activate_prefetch swaps it in and advances the position.  Under
   MINIMUM_MEMORY both report REBIND_FAILED. */
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_owner_create(
    void* handle, const PrometheusNoiseRefinerRebindRequest* request, uint64_t* out_block_id,
    PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_retarget(
    void* handle, const PrometheusCompiledModelRetargetRequest* request, PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_prefetch(
    void* handle, const PrometheusCompiledModelPrefetchRequest* request, PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_activate_prefetch(
    void* handle, uint64_t session_id, PrometheusModelBlockEvidence* out_evidence);
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_evaluation_reset(
    void* handle, uint64_t session_id, PrometheusCompiledModelSessionEvidence* out_evidence);

#ifdef __cplusplus
}
#endif
#endif
