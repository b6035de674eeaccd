// C-ABI entry points for GEMM, row reductions and RMSNorm.
//
// Host-pointer entries mirror the reference's synchronous contract
// (internal/prometheus/native/reactor_api.h:2587-2699): validate, copy in,
// launch on the one stream, copy out, wait, and report stage/detail.
// Device-pointer entries (NEW) only validate and enqueue.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "reactor_internal.h"

using namespace prom;

namespace {

// ------------------------------------------------------------------ GEMM

// Common validation of reactor_sgemm.cpp:4152-4191; returns PROM_OK to proceed.
int gemm_validate(Runtime* rt, const void* a, const void* b, const void* c, uint32_t m, uint32_t n, uint32_t k,
                  uint32_t* out_stage, int* out_detail) {
  set_status(out_stage, out_detail, PROM_STAGE_NONE, 0);
  if (rt == nullptr) {
    set_status(out_stage, out_detail, PROM_STAGE_INIT, PROM_INVALID_HANDLE);
    return PROM_INVALID_HANDLE;
  }
  if (a == nullptr || b == nullptr || c == nullptr) {
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_IN, PROM_ERROR);
    return PROM_ERROR;
  }
  if (m == 0u || n == 0u || k == 0u) {
    set_status(out_stage, out_detail, PROM_STAGE_INIT, PROM_ERROR);
    return PROM_ERROR;
  }
  if (!rt->available) {
    set_status(out_stage, out_detail, PROM_STAGE_INIT, rt->init_detail);
    return PROM_ERROR;
  }
  if (!gemm_shape_fits(m, n, k)) {
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_IN, PROM_DETAIL_SIZE_OVERFLOW);
    return PROM_ERROR;
  }
  return PROM_OK;
}

template <typename TIn>
int gemm_host(void* handle, const TIn* a, const TIn* b, float* c, uint32_t m, uint32_t n, uint32_t k,
              uint32_t* out_stage, int* out_detail,
              hipError_t (*launch)(const TIn*, const TIn*, float*, uint32_t, uint32_t, uint32_t, hipStream_t, int*)) {
  Runtime* rt = lookup(handle);
  const int v = gemm_validate(rt, a, b, c, m, n, k, out_stage, out_detail);
  if (v != PROM_OK) return v;
  rt->requests++;
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  const size_t a_bytes = (size_t)m * k * sizeof(TIn);
  const size_t b_bytes = (size_t)k * n * sizeof(TIn);
  const size_t c_bytes = (size_t)m * n * sizeof(float);
  if (rt->test_flags & PROM_TESTCFG_FAIL_BUFFER_ALLOC) {
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_IN, PROM_DETAIL_HIP_ALLOC_FAILED);
    return PROM_ERROR;
  }
  TIn* da = static_cast<TIn*>(staging(0, a_bytes));
  TIn* db = static_cast<TIn*>(staging(1, b_bytes));
  float* dc = static_cast<float*>(staging(2, c_bytes));
  if (da == nullptr || db == nullptr || dc == nullptr) {
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_IN, PROM_DETAIL_HIP_ALLOC_FAILED);
    return PROM_ERROR;
  }
  set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_IN, 0);
  if (rt->test_flags & PROM_TESTCFG_FAIL_UPLOAD) {
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_IN, PROM_DETAIL_INJECTED_UPLOAD_FAILURE);
    return PROM_ERROR;
  }
  if (upload_host(da, a, a_bytes, cx.stream) != hipSuccess ||
      upload_host(db, b, b_bytes, cx.stream) != hipSuccess) {
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_IN, PROM_DETAIL_HIP_COPY_FAILED);
    return PROM_ERROR;
  }
  set_status(out_stage, out_detail, PROM_STAGE_SUBMIT, 0);
  if (rt->test_flags & PROM_TESTCFG_FAIL_DISPATCH) {
    (void)hipStreamSynchronize(cx.stream);
    set_status(out_stage, out_detail, PROM_STAGE_SUBMIT, PROM_DETAIL_INJECTED_DISPATCH_FAILURE);
    return PROM_ERROR;
  }
  if (rt->test_flags & (PROM_TESTCFG_FAIL_COMMAND_END | PROM_TESTCFG_FAIL_QUEUE_SUBMIT)) {
    (void)hipStreamSynchronize(cx.stream);
    set_status(out_stage, out_detail, PROM_STAGE_SUBMIT, -4);  // VK_ERROR_DEVICE_LOST, reactor_sgemm.cpp:5071-5078
    return PROM_ERROR;
  }
  int path = 0;
  if (launch(da, db, dc, m, n, k, cx.stream, &path) != hipSuccess) {
    (void)hipStreamSynchronize(cx.stream);
    set_status(out_stage, out_detail, PROM_STAGE_SUBMIT, PROM_DETAIL_HIP_LAUNCH_FAILED);
    return PROM_ERROR;
  }
  set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_OUT, 0);
  if (rt->test_flags & PROM_TESTCFG_FAIL_DOWNLOAD) {
    (void)hipStreamSynchronize(cx.stream);
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_OUT, PROM_DETAIL_INJECTED_DOWNLOAD_FAILURE);
    return PROM_ERROR;
  }
  if (download_host(c, dc, c_bytes, cx.stream) != hipSuccess) {
    (void)hipStreamSynchronize(cx.stream);
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_OUT, PROM_DETAIL_HIP_COPY_FAILED);
    return PROM_ERROR;
  }
  if (hipStreamSynchronize(cx.stream) != hipSuccess) {
    set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_OUT, PROM_DETAIL_HIP_SYNC_FAILED);
    return PROM_ERROR;
  }
  rt->successes++;
  set_status(out_stage, out_detail, PROM_STAGE_TRANSFER_OUT, path);
  return PROM_OK;
}

template <typename TIn>
int gemm_device(void* handle, const TIn* a, const TIn* b, float* c, uint32_t m, uint32_t n, uint32_t k,
                uint32_t* out_stage, int* out_detail,
                hipError_t (*launch)(const TIn*, const TIn*, float*, uint32_t, uint32_t, uint32_t, hipStream_t, int*)) {
  Runtime* rt = lookup(handle);
  const int v = gemm_validate(rt, a, b, c, m, n, k, out_stage, out_detail);
  if (v != PROM_OK) return v;
  int path = 0;
  // The lock covers the launcher's use of runtime-owned workspace (split-K partials).
  std::lock_guard<std::mutex> lock(ctx().mu);
  if (launch(a, b, c, m, n, k, ctx().stream, &path) != hipSuccess) {
    set_status(out_stage, out_detail, PROM_STAGE_SUBMIT, PROM_DETAIL_HIP_LAUNCH_FAILED);
    return PROM_ERROR;
  }
  set_status(out_stage, out_detail, PROM_STAGE_SUBMIT, path);
  return PROM_OK;
}

// ------------------------------------------------------------ reductions

struct ReductionLimits {
  uint64_t max_rows;
  uint64_t max_width;
  uint64_t max_total;
};
constexpr ReductionLimits kReferenceLimits = {PROM_REDUCTION_MAX_ROWS, PROM_REDUCTION_MAX_ELEMENTS_PER_ROW,
                                              PROM_REDUCTION_MAX_TOTAL_ELEMENTS};
constexpr ReductionLimits kLiftedLimits = {PROM_REDUCTION_V2_MAX_ROWS, PROM_REDUCTION_V2_MAX_ELEMENTS_PER_ROW,
                                           PROM_REDUCTION_V2_MAX_TOTAL_ELEMENTS};

// internal/prometheus/reactors/PrometheusReduction.concept:68-89 (ValidateShape),
// with the envelope as a parameter.
int32_t reduction_validate_shape(const PrometheusReductionRequest* r, const ReductionLimits& lim) {
  if (r->row_count == 0u) return PROM_REDUCTION_DETAIL_ZERO_ROW_COUNT;
  if (r->elements_per_row == 0u) return PROM_REDUCTION_DETAIL_ZERO_ROW_WIDTH;
  if (r->row_count > lim.max_rows) return PROM_REDUCTION_DETAIL_ROW_LIMIT;
  if (r->elements_per_row > lim.max_width) return PROM_REDUCTION_DETAIL_WIDTH_LIMIT;
  const uint64_t total = (uint64_t)r->row_count * (uint64_t)r->elements_per_row;
  if (total > lim.max_total) return PROM_REDUCTION_DETAIL_ELEMENT_LIMIT;
  if (r->operation != PROM_REDUCTION_OPERATION_SUM && r->operation != PROM_REDUCTION_OPERATION_MAX &&
      r->operation != PROM_REDUCTION_OPERATION_SOFTMAX)
    return PROM_REDUCTION_DETAIL_UNSUPPORTED_OPERATION;
  uint64_t output = r->row_count;
  if (r->operation == PROM_REDUCTION_OPERATION_SOFTMAX) {
    if (r->finalization != PROM_REDUCTION_FINALIZATION_STABLE_SOFTMAX) return PROM_REDUCTION_DETAIL_INVALID_FINALIZATION;
    output = total;
  } else if (r->finalization != PROM_REDUCTION_FINALIZATION_NONE) {
    return PROM_REDUCTION_DETAIL_INVALID_FINALIZATION;
  }
  if (r->flags > 2u || (r->operation != PROM_REDUCTION_OPERATION_SOFTMAX && r->flags != 0u))
    return PROM_REDUCTION_DETAIL_UNSUPPORTED_STRATEGY;
  if (r->flags == PROM_REDUCTION_FLAG_FORCE_FUSED && r->elements_per_row > PROM_REDUCTION_FORCE_FUSED_MAX_ELEMENTS_PER_ROW)
    return PROM_REDUCTION_DETAIL_UNSUPPORTED_STRATEGY;
  if (r->input_element_count != total) return PROM_REDUCTION_DETAIL_INPUT_SIZE_MISMATCH;
  if (r->output_element_count != output) return PROM_REDUCTION_DETAIL_OUTPUT_SIZE_MISMATCH;
  return 0;
}

// FNV-1a over the little-endian bytes of each word
// (native/reactor_vulkan_runtime_internal.h:667-674).
uint64_t fnv_u32(uint64_t h, uint32_t v) {
  for (uint32_t i = 0; i < 4u; ++i) {
    h ^= (uint64_t)((v >> (i * 8u)) & 0xffu);
    h *= 1099511628211ull;
  }
  return h;
}

// native/reactor_vulkan_fused_reduction.c:43-66
uint64_t plan_replay_id(const PrometheusReductionPlan* p) {
  uint64_t h = 1469598103934665603ull;
  h = fnv_u32(h, p->operation);
  h = fnv_u32(h, p->row_count);
  h = fnv_u32(h, p->elements_per_row);
  h = fnv_u32(h, p->strategy);
  h = fnv_u32(h, p->partial_count);
  h = fnv_u32(h, p->stage_count);
  for (uint32_t i = 0; i < p->stage_count; ++i) {
    const PrometheusReductionStageDispatch& s = p->stages[i];
    h = fnv_u32(h, s.stage_role);
    h = fnv_u32(h, s.shader_id);
    h = fnv_u32(h, s.implementation_id);
    h = fnv_u32(h, s.groups_x);
    h = fnv_u32(h, s.input_elements_per_row);
    h = fnv_u32(h, s.output_partials_per_row);
    h = fnv_u32(h, s.temporary_role);
    h = fnv_u32(h, (uint32_t)s.temporary_bytes_written);
    h = fnv_u32(h, (uint32_t)(s.temporary_bytes_written >> 32u));
  }
  return h;
}

const uint32_t kShaderForRole[8] = {0u,
                                    PROM_REDUCTION_SHADER_ROW_SUM,
                                    PROM_REDUCTION_SHADER_ROW_MAX,
                                    PROM_REDUCTION_SHADER_SOFTMAX_EXP_SUM,
                                    PROM_REDUCTION_SHADER_SOFTMAX_NORMALIZE,
                                    PROM_REDUCTION_SHADER_SOFTMAX_FUSED,
                                    PROM_REDUCTION_SHADER_ROW_SUM_PACKED_SHORT,
                                    PROM_REDUCTION_SHADER_SOFTMAX_PACKED_SHORT};
const uint32_t kImplForRole[8] = {0u,
                                  PROM_REDUCTION_IMPLEMENTATION_ROW_SUM,
                                  PROM_REDUCTION_IMPLEMENTATION_ROW_MAX,
                                  PROM_REDUCTION_IMPLEMENTATION_SOFTMAX_EXP_SUM,
                                  PROM_REDUCTION_IMPLEMENTATION_SOFTMAX_NORMALIZE,
                                  PROM_REDUCTION_IMPLEMENTATION_SOFTMAX_FUSED,
                                  PROM_REDUCTION_IMPLEMENTATION_ROW_SUM_PACKED_SHORT,
                                  PROM_REDUCTION_IMPLEMENTATION_SOFTMAX_PACKED_SHORT};

void plan_append(PrometheusReductionPlan* p, uint32_t role, uint32_t groups, uint32_t width, uint32_t partials,
                 uint32_t temp_role, uint64_t temp_bytes) {
  PrometheusReductionStageDispatch& s = p->stages[p->stage_count++];
  s.stage_role = role;
  s.shader_id = kShaderForRole[role];
  s.implementation_id = kImplForRole[role];
  s.groups_x = groups;
  s.groups_y = 1u;
  s.groups_z = 1u;
  s.input_elements_per_row = width;
  s.output_partials_per_row = partials;
  s.temporary_role = temp_role;
  s.temporary_bytes_written = temp_bytes;
}

uint32_t div_up(uint32_t a, uint32_t b) { return (a + b - 1u) / b; }

// The reference planner (PrometheusReduction.concept:91-164, BuildSchedule),
// serialised as reactor_vulkan_fused_reduction.c:101-148 does.  It describes
// the reference's multi-stage Vulkan schedule; it is reported for ABI parity.
void build_reference_plan(const PrometheusReductionRequest* r, PrometheusReductionPlan* p) {
  memset(p, 0, sizeof(*p));
  p->struct_size = sizeof(*p);
  const uint32_t rows = r->row_count, width = r->elements_per_row, op = r->operation;
  const uint32_t partials = div_up(width, PROM_REDUCTION_ELEMENTS_PER_PARTIAL);
  const uint64_t row_bytes = (uint64_t)rows * 4u;
  const uint64_t partial_bytes = partials > 1u ? row_bytes * partials : 0u;
  p->operation = op;
  p->row_count = rows;
  p->elements_per_row = width;
  p->strategy = PROM_REDUCTION_STRATEGY_COMPOSED;
  p->local_size = PROM_REDUCTION_LOCAL_SIZE;
  p->elements_per_partial = PROM_REDUCTION_ELEMENTS_PER_PARTIAL;
  p->partial_count = partials;
  p->temporary_alignment_bytes = sizeof(float);
  bool packed;
  if (op == PROM_REDUCTION_OPERATION_SOFTMAX)
    packed = r->flags == 0u && width <= 128u;
  else if (op != PROM_REDUCTION_OPERATION_SUM)
    packed = false;
  else
    packed = (width <= 96u && rows >= 512u) || (width <= 128u && rows >= 1024u);
  auto reduce = [&](uint32_t partial_role, uint32_t final_role, uint32_t destination, uint64_t dest_bytes) {
    uint32_t first_dest = destination;
    uint64_t first_bytes = dest_bytes;
    if (partials > 1u) {
      first_dest = PROM_REDUCTION_TEMPORARY_PARTIALS;
      first_bytes = (uint64_t)rows * 4u * partials;
    }
    plan_append(p, partial_role, rows * partials, width, partials, first_dest, first_bytes);
    if (partials > 1u) plan_append(p, final_role, rows, partials, 1u, destination, dest_bytes);
  };
  if (packed) {
    p->strategy = PROM_REDUCTION_STRATEGY_PACKED_SHORT_ROWS;
    const uint32_t role = op == PROM_REDUCTION_OPERATION_SOFTMAX ? PROM_REDUCTION_STAGE_SOFTMAX_PACKED_SHORT
                                                                 : PROM_REDUCTION_STAGE_ROW_SUM_PACKED_SHORT;
    plan_append(p, role, div_up(rows, 8u), width, 1u, 0u, 0u);
  } else if (op != PROM_REDUCTION_OPERATION_SOFTMAX) {
    reduce(op, op, PROM_REDUCTION_TEMPORARY_NONE, 0u);
    p->temporary_bytes = partial_bytes;
  } else if (r->flags != PROM_REDUCTION_FLAG_FORCE_COMPOSED &&
             (r->flags == PROM_REDUCTION_FLAG_FORCE_FUSED || width <= PROM_REDUCTION_ELEMENTS_PER_PARTIAL)) {
    p->strategy = PROM_REDUCTION_STRATEGY_FUSED_SINGLE_WORKGROUP;
    plan_append(p, PROM_REDUCTION_STAGE_SOFTMAX_FUSED, rows, width, 1u, 0u, 0u);
  } else {
    reduce(PROM_REDUCTION_STAGE_ROW_MAX, PROM_REDUCTION_STAGE_ROW_MAX, PROM_REDUCTION_TEMPORARY_ROW_MAX, row_bytes);
    reduce(PROM_REDUCTION_STAGE_SOFTMAX_EXP_SUM, PROM_REDUCTION_STAGE_ROW_SUM, PROM_REDUCTION_TEMPORARY_ROW_SUM,
           row_bytes);
    plan_append(p, PROM_REDUCTION_STAGE_SOFTMAX_NORMALIZE, div_up(rows * width, PROM_REDUCTION_LOCAL_SIZE), width, 1u,
                0u, 0u);
    p->temporary_bytes = partial_bytes + 2u * row_bytes;
  }
  p->replay_id = plan_replay_id(p);
}

// The plan this library executes: one fused dispatch, one wave per row.
void build_executed_plan(uint32_t rows, uint32_t width, uint32_t op, PrometheusReductionPlan* p) {
  memset(p, 0, sizeof(*p));
  p->struct_size = sizeof(*p);
  p->operation = op;
  p->row_count = rows;
  p->elements_per_row = width;
  p->strategy = PROM_REDUCTION_STRATEGY_FUSED_SINGLE_WORKGROUP;
  p->local_size = PROM_REDUCTION_LOCAL_SIZE;
  p->elements_per_partial = PROM_REDUCTION_ELEMENTS_PER_PARTIAL;
  p->partial_count = 1u;
  p->temporary_alignment_bytes = sizeof(float);
  const uint32_t role = op == PROM_REDUCTION_OPERATION_SUM   ? PROM_REDUCTION_STAGE_ROW_SUM
                        : op == PROM_REDUCTION_OPERATION_MAX ? PROM_REDUCTION_STAGE_ROW_MAX
                                                             : PROM_REDUCTION_STAGE_SOFTMAX_FUSED;
  plan_append(p, role, div_up(rows, 4u), width, 1u, 0u, 0u);
  p->replay_id = plan_replay_id(p);
}

bool find_nonfinite(const float* x, uint64_t count, uint64_t* index) {
  for (uint64_t i = 0; i < count; ++i) {
    if (!isfinite(x[i])) {
      *index = i;
      return true;
    }
  }
  return false;
}

int reduction_execute_once(void* handle, const PrometheusReductionRequest* request,
                           PrometheusReductionExecutionResult* dst, const ReductionLimits& lim, bool reference_plan) {
  PrometheusReductionExecutionResult local;
  PrometheusReductionExecutionResult& out = dst ? *dst : local;
  memset(&out, 0, sizeof(out));
  out.struct_size = sizeof(out);
  out.physical_slot_id = UINT32_MAX;
  out.first_nonfinite_index = UINT64_MAX;
  const uint64_t t0 = wall_ns();
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    out.stage = PROM_STAGE_INIT;
    out.detail_code = PROM_REDUCTION_DETAIL_RUNTIME_UNAVAILABLE;
    return PROM_INVALID_HANDLE;
  }
  out.stage = PROM_STAGE_INIT;
  out.detail_code = PROM_REDUCTION_DETAIL_INVALID_REQUEST;
  if (request == nullptr || request->struct_size < sizeof(*request)) return PROM_ERROR;
  if (request->input == nullptr) {
    out.detail_code = PROM_REDUCTION_DETAIL_NULL_INPUT;
    return PROM_ERROR;
  }
  if (request->output == nullptr) {
    out.detail_code = PROM_REDUCTION_DETAIL_NULL_OUTPUT;
    return PROM_ERROR;
  }
  const int32_t shape_detail = reduction_validate_shape(request, lim);
  if (shape_detail != 0) {
    out.detail_code = shape_detail;
    return PROM_ERROR;
  }
  const uint64_t total = request->input_element_count;
  uint64_t bad = 0;
  if (find_nonfinite(request->input, total, &bad)) {
    out.stage = PROM_STAGE_TRANSFER_IN;
    out.detail_code = PROM_REDUCTION_DETAIL_NONFINITE_INPUT;
    out.first_nonfinite_index = bad;
    return PROM_ERROR;
  }
  const uint32_t rows = request->row_count, width = request->elements_per_row, op = request->operation;
  if (reference_plan)
    build_reference_plan(request, &out.plan);
  else
    build_executed_plan(rows, width, op, &out.plan);
  if (!rt->available) {
    out.stage = PROM_STAGE_INIT;
    out.detail_code = PROM_REDUCTION_DETAIL_RUNTIME_UNAVAILABLE;
    return PROM_ERROR;
  }
  out.logical_request_id = ++rt->requests;
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  const uint64_t out_count = request->output_element_count;
  float* din = static_cast<float*>(staging(0, total * sizeof(float)));
  float* dout = static_cast<float*>(staging(2, out_count * sizeof(float)));
  if (din == nullptr || dout == nullptr) {
    out.detail_code = PROM_REDUCTION_DETAIL_RESOURCE_CREATE_FAILED;
    return PROM_ERROR;
  }
  out.stage = PROM_STAGE_TRANSFER_IN;
  if (upload_host(din, request->input, total * sizeof(float), cx.stream) != hipSuccess) {
    out.detail_code = PROM_REDUCTION_DETAIL_RESOURCE_CREATE_FAILED;
    return PROM_ERROR;
  }
  out.stage = PROM_STAGE_SUBMIT;
  if (rt->reduction_test_flags & (1u << 1)) {  // PROM_REDUCTION_TESTCFG_FAIL_QUEUE_SUBMIT
    (void)hipStreamSynchronize(cx.stream);
    out.detail_code = PROM_REDUCTION_DETAIL_QUEUE_SUBMIT_FAILED;
    return PROM_ERROR;
  }
  (void)hipEventRecord(cx.op_begin, cx.stream);
  if (launch_row_reduction(din, dout, rows, width, op, cx.stream) != hipSuccess) {
    (void)hipStreamSynchronize(cx.stream);
    out.detail_code = PROM_REDUCTION_DETAIL_COMMAND_RECORD_FAILED;
    return PROM_ERROR;
  }
  (void)hipEventRecord(cx.op_end, cx.stream);
  out.stage = PROM_STAGE_TRANSFER_OUT;
  if (download_host(request->output, dout, out_count * sizeof(float), cx.stream) != hipSuccess ||
      hipStreamSynchronize(cx.stream) != hipSuccess) {
    out.detail_code = PROM_REDUCTION_DETAIL_READBACK_FAILED;
    return PROM_ERROR;
  }
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, cx.op_begin, cx.op_end) == hipSuccess) {
    out.gpu_timestamp_valid = 1u;
    out.gpu_duration_ns = (uint64_t)((double)ms * 1.0e6);
  }
  out.physical_slot_id = 0u;
  out.physical_slot_recyclable = 1u;
  out.detail_code = 0;
  out.end_to_end_ns = wall_ns() - t0;
  rt->successes++;
  return PROM_OK;
}

// One reduction call, counted for the diagnostics entry.
int reduction_execute(void* handle, const PrometheusReductionRequest* request, PrometheusReductionExecutionResult* dst,
                      const ReductionLimits& lim, bool reference_plan) {
  PrometheusReductionExecutionResult local;
  PrometheusReductionExecutionResult* out = dst ? dst : &local;
  const int rc = reduction_execute_once(handle, request, out, lim, reference_plan);
  Runtime* rt = lookup(handle);
  if (rt != nullptr) {
    std::lock_guard<std::mutex> lock(ctx().mu);
    rt->reduction_total++;
    if (rc == PROM_OK) {
      rt->reduction_successes++;
      rt->reduction_last_replay = out->plan.replay_id;
      rt->reduction_last_gpu_ns = out->gpu_duration_ns;
      rt->reduction_last_e2e_ns = out->end_to_end_ns;
      rt->reduction_last_stages = out->plan.stage_count;
    } else {
      rt->reduction_failures++;
    }
    rt->reduction_last_detail = out->detail_code;
  }
  return rc;
}

// reactor_vulkan_fused_reduction.c:1044-1114: the benchmark's acceptance rule
// of `actual` against `expected`; fills the first mismatch.
bool reduction_outputs_agree(const PrometheusReductionRequest& r, const float* expected, const float* actual,
                             PrometheusReductionBenchmarkResult* res) {
  const bool softmax = r.operation == PROM_REDUCTION_OPERATION_SOFTMAX;
  const bool max_op = r.operation == PROM_REDUCTION_OPERATION_MAX;
  const uint64_t count = softmax ? r.input_element_count : r.row_count;
  const float abs_tol = softmax ? 2.0e-5f : (max_op ? 0.0f : 2.0e-5f * (float)r.elements_per_row);
  const float rel_tol = softmax ? 2.0e-4f : (max_op ? 0.0f : 2.0e-5f);
  auto mismatch = [&](uint32_t row, uint32_t col, float e, float a, float ae, float re) {
    res->first_mismatch_row = row;
    res->first_mismatch_column = col;
    res->first_expected = e;
    res->first_actual = a;
    res->first_absolute_error = ae;
    res->first_relative_error = re;
    return false;
  };
  for (uint64_t i = 0; i < count; ++i) {
    const float ae = fabsf(actual[i] - expected[i]);
    float den = fabsf(expected[i]);
    if (den < 1.0e-20f) den = 1.0f;
    const float re = ae / den;
    if (!isfinite(actual[i]) || (ae > abs_tol && re > rel_tol))
      return mismatch(softmax ? (uint32_t)(i / r.elements_per_row) : (uint32_t)i,
                      softmax ? (uint32_t)(i % r.elements_per_row) : UINT32_MAX, expected[i], actual[i], ae, re);
  }
  if (!softmax) return true;
  for (uint32_t row = 0; row < r.row_count; ++row) {
    double sum = 0.0;
    for (uint32_t c = 0; c < r.elements_per_row; ++c) {
      const float v = actual[(uint64_t)row * r.elements_per_row + c];
      if (!isfinite(v) || v < -2.0e-7f) return mismatch(row, c, 0.0f, v, fabsf(v), fabsf(v));
      sum += v;
    }
    if (fabs(sum - 1.0) > 3.0e-4)
      return mismatch(row, UINT32_MAX, 1.0f, (float)sum, (float)fabs(sum - 1.0), (float)fabs(sum - 1.0));
  }
  return true;
}

// -------------------------------------------------------------- RMSNorm

struct RmsArgs {
  const float* input;
  const float* weight;
  float* output;
  float* inv_rms;
  uint32_t tokens, width, stride;
  float eps;
};

// Host path shared by the Gemma and generic entries.  Returns PROM_* and sets stage/detail.
int rmsnorm_host(Runtime* rt, const RmsArgs& a, uint32_t* stage, int32_t* detail, uint64_t* gpu_ns) {
  const uint64_t in_count = (uint64_t)(a.tokens - 1u) * a.stride + a.width;
  for (uint64_t t = 0; t < a.tokens; ++t) {
    uint64_t bad;
    if (find_nonfinite(a.input + t * a.stride, a.width, &bad)) {
      *stage = PROM_STAGE_TRANSFER_IN;
      *detail = PROM_M46_DETAIL_NONFINITE_INPUT;
      return PROM_ERROR;
    }
  }
  uint64_t bad;
  if (find_nonfinite(a.weight, a.width, &bad)) {
    *stage = PROM_STAGE_TRANSFER_IN;
    *detail = PROM_M46_DETAIL_NONFINITE_INPUT;
    return PROM_ERROR;
  }
  if (!rt->available) {
    *stage = PROM_STAGE_INIT;
    *detail = rt->init_detail;
    return PROM_ERROR;
  }
  rt->requests++;
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  const uint64_t out_count = (uint64_t)a.tokens * a.width;
  float* din = static_cast<float*>(staging(0, in_count * sizeof(float)));
  float* dw = static_cast<float*>(staging(1, a.width * sizeof(float)));
  float* dout = static_cast<float*>(staging(2, out_count * sizeof(float)));
  float* dinv = static_cast<float*>(staging(3, a.tokens * sizeof(float)));
  if (!din || !dw || !dout || !dinv) {
    *stage = PROM_STAGE_TRANSFER_IN;
    *detail = PROM_DETAIL_HIP_ALLOC_FAILED;
    return PROM_ERROR;
  }
  *stage = PROM_STAGE_TRANSFER_IN;
  if (upload_host(din, a.input, in_count * sizeof(float), cx.stream) != hipSuccess ||
      upload_host(dw, a.weight, a.width * sizeof(float), cx.stream) != hipSuccess) {
    *detail = PROM_DETAIL_HIP_COPY_FAILED;
    return PROM_ERROR;
  }
  *stage = PROM_STAGE_SUBMIT;
  (void)hipEventRecord(cx.op_begin, cx.stream);
  if (launch_rmsnorm(din, dw, dout, dinv, a.tokens, a.width, a.stride, a.eps, cx.stream) != hipSuccess) {
    (void)hipStreamSynchronize(cx.stream);
    *detail = PROM_DETAIL_HIP_LAUNCH_FAILED;
    return PROM_ERROR;
  }
  (void)hipEventRecord(cx.op_end, cx.stream);
  *stage = PROM_STAGE_TRANSFER_OUT;
  if (download_host(a.output, dout, out_count * sizeof(float), cx.stream) != hipSuccess ||
      (a.inv_rms != nullptr &&
       download_host(a.inv_rms, dinv, a.tokens * sizeof(float), cx.stream) != hipSuccess) ||
      hipStreamSynchronize(cx.stream) != hipSuccess) {
    *detail = PROM_DETAIL_HIP_COPY_FAILED;
    return PROM_ERROR;
  }
  float ms = 0.f;
  if (gpu_ns && hipEventElapsedTime(&ms, cx.op_begin, cx.op_end) == hipSuccess) *gpu_ns = (uint64_t)((double)ms * 1e6);
  *detail = 0;
  rt->successes++;
  return PROM_OK;
}

}  // namespace

extern "C" {

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm(void* handle, const float* a, const float* b, float* c,
                                                      uint32_t m, uint32_t n, uint32_t k, uint32_t* out_stage,
                                                      int* out_detail_code) {
  // reactor_sgemm.cpp:4204-4211: no synchronous SGEMM while async tasks are unconsumed.
  if (Runtime* rt = lookup(handle); rt != nullptr && async_outstanding(rt) != 0u) {
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_ASYNC_UNCONSUMED);
    return PROM_ERROR;
  }
  return gemm_host<float>(handle, a, b, c, m, n, k, out_stage, out_detail_code, launch_sgemm_f32);
}

PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_device(void* handle, const float* a, const float* b, float* c,
                                                             uint32_t m, uint32_t n, uint32_t k, uint32_t* out_stage,
                                                             int* out_detail_code) {
  return gemm_device<float>(handle, a, b, c, m, n, k, out_stage, out_detail_code, launch_sgemm_f32);
}

// A caller-chosen SGEMM kernel variant (no reference counterpart): tuning and
// the per-variant parity tests run every kernel regardless of the plan model.
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_device_variant(void* handle, const float* a, const float* b,
                                                                     float* c, uint32_t m, uint32_t n, uint32_t k,
                                                                     uint32_t tile, uint32_t k_slices,
                                                                     uint32_t* out_stage, int* out_detail_code) {
  Runtime* rt = lookup(handle);
  const int v = gemm_validate(rt, a, b, c, m, n, k, out_stage, out_detail_code);
  if (v != PROM_OK) return v;
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  const hipError_t e = launch_sgemm_f32_variant(a, b, c, m, n, k, tile, k_slices, cx.stream);
  if (e == hipErrorInvalidValue) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_DETAIL_INVALID_ARGUMENT);
    return PROM_ERROR;
  }
  if (e != hipSuccess) {
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_HIP_LAUNCH_FAILED);
    return PROM_ERROR;
  }
  set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_PATH_HIP_MFMA_F32);
  return PROM_OK;
}

// bf16 flash attention on device pointers (no reference counterpart: the
// reference's attention exists only inside its Z-Image block shaders).  The
// DiT block calls the same launcher; this entry gives the kernel its own
// parity tests.  Scale 1/sqrt(128) (the block's).
PROM_REACTOR_API int prometheus_reactor_runtime_attention_bf16_device(void* handle, const uint16_t* q,
                                                                      const uint16_t* k, const uint16_t* v,
                                                                      uint16_t* o, uint32_t tokens, uint32_t heads,
                                                                      uint32_t ld, uint32_t variant,
                                                                      uint32_t* out_stage, int* out_detail_code) {
  Runtime* rt = lookup(handle);
  set_status(out_stage, out_detail_code, PROM_STAGE_NONE, 0);
  if (rt == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_INVALID_HANDLE);
    return PROM_INVALID_HANDLE;
  }
  auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const bool ok = q != nullptr && k != nullptr && v != nullptr && o != nullptr && aligned(q) && aligned(k) &&
                  aligned(v) && aligned(o) && tokens != 0u && heads != 0u && (uint64_t)heads * 128u <= ld &&
                  ld % 8u == 0u && ld < (1u << 24) && (uint64_t)tokens * ld * 2u <= 0x7fffffffull && variant <= 1u;
  if (!ok) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_DETAIL_INVALID_ARGUMENT);
    return PROM_ERROR;
  }
  if (!rt->available) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, rt->init_detail);
    return PROM_ERROR;
  }
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  if (launch_flash_attn_bf16(q, (int)ld, k, (int)ld, v, (int)ld, o, (int)ld, (int)tokens, (int)heads,
                             1.0f / sqrtf(128.0f), cx.stream, (int)variant) != hipSuccess) {
    (void)hipGetLastError();
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_HIP_LAUNCH_FAILED);
    return PROM_ERROR;
  }
  set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, 0);
  return PROM_OK;
}

// Allocation-free form of ..._sgemm_device (no reference counterpart): the
// lookup, validation, lock and launch path allocate nothing.
PROM_REACTOR_API int prometheus_reactor_runtime_sgemm_device_noalloc(void* handle, const float* a, const float* b,
                                                                     float* c, uint32_t m, uint32_t n, uint32_t k,
                                                                     uint32_t* out_stage, int* out_detail_code) {
  Runtime* rt = lookup(handle);
  const int v = gemm_validate(rt, a, b, c, m, n, k, out_stage, out_detail_code);
  if (v != PROM_OK) return v;
  DeviceContext& cx = ctx();
  std::lock_guard<std::mutex> lock(cx.mu);
  int path = 0;
  const int r = launch_sgemm_f32_noalloc(a, b, c, m, n, k, cx.device, cx.stream, &path);
  if (r == PROM_DETAIL_SCRATCH_LIMIT) {
    set_status(out_stage, out_detail_code, PROM_STAGE_TRANSFER_IN, PROM_DETAIL_SCRATCH_LIMIT);
    return PROM_ERROR;
  }
  if (r == PROM_DETAIL_SCRATCH_UNAVAILABLE) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_DETAIL_SCRATCH_UNAVAILABLE);
    return PROM_ERROR;
  }
  if (r != PROM_OK) {
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_HIP_LAUNCH_FAILED);
    return PROM_ERROR;
  }
  set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, path);
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_gemm_bf16(void* handle, const uint16_t* a, const uint16_t* b, float* c,
                                                          uint32_t m, uint32_t n, uint32_t k, uint32_t* out_stage,
                                                          int* out_detail_code) {
  return gemm_host<uint16_t>(handle, a, b, c, m, n, k, out_stage, out_detail_code, launch_gemm_bf16);
}

PROM_REACTOR_API int prometheus_reactor_runtime_gemm_bf16_device(void* handle, const uint16_t* a, const uint16_t* b,
                                                                 float* c, uint32_t m, uint32_t n, uint32_t k,
                                                                 uint32_t* out_stage, int* out_detail_code) {
  return gemm_device<uint16_t>(handle, a, b, c, m, n, k, out_stage, out_detail_code, launch_gemm_bf16);
}

PROM_REACTOR_API int prometheus_reactor_reduction_plan(const PrometheusReductionRequest* request,
                                                        PrometheusReductionPlan* out_plan) {
  if (out_plan == nullptr) return PROM_ERROR;
  memset(out_plan, 0, sizeof(*out_plan));
  out_plan->struct_size = sizeof(*out_plan);
  if (request == nullptr || request->struct_size < sizeof(*request)) return PROM_ERROR;
  if (reduction_validate_shape(request, kReferenceLimits) != 0) return PROM_ERROR;
  build_reference_plan(request, out_plan);
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_reduction(void* handle, const PrometheusReductionRequest* request,
                                                          PrometheusReductionExecutionResult* out_result) {
  return reduction_execute(handle, request, out_result, kReferenceLimits, true);
}

PROM_REACTOR_API int prometheus_reactor_runtime_reduction_diagnostics(void* handle,
                                                                      PrometheusReductionDiagnostics* out_diag) {
  if (out_diag == nullptr) return PROM_ERROR;
  memset(out_diag, 0, sizeof(*out_diag));
  out_diag->struct_size = sizeof(*out_diag);
  Runtime* rt = lookup(handle);
  if (rt == nullptr) return PROM_INVALID_HANDLE;
  std::lock_guard<std::mutex> lock(ctx().mu);
  out_diag->initialized = rt->available;
  out_diag->production_enabled = rt->available;
  out_diag->configured_ring_depth = 1u;  // one runtime stream
  out_diag->physical_slot_count = 1u;
  out_diag->next_logical_request_id = rt->requests + 1;
  out_diag->total_requests = rt->reduction_total;
  out_diag->successful_requests = rt->reduction_successes;
  out_diag->logical_failure_count = rt->reduction_failures;
  out_diag->physical_recycle_count = rt->reduction_successes;
  out_diag->command_record_count = rt->reduction_successes;  // one fused launch per call
  out_diag->queue_submit_count = rt->reduction_successes;
  out_diag->last_replay_id = rt->reduction_last_replay;
  out_diag->last_gpu_duration_ns = rt->reduction_last_gpu_ns;
  out_diag->last_end_to_end_ns = rt->reduction_last_e2e_ns;
  out_diag->last_stage_count = rt->reduction_last_stages;
  out_diag->last_detail_code = rt->reduction_last_detail;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_reduction_benchmark(void* handle,
                                                                    const PrometheusReductionBenchmarkRequest* request,
                                                                    PrometheusReductionBenchmarkResult* out_result) {
  if (out_result == nullptr) return PROM_ERROR;
  PrometheusReductionBenchmarkResult& res = *out_result;
  memset(&res, 0, sizeof(res));
  res.struct_size = sizeof(res);
  res.first_mismatch_row = UINT32_MAX;
  res.first_mismatch_column = UINT32_MAX;
  if (request == nullptr || request->struct_size < sizeof(*request) || request->measured_iterations == 0u ||
      request->measured_iterations > 10000u) {
    res.detail_code = PROM_REDUCTION_DETAIL_INVALID_REQUEST;
    return PROM_ERROR;
  }
  const PrometheusReductionRequest& r = request->reduction;
  PrometheusReductionExecutionResult er;
  std::vector<uint64_t> gpu, e2e;
  gpu.reserve(request->measured_iterations);
  e2e.reserve(request->measured_iterations);
  const uint64_t total = (uint64_t)request->warmup_iterations + request->measured_iterations;
  for (uint64_t it = 0; it < total; ++it) {
    if (reduction_execute(handle, &r, &er, kReferenceLimits, true) != PROM_OK) {
      res.detail_code = er.detail_code;
      return er.detail_code == PROM_REDUCTION_DETAIL_RUNTIME_UNAVAILABLE && lookup(handle) == nullptr
                 ? PROM_INVALID_HANDLE
                 : PROM_ERROR;
    }
    if (it >= request->warmup_iterations) {
      gpu.push_back(er.gpu_duration_ns);
      e2e.push_back(er.end_to_end_ns);
      res.completed_iterations += 1u;
    }
  }
  // the last output against the binary64 evaluation of the same rows on the device
  const bool softmax = r.operation == PROM_REDUCTION_OPERATION_SOFTMAX;
  const uint64_t out_count = softmax ? r.input_element_count : r.row_count;
  std::vector<float> expected(out_count);
  {
    DeviceContext& cx = ctx();
    std::lock_guard<std::mutex> lock(cx.mu);
    float* din = static_cast<float*>(staging(0, r.input_element_count * sizeof(float)));
    float* dexp = static_cast<float*>(staging(2, out_count * sizeof(float)));
    if (din == nullptr || dexp == nullptr ||
        upload_host(din, r.input, r.input_element_count * sizeof(float), cx.stream) != hipSuccess ||
        launch_row_reduction_check(din, dexp, r.row_count, r.elements_per_row, r.operation, cx.stream) !=
            hipSuccess ||
        download_host(expected.data(), dexp, out_count * sizeof(float), cx.stream) != hipSuccess ||
        hipStreamSynchronize(cx.stream) != hipSuccess) {
      (void)hipGetLastError();
      res.detail_code = PROM_REDUCTION_DETAIL_READBACK_FAILED;
      return PROM_ERROR;
    }
  }
  if (!reduction_outputs_agree(r, expected.data(), r.output, &res)) {
    res.detail_code = PROM_REDUCTION_DETAIL_READBACK_FAILED;
    return PROM_ERROR;
  }
  res.correctness_passed = 1u;
  res.validation_passed = 1u;  // no validation layer: its error count stays 0
  std::sort(gpu.begin(), gpu.end());
  std::sort(e2e.begin(), e2e.end());
  const size_t n = gpu.size();
  res.gpu_min_ns = gpu[0];
  res.gpu_median_ns = gpu[n / 2];
  res.gpu_max_ns = gpu[n - 1];
  res.end_to_end_min_ns = e2e[0];
  res.end_to_end_median_ns = e2e[n / 2];
  res.end_to_end_max_ns = e2e[n - 1];
  res.stage_count = er.plan.stage_count;
  res.temporary_bytes = er.plan.temporary_bytes;
  res.replay_id = er.plan.replay_id;
  res.detail_code = 0;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_reduction_v2(void* handle, const PrometheusReductionRequest* request,
                                                             PrometheusReductionExecutionResult* out_result) {
  return reduction_execute(handle, request, out_result, kLiftedLimits, false);
}

PROM_REACTOR_API int prometheus_reactor_runtime_reduction_device(void* handle, const float* input, float* output,
                                                                 uint32_t rows, uint32_t width, uint32_t operation,
                                                                 uint32_t* out_stage, int* out_detail_code) {
  set_status(out_stage, out_detail_code, PROM_STAGE_NONE, 0);
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_REDUCTION_DETAIL_RUNTIME_UNAVAILABLE);
    return PROM_INVALID_HANDLE;
  }
  PrometheusReductionRequest r;
  memset(&r, 0, sizeof(r));
  r.struct_size = sizeof(r);
  r.input = input;
  r.output = output;
  r.row_count = rows;
  r.elements_per_row = width;
  r.input_element_count = (uint64_t)rows * width;
  r.output_element_count = operation == PROM_REDUCTION_OPERATION_SOFTMAX ? r.input_element_count : rows;
  r.operation = operation;
  r.finalization = operation == PROM_REDUCTION_OPERATION_SOFTMAX ? PROM_REDUCTION_FINALIZATION_STABLE_SOFTMAX : 0u;
  if (input == nullptr || output == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT,
               input == nullptr ? PROM_REDUCTION_DETAIL_NULL_INPUT : PROM_REDUCTION_DETAIL_NULL_OUTPUT);
    return PROM_ERROR;
  }
  const int32_t d = reduction_validate_shape(&r, kLiftedLimits);
  if (d != 0) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, d);
    return PROM_ERROR;
  }
  if (!rt->available) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_REDUCTION_DETAIL_RUNTIME_UNAVAILABLE);
    return PROM_ERROR;
  }
  if (launch_row_reduction(input, output, rows, width, operation, ctx().stream) != hipSuccess) {
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_REDUCTION_DETAIL_COMMAND_RECORD_FAILED);
    return PROM_ERROR;
  }
  set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, 0);
  return PROM_OK;
}

// native/reactor_vulkan_fused_reduction.c:892-994
PROM_REACTOR_API int prometheus_reactor_runtime_row_wise_softmax(void* handle,
                                                                 const PrometheusRowWiseSoftmaxRequest* request,
                                                                 PrometheusRowWiseSoftmaxResult* out_result) {
  PrometheusRowWiseSoftmaxResult local;
  PrometheusRowWiseSoftmaxResult& res = out_result ? *out_result : local;
  memset(&res, 0, sizeof(res));
  res.struct_size = sizeof(res);
  res.first_nonfinite_index = UINT64_MAX;
  auto fail = [&](uint32_t stage, int32_t detail) {
    res.stage = stage;
    res.detail_code = detail;
    res.output_written = 0u;
    return PROM_ERROR;
  };
  if (request == nullptr || request->struct_size < sizeof(*request))
    return fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_INVALID_REQUEST);
  const uint64_t total = (uint64_t)request->row_count * (uint64_t)request->elements_per_row;
  if (request->input_element_count != total || request->output_element_count != total)
    return fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_COUNT_MISMATCH);
  if (total == 0u) {
    res.stage = PROM_STAGE_NONE;
    res.detail_code = 0;
    return PROM_OK;
  }
  if (request->input == nullptr) return fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_NULL_INPUT);
  if (request->output == nullptr) return fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_NULL_OUTPUT);
  if (request->row_count > PROM_ROW_WISE_SOFTMAX_MAX_ROWS) return fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_ROW_LIMIT);
  if (request->elements_per_row > PROM_ROW_WISE_SOFTMAX_MAX_ELEMENTS_PER_ROW)
    return fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_WIDTH_LIMIT);
  if (total > PROM_ROW_WISE_SOFTMAX_MAX_TOTAL_ELEMENTS) return fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_ELEMENT_LIMIT);
  {
    const uintptr_t ib = reinterpret_cast<uintptr_t>(request->input);
    const uintptr_t ob = reinterpret_cast<uintptr_t>(request->output);
    const uint64_t bytes = total * sizeof(float);
    if (ib != ob) {
      const bool overflow = ib > UINTPTR_MAX - bytes || ob > UINTPTR_MAX - bytes;
      if (overflow || (ib < ob + bytes && ob < ib + bytes)) return fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_PARTIAL_ALIAS);
    }
  }
  uint64_t bad = 0;
  if (find_nonfinite(request->input, total, &bad)) {
    res.first_nonfinite_index = bad;
    return fail(PROM_STAGE_TRANSFER_IN, PROM_SOFTMAX_DETAIL_NONFINITE_INPUT);
  }
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_RUNTIME_UNAVAILABLE);
    return PROM_INVALID_HANDLE;
  }
  if (!rt->available) return fail(PROM_STAGE_INIT, PROM_SOFTMAX_DETAIL_RUNTIME_UNAVAILABLE);
  PrometheusReductionRequest r;
  memset(&r, 0, sizeof(r));
  r.struct_size = sizeof(r);
  r.input = request->input;
  r.output = request->output;
  r.row_count = request->row_count;
  r.elements_per_row = request->elements_per_row;
  r.input_element_count = total;
  r.output_element_count = total;
  r.operation = PROM_REDUCTION_OPERATION_SOFTMAX;
  r.finalization = PROM_REDUCTION_FINALIZATION_STABLE_SOFTMAX;
  r.flags = PROM_REDUCTION_FLAG_FORCE_FUSED;
  PrometheusReductionExecutionResult er;
  const int status = reduction_execute(handle, &r, &er, kReferenceLimits, true);
  res.stage = er.stage;
  res.detail_code = er.detail_code;
  res.gpu_timestamp_valid = er.gpu_timestamp_valid;
  res.gpu_duration_ns = er.gpu_duration_ns;
  res.end_to_end_ns = er.end_to_end_ns;
  res.first_nonfinite_index = er.first_nonfinite_index;
  if (status != PROM_OK) return status;
  res.physical_dispatch_count = 1u;
  res.physical_submission_count = 1u;
  res.output_written = 1u;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_rmsnorm(void* handle, const PrometheusRmsNormRequest* request,
                                                        PrometheusRmsNormResult* out_result) {
  if (out_result == nullptr) return PROM_ERROR;
  memset(out_result, 0, sizeof(*out_result));
  out_result->struct_size = sizeof(*out_result);
  const uint64_t t0 = wall_ns();
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    out_result->stage = PROM_STAGE_INIT;
    out_result->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
    return PROM_INVALID_HANDLE;
  }
  const PrometheusRmsNormRequest* r = request;
  if (r == nullptr || r->struct_size < sizeof(*r) || r->input == nullptr || r->weight == nullptr ||
      r->output == nullptr || r->tokens == 0u || r->width == 0u) {
    out_result->stage = PROM_STAGE_INIT;
    out_result->detail_code = PROM_M46_DETAIL_INVALID_REQUEST;
    return PROM_ERROR;
  }
  if (r->input_row_stride < r->width) {
    out_result->stage = PROM_STAGE_INIT;
    out_result->detail_code = PROM_M46_DETAIL_STRIDE;
    return PROM_ERROR;
  }
  if ((uint64_t)r->tokens * r->input_row_stride > (1ull << 32)) {
    out_result->stage = PROM_STAGE_INIT;
    out_result->detail_code = PROM_M46_DETAIL_SIZE_OVERFLOW;
    return PROM_ERROR;
  }
  if (!isfinite(r->epsilon) || r->epsilon <= 0.0f) {
    out_result->stage = PROM_STAGE_INIT;
    out_result->detail_code = PROM_M46_DETAIL_EPSILON;
    return PROM_ERROR;
  }
  RmsArgs a{r->input, r->weight, r->output, r->inv_rms_output, r->tokens, r->width, r->input_row_stride, r->epsilon};
  uint32_t stage = PROM_STAGE_NONE;
  int32_t detail = 0;
  uint64_t gpu_ns = 0;
  const int status = rmsnorm_host(rt, a, &stage, &detail, &gpu_ns);
  out_result->stage = stage;
  out_result->detail_code = detail;
  out_result->gpu_duration_ns = gpu_ns;
  out_result->end_to_end_ns = wall_ns() - t0;
  if (status != PROM_OK) return status;
  out_result->output_written = 1u;
  return PROM_OK;
}

PROM_REACTOR_API int prometheus_reactor_runtime_rmsnorm_device(void* handle, const float* input, const float* weight,
                                                               float* output, float* inv_rms, uint32_t tokens,
                                                               uint32_t width, uint32_t input_row_stride, float epsilon,
                                                               uint32_t* out_stage, int* out_detail_code) {
  set_status(out_stage, out_detail_code, PROM_STAGE_NONE, 0);
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_M46_DETAIL_INVALID_REQUEST);
    return PROM_INVALID_HANDLE;
  }
  if (input == nullptr || weight == nullptr || output == nullptr || tokens == 0u || width == 0u ||
      input_row_stride < width || !isfinite(epsilon) || epsilon <= 0.0f) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, PROM_M46_DETAIL_INVALID_REQUEST);
    return PROM_ERROR;
  }
  if (!rt->available) {
    set_status(out_stage, out_detail_code, PROM_STAGE_INIT, rt->init_detail);
    return PROM_ERROR;
  }
  if (launch_rmsnorm(input, weight, output, inv_rms, tokens, width, input_row_stride, epsilon, ctx().stream) !=
      hipSuccess) {
    set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, PROM_DETAIL_HIP_LAUNCH_FAILED);
    return PROM_ERROR;
  }
  set_status(out_stage, out_detail_code, PROM_STAGE_SUBMIT, 0);
  return PROM_OK;
}

}  // extern "C"
