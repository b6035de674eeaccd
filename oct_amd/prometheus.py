"""Host-side bridge to the MI355X Prometheus reactor.

This module mirrors the reference's Go bridge (``internal/prometheus``) over the
same C ABI, using ``ctypes``: library discovery (``bridge.go:552-601``), ABI
check / create / probe (``bridge.go:276-394``), ``nativeRuntime.SGEMM``
(``bridge.go:410-436``), status mapping (``status.go``, ``bridge.go:535-550``)
and the strict ``@`` path that never substitutes the CPU
(``strict.go:11-32``).  The Go toolchain is absent from this image, so the
host side is Python, over the same exported symbols a cgo binding resolves.

Everything here calls the HIP library.  There is no CPU fallback: a missing
library or device raises :class:`ReactorIssue`.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, byref, c_char, c_float, c_int, c_uint16, c_uint32, c_uint64, c_void_p
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Sequence, Tuple

import numpy as np

REACTOR_ENV_VAR = "OCT_PROMETHEUS_REACTOR"
REACTOR_TEST_FLAGS_ENV_VAR = "OCT_PROMETHEUS_REACTOR_TEST_FLAGS"
REACTOR_EXPECTED_ABI_VERSION = 1
LIBRARY_BASENAME = "libprometheus_reactor.so"
PACKAGE_DIR = Path(__file__).resolve().parent

# ---- ABI constants (include/prometheus_reactor.h) --------------------------
PROM_OK, PROM_ERROR, PROM_INVALID_HANDLE, PROM_INTERNAL_ERROR = 0, 1, 2, 3
PROM_BACKEND_UNKNOWN, PROM_BACKEND_STUB, PROM_BACKEND_HARDWARE_GPU, PROM_BACKEND_SOFTWARE = 0, 1, 2, 3
PROM_REASON_NONE, PROM_REASON_STUB_UNAVAILABLE, PROM_REASON_VULKAN_UNAVAILABLE = 0, 1, 2
STAGE_NONE, STAGE_INIT, STAGE_TRANSFER_IN, STAGE_SUBMIT, STAGE_TRANSFER_OUT, STAGE_CLEANUP = range(6)
OP_SUM, OP_MAX, OP_SOFTMAX = 1, 2, 3
# row-reduction details (reactor_api.h:404-430)
REDUCTION_DETAIL = {"INVALID_REQUEST": -6801, "NULL_INPUT": -6802, "NULL_OUTPUT": -6803,
                    "RESOURCE_CREATE_FAILED": -6818, "READBACK_FAILED": -6824, "RUNTIME_UNAVAILABLE": -6825}
FINALIZATION_NONE, FINALIZATION_STABLE_SOFTMAX = 0, 1
FLAG_FORCE_FUSED, FLAG_FORCE_COMPOSED = 1, 2
TESTCFG_FAIL_DEVICE_CREATE = 1 << 0
TESTCFG_FAIL_BUFFER_ALLOC = 1 << 2
TESTCFG_FAIL_UPLOAD = 1 << 3
TESTCFG_FAIL_DISPATCH = 1 << 4
TESTCFG_FAIL_DOWNLOAD = 1 << 5
TESTCFG_SKIP_VULKAN_INIT = 1 << 7
TESTCFG_FAIL_ASYNC_POLL = 1 << 15
TESTCFG_FAIL_COMMAND_END = 1 << 20
TESTCFG_FAIL_QUEUE_SUBMIT = 1 << 22
DETAIL_INJECTED_UPLOAD_FAILURE = -6001
DETAIL_INJECTED_DISPATCH_FAILURE = -6002
DETAIL_INJECTED_DOWNLOAD_FAILURE = -6003
DETAIL_SIZE_OVERFLOW = -6004
DETAIL_PATH_HIP_MFMA_F32 = 6120
DETAIL_PATH_HIP_GEMV_F32 = 6121
DETAIL_PATH_HIP_MFMA_BF16 = 6122
DETAIL_HIP_UNAVAILABLE = -6905
DETAIL_INVALID_ARGUMENT = -6906
DETAIL_SCRATCH_LIMIT = -6930
DETAIL_SCRATCH_UNAVAILABLE = -6931
SGEMM_NOALLOC_SCRATCH_BYTES = 64 << 20
# async and batch (reactor_api.h:84-114, 250-260, 282-295, 1448-1545)
ASYNC_IDLE, ASYNC_SUBMITTED, ASYNC_READY, ASYNC_FAILED, ASYNC_CONSUMED = range(5)
DETAIL_ASYNC_NOT_READY = -6108
DETAIL_ASYNC_NO_TASK = -6109
DETAIL_ASYNC_ALREADY_CONSUMED = -6110
DETAIL_ASYNC_INVALID_TASK = -6111
DETAIL_ASYNC_FAILED = -6114
DETAIL_ASYNC_UNCONSUMED = -6115
DETAIL_INJECTED_ASYNC_POLL_FAILURE = -6116
DETAIL_ASYNC_QUEUE_FULL = -6117
DETAIL_BATCH_PLAN_INVALID = -6602
DETAIL_BATCH_EXECUTION_FAILED = -6604
DETAIL_BATCH_UNSUPPORTED_OPTION = -6613
BATCH_FLAG_PARTITION_CONTIGUOUS = 1 << 8
BATCH_FLAG_FAIL_AFTER_FIRST_SUBMIT = 1 << 9
BATCH_FLAG_TEST_SEPARATE_COMPUTE_FAMILY = 1 << 10
BATCH_FLAG_TEST_DUAL_FAIL_FIRST_TWO = 1 << 22
BATCH_FLAG_TEST_FAIL_ENTRY_SHIFT = 24
BATCH_PARTITION_ROUND_ROBIN, BATCH_PARTITION_CONTIGUOUS = 1, 2
BATCH_STATE_FAILED, BATCH_STATE_SUCCEEDED = 5, 6
BATCH_EXECUTION_SINGLE_WORKER = 1
# FFT (reactor_api.h:361-379)
DETAIL_FFT_INVALID_REQUEST = -6702
DETAIL_FFT_VULKAN_UNAVAILABLE = -6712
# Gemma-4-E2B M1 (reactor_vulkan.h:1869-1888)
DETAIL_M46_INVALID_REQUEST = -7401
DETAIL_M46_STALE_WEIGHT_GENERATION = -7406
DETAIL_M46_RESOURCE = -7411
DETAIL_M46_NONFINITE_INPUT = -7418


# ---- ABI structs -----------------------------------------------------------
def _fields(spec: str):
    """'u32 a, u64 b, f32 c, p d, i32 e' -> ctypes field list."""
    kinds = {"u32": c_uint32, "u64": c_uint64, "f32": c_float, "p": c_void_p, "i32": ctypes.c_int32}
    out = []
    for item in spec.split(","):
        kind, name = item.split()
        out.append((name, kinds[kind]))
    return out


class PrometheusCaps(Structure):
    _fields_ = [("available", c_uint32), ("backend_type", c_uint32), ("reason_code", c_uint32)]


class PrometheusReactorConfig(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("test_flags", c_uint32),
        ("p15_shadow_disabled", c_uint32),
        ("async_test_flags", c_uint32),
        ("batch_ring_depth", c_uint32),
        ("reduction_test_flags", c_uint32),
        ("reduction_ring_depth", c_uint32),
        ("shader_package_root", ctypes.c_char_p),
    ]


class PrometheusVulkanDeviceDiagnostics(Structure):
    _fields_ = [
        ("device_name", c_char * 256),
        ("vendor_id", c_uint32),
        ("device_id", c_uint32),
        ("device_type", c_uint32),
        ("driver_version", c_uint32),
        ("api_version", c_uint32),
        ("software_vulkan", c_uint32),
        ("compute_queue_family", c_uint32),
        ("transfer_queue_family", c_uint32),
    ]


class PrometheusSgemmPlanInfo(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("detail_code", ctypes.c_int32),
        ("products", c_uint32),
        ("head_rows", c_uint32),
        ("tile_m", c_uint32 * 2),
        ("tile_n", c_uint32 * 2),
        ("direct_to_lds", c_uint32 * 2),
        ("k_slices", c_uint32 * 2),
        ("k_slice_len", c_uint32 * 2),
        ("launches", c_uint32),
        ("repacked", c_uint32),
        ("partial_bytes", c_uint64),
        ("estimated_us", ctypes.c_double),
        ("repack_bytes", c_uint64),
        ("scratch_bytes", c_uint64),
    ]


class PrometheusHipDeviceDiagnostics(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("device_name", c_char * 256),
        ("gcn_arch_name", c_char * 64),
        ("compute_units", c_uint32),
        ("clock_khz", c_uint32),
        ("memory_clock_khz", c_uint32),
        ("memory_bus_width", c_uint32),
        ("total_global_mem", c_uint64),
        ("lds_bytes_per_workgroup", c_uint32),
        ("wavefront_size", c_uint32),
        ("hip_runtime_version", ctypes.c_int32),
        ("device_ordinal", ctypes.c_int32),
        ("staging_allocations", c_uint64),
        ("staging_bytes", c_uint64),
    ]


class PrometheusReductionRequest(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("input", c_void_p),
        ("output", c_void_p),
        ("row_count", c_uint32),
        ("elements_per_row", c_uint32),
        ("input_element_count", c_uint64),
        ("output_element_count", c_uint64),
        ("operation", c_uint32),
        ("finalization", c_uint32),
        ("flags", c_uint32),
    ]


class PrometheusReductionStageDispatch(Structure):
    _fields_ = [
        ("stage_role", c_uint32),
        ("shader_id", c_uint32),
        ("implementation_id", c_uint32),
        ("groups_x", c_uint32),
        ("groups_y", c_uint32),
        ("groups_z", c_uint32),
        ("input_elements_per_row", c_uint32),
        ("output_partials_per_row", c_uint32),
        ("temporary_role", c_uint32),
        ("temporary_bytes_written", c_uint64),
    ]


class PrometheusReductionPlan(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("operation", c_uint32),
        ("row_count", c_uint32),
        ("elements_per_row", c_uint32),
        ("strategy", c_uint32),
        ("local_size", c_uint32),
        ("elements_per_partial", c_uint32),
        ("partial_count", c_uint32),
        ("stage_count", c_uint32),
        ("temporary_alignment_bytes", c_uint32),
        ("temporary_bytes", c_uint64),
        ("replay_id", c_uint64),
        ("stages", PrometheusReductionStageDispatch * 8),
    ]


class PrometheusReductionExecutionResult(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("stage", c_uint32),
        ("detail_code", ctypes.c_int32),
        ("logical_request_id", c_uint64),
        ("physical_slot_id", c_uint32),
        ("physical_slot_generation", c_uint32),
        ("physical_slot_recyclable", c_uint32),
        ("gpu_timestamp_valid", c_uint32),
        ("gpu_duration_ns", c_uint64),
        ("end_to_end_ns", c_uint64),
        ("first_nonfinite_index", c_uint64),
        ("validation_error_count_before", c_uint32),
        ("validation_error_count_after", c_uint32),
        ("plan", PrometheusReductionPlan),
    ]


class PrometheusReductionDiagnostics(Structure):
    """reactor_api.h:600-633"""
    _fields_ = _fields(
        "u32 struct_size, u32 initialized, u32 production_enabled, u32 experimental_enabled, "
        "u32 configured_ring_depth, u32 physical_slot_count, u32 acquire_cursor, u32 outstanding_slots, "
        "u32 quarantined_slots, u64 next_logical_request_id, u64 total_requests, u64 successful_requests, "
        "u64 logical_failure_count, u64 physical_recycle_count, u64 quarantine_count, u64 reap_count, "
        "u64 pipeline_create_count, u64 descriptor_update_count, u64 command_record_count, u64 queue_submit_count, "
        "u64 buffer_allocation_count, u64 buffer_reuse_count, u64 temporary_capacity_bytes, u64 last_replay_id, "
        "u64 last_gpu_duration_ns, u64 last_end_to_end_ns, u32 last_stage_count, u32 last_physical_slot_id, "
        "u32 last_physical_slot_generation, i32 last_detail_code, u32 validation_enabled, "
        "u32 validation_error_count")


class PrometheusReductionBenchmarkRequest(Structure):
    """reactor_api.h:635-640"""
    _fields_ = [("struct_size", c_uint32), ("reduction", PrometheusReductionRequest),
                ("warmup_iterations", c_uint32), ("measured_iterations", c_uint32)]


class PrometheusReductionBenchmarkResult(Structure):
    """reactor_api.h:642-664"""
    _fields_ = _fields(
        "u32 struct_size, u32 completed_iterations, u32 correctness_passed, u32 validation_passed, u32 device_lost, "
        "u32 stage_count, u64 temporary_bytes, u64 replay_id, u64 gpu_min_ns, u64 gpu_median_ns, u64 gpu_max_ns, "
        "u64 end_to_end_min_ns, u64 end_to_end_median_ns, u64 end_to_end_max_ns, u32 first_mismatch_row, "
        "u32 first_mismatch_column, f32 first_expected, f32 first_actual, f32 first_absolute_error, "
        "f32 first_relative_error, i32 detail_code")


class PrometheusRowWiseSoftmaxRequest(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("input", c_void_p),
        ("output", c_void_p),
        ("row_count", c_uint32),
        ("elements_per_row", c_uint32),
        ("input_element_count", c_uint64),
        ("output_element_count", c_uint64),
    ]


class PrometheusRowWiseSoftmaxResult(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("stage", c_uint32),
        ("detail_code", ctypes.c_int32),
        ("output_written", c_uint32),
        ("physical_dispatch_count", c_uint32),
        ("physical_submission_count", c_uint32),
        ("gpu_timestamp_valid", c_uint32),
        ("gpu_duration_ns", c_uint64),
        ("end_to_end_ns", c_uint64),
        ("first_nonfinite_index", c_uint64),
    ]


class PrometheusGemma4E2BM1InputRmsNormRequest(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("input", c_void_p),
        ("weight", c_void_p),
        ("output", c_void_p),
        ("inv_rms_output", c_void_p),
        ("input_element_count", c_uint64),
        ("weight_element_count", c_uint64),
        ("output_element_count", c_uint64),
        ("inv_rms_output_element_count", c_uint64),
        ("tokens", c_uint32),
        ("model_width", c_uint32),
        ("input_row_stride", c_uint32),
        ("epsilon", c_float),
        ("input_generation", c_uint64),
        ("weight_generation", c_uint64),
        ("exact_source_hash", c_uint64),
    ]


class PrometheusGemma4E2BM1InputRmsNormResult(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("stage", c_uint32),
        ("detail_code", ctypes.c_int32),
        ("output_written", c_uint32),
        ("matched_input", c_uint32),
        ("input_hash", c_uint64),
        ("weight_hash", c_uint64),
        ("output_hash", c_uint64),
        ("inv_rms_hash", c_uint64),
        ("submit_count", c_uint32),
        ("final_readback_count", c_uint32),
        ("no_product_intermediate_readback_change", c_uint32),
        ("reserved0", c_uint32),
        ("retained_bytes", c_uint64),
        ("buffer_allocation_count", c_uint64),
        ("buffer_reuse_count", c_uint64),
        ("descriptor_update_count", c_uint64),
        ("pipeline_create_count", c_uint64),
        ("command_buffer_reuse_count", c_uint64),
        ("reduction_gpu_ns", c_uint64),
        ("final_reduction_gpu_ns", c_uint64),
        ("inv_rms_gpu_ns", c_uint64),
        ("apply_gpu_ns", c_uint64),
        ("end_to_end_ns", c_uint64),
    ]


class PrometheusRmsNormRequest(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("input", c_void_p),
        ("weight", c_void_p),
        ("output", c_void_p),
        ("inv_rms_output", c_void_p),
        ("tokens", c_uint32),
        ("width", c_uint32),
        ("input_row_stride", c_uint32),
        ("epsilon", c_float),
    ]


class PrometheusRmsNormResult(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("stage", c_uint32),
        ("detail_code", ctypes.c_int32),
        ("output_written", c_uint32),
        ("gpu_duration_ns", c_uint64),
        ("end_to_end_ns", c_uint64),
    ]


class PrometheusDecoderLayerF32Request(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("tokens", c_uint32),
        ("hidden", c_uint32),
        ("q_heads", c_uint32),
        ("kv_heads", c_uint32),
        ("head_dim", c_uint32),
        ("ffn_hidden", c_uint32),
        ("position_offset", c_uint32),
        ("rms_epsilon", c_float),
        ("rope_base", c_float),
        ("input", c_void_p),
        ("attn_norm_weight", c_void_p),
        ("w_qkv", c_void_p),
        ("w_o", c_void_p),
        ("ffn_norm_weight", c_void_p),
        ("w_gate_up", c_void_p),
        ("w_down", c_void_p),
        ("output", c_void_p),
    ]


class PrometheusDitBlockBf16Request(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("tokens", c_uint32),
        ("hidden", c_uint32),
        ("heads", c_uint32),
        ("head_dim", c_uint32),
        ("ffn_hidden", c_uint32),
        ("cond_dim", c_uint32),
        ("rope_axes", c_uint32 * 3),
        ("rope_theta", c_float),
        ("rms_epsilon", c_float),
        ("input", c_void_p),
        ("coordinates", c_void_p),
        ("condition", c_void_p),
        ("w_adaln", c_void_p),
        ("b_adaln", c_void_p),
        ("attn_norm1", c_void_p),
        ("attn_norm2", c_void_p),
        ("ffn_norm1", c_void_p),
        ("ffn_norm2", c_void_p),
        ("q_norm", c_void_p),
        ("k_norm", c_void_p),
        ("w_qkv", c_void_p),
        ("w_out", c_void_p),
        ("w_13", c_void_p),
        ("w_2", c_void_p),
        ("output", c_void_p),
    ]


class PrometheusBlockResult(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("stage", c_uint32),
        ("detail_code", ctypes.c_int32),
        ("output_written", c_uint32),
        ("kernel_launches", c_uint32),
        ("reserved0", c_uint32),
        ("gpu_duration_ns", c_uint64),
        ("end_to_end_ns", c_uint64),
        ("workspace_bytes", c_uint64),
    ]


class PrometheusAsyncStatus(Structure):
    _fields_ = [("lifecycle_state", c_uint32), ("stage", c_uint32), ("detail_code", c_int),
                ("ready", c_uint32), ("failed", c_uint32), ("consumed", c_uint32), ("outstanding_tasks", c_uint32)]


class PrometheusSgemmBatchEntry(Structure):
    _fields_ = [("a", c_void_p), ("b", c_void_p), ("c", c_void_p), ("m", c_uint32), ("n", c_uint32), ("k", c_uint32)]


def _u32(name, count=None):
    return (name, c_uint32 * count) if count else (name, c_uint32)


class PrometheusSgemmBatchDiagnostics(Structure):
    """reactor_api.h:1316-1447, field for field."""
    _fields_ = (
        [_u32(f) for f in (
            "last_batch_entry_count", "requested_workers", "effective_workers", "hardware_queue_cap",
            "memory_worker_cap", "worker_cap_reason", "partition_policy", "batch_state", "failed_entry_id",
            "failed_worker_id", "failure_stage")]
        + [("failure_detail", ctypes.c_int32)]
        + [_u32(f) for f in (
            "failure_count", "first_failure_stable", "event_overflow_count", "event_drain_count", "output_committed",
            "plan_generation", "worker_judgment_count", "execution_mode", "worker_resource_mode",
            "queue_topology_classification", "queue_mapping_mode", "lane_worker_count", "real_worker_thread_count",
            "serialized_vulkan", "serialized_bridge_enter_count", "serialized_execution_count",
            "serialized_wait_count", "max_concurrent_serialized_entries", "hardware_parallelism_claimed",
            "resource_ownership_violation_count", "resource_creation_failure_count", "worker_active_mask")]
        + [_u32(f, 8) for f in (
            "worker_assigned_count", "worker_completed_count", "worker_event_count", "worker_queue_index",
            "worker_submit_count", "worker_wait_count", "worker_in_flight", "worker_slot_id",
            "worker_output_staging_id", "worker_arena_bank_id", "worker_command_pool_id",
            "worker_command_buffer_id", "worker_fence_id", "worker_command_pool_valid",
            "worker_command_buffer_valid", "worker_fence_valid", "worker_reset_count", "worker_record_count",
            "worker_failure_stage")]
        + [("worker_failure_detail", ctypes.c_int32 * 8)]
        + [_u32(f) for f in (
            "reported_compute_queue_count", "independent_compute_queue_count", "true_multi_queue_selected",
            "hardware_parallelism_eligible", "serialized_fallback_reason")]
        + [_u32(f, 8) for f in ("per_worker_queue_family", "per_worker_fence_state")]
        + [_u32(f) for f in (
            "queue_drain_count", "drain_timeout_count", "queue_family_ownership_handoff_count",
            "transfer_compute_sync_wait_count", "unsafe_to_reuse", "slots_per_worker_target",
            "effective_slots_per_worker", "total_slot_count", "slot_cap_reason", "slot_refill_count",
            "slot_full_scan_poll_count", "slot_attention_poll_count", "slot_polling_avoided_count",
            "slot_failure_count", "slot_drain_count", "slot_boundary_generation", "slot_dirty_mask",
            "slot_ready_mask", "slot_failed_mask", "slot_invalidated_mask", "slot_attention_mask")]
        + [_u32(f, 16) for f in (
            "slot_owner_worker_id", "slot_state", "slot_generation", "slot_entry_id", "slot_queue_id",
            "slot_command_resource_id", "slot_arena_id", "slot_output_staging_id", "slot_in_flight", "slot_ready",
            "slot_invalidated", "slot_failure_stage")]
        + [("slot_failure_detail", ctypes.c_int32 * 16)]
        + [(f, c_uint64) for f in (
            "p13_m10_lease_request_count", "p13_m10_lease_grant_count", "p13_m10_lease_deny_count",
            "p13_m10_lease_yield_count")]
        + [_u32(f) for f in (
            "p13_m10_lease_last_state", "p13_m10_lease_last_deny_reason", "p13_m10_lookahead_requested",
            "p13_m10_lookahead_allowed", "p13_m10_lookahead_blocked_reason", "p13_m10_selected_recipe_variant",
            "physical_ring_depth_configured", "physical_ring_depth_effective", "current_in_flight", "max_in_flight")]
        + [(f, c_uint64) for f in (
            "total_submits", "total_polls", "total_forced_waits", "ring_full_count", "refill_count",
            "query_harvest_count", "quarantine_count", "reap_count", "feedback_committed_count",
            "feedback_skipped_count")]
        + [_u32("m31_completion_count"), _u32("m31_commit_count"), ("m31_submission_sequence", c_uint64 * 64),
           _u32("m31_physical_slot_id", 64), _u32("m31_completion_status", 64), ("m31_gpu_duration_ns", c_uint64 * 64),
           _u32("m31_completion_order", 64), _u32("m31_commit_order", 64)]
    )


class PrometheusSgemmAsyncTaskDiagnostics(Structure):
    _fields_ = [("task_id", ctypes.c_int32), ("generation", c_uint32), ("lifecycle_state", c_uint32),
                ("physical_slot_id", c_uint32), ("physical_slot_generation", c_uint32),
                ("submission_sequence", c_uint64), ("timing_valid", c_uint32), ("gpu_duration_ns", c_uint64),
                ("feedback_pending", c_uint32), ("feedback_committed", c_uint32), ("failure_detail", ctypes.c_int32),
                ("failure_class", c_uint32), ("abandoned", c_uint32), ("physical_slot_state", c_uint32),
                ("quarantined", c_uint32), ("physical_completion_confirmed", c_uint32), ("reap_pending", c_uint32),
                ("reap_completed", c_uint32)]


class PrometheusSgemmAsyncDiagnostics(Structure):
    _fields_ = [("task_capacity", c_uint32), ("active_task_count", c_uint32), ("submitted_count", c_uint32),
                ("ready_count", c_uint32), ("failed_count", c_uint32), ("consumed_count", c_uint32),
                ("abandoned_count", c_uint32), ("queue_full_count", c_uint64), ("stale_id_rejection_count", c_uint64),
                ("max_in_flight", c_uint32), ("feedback_pending_count", c_uint32),
                ("feedback_committed_count", c_uint64), ("feedback_skipped_count", c_uint64),
                ("next_feedback_sequence", c_uint64), ("quarantined_slot_count", c_uint32),
                ("quarantine_event_count", c_uint64), ("reap_poll_count", c_uint64), ("reap_success_count", c_uint64),
                ("reap_wait_count", c_uint64), ("reap_failure_count", c_uint64), ("max_quarantine_depth", c_uint32),
                ("runtime_unsafe_to_reuse", c_uint32), ("tasks", PrometheusSgemmAsyncTaskDiagnostics * 4)]


class PrometheusGemma4E2BM1RopeRequest(Structure):
    """reactor_api.h:1837-1852"""
    _fields_ = _fields("u32 struct_size, p source, p cosine, p sine, p output, u64 source_element_count, "
                       "u64 cosine_element_count, u64 sine_element_count, u64 output_element_count, u32 tokens, "
                       "u32 heads, u32 head_width, u32 reserved0, u64 source_generation, u64 table_generation")


class PrometheusGemma4E2BM1RopeResult(Structure):
    _fields_ = _fields("u32 struct_size, u32 stage, i32 detail_code, u32 output_written, u32 dispatch_count, "
                       "u64 source_hash, u64 cosine_hash, u64 sine_hash, u64 output_hash, "
                       "u64 buffer_allocation_count, u64 buffer_reuse_count, u64 descriptor_update_count, "
                       "u64 pipeline_create_count, u64 command_buffer_reuse_count")


class PrometheusGemma4E2BM1HeadRmsNormRopeRequest(Structure):
    """reactor_api.h:1875-1897"""
    _fields_ = _fields("u32 struct_size, p input, p weight, p cosine, p sine, p output, u64 input_element_count, "
                       "u64 weight_element_count, u64 cosine_element_count, u64 sine_element_count, "
                       "u64 output_element_count, u32 tokens, u32 heads, u32 head_width, u32 reserved0, "
                       "f32 epsilon, u64 input_generation, u64 weight_generation, u64 table_generation, "
                       "u64 exact_source_hash")


class PrometheusGemma4E2BM1HeadRmsNormRopeResult(Structure):
    _fields_ = _fields("u32 struct_size, u32 stage, i32 detail_code, u32 output_written, u32 dispatch_count, "
                       "u32 resident_source_bound, u32 normalized_readback_count, u64 source_byte_offset, "
                       "u64 source_byte_range, u64 destination_byte_offset, u64 destination_byte_range, "
                       "u64 input_hash, u64 weight_hash, u64 output_hash, u64 buffer_allocation_count, "
                       "u64 buffer_reuse_count, u64 descriptor_update_count, u64 pipeline_create_count, "
                       "u64 command_buffer_reuse_count, u64 observed_weight_generation, "
                       "u64 requested_weight_generation")


class PrometheusGemma4E2BM1AttentionScoresRequest(Structure):
    """reactor_api.h:1926-1959"""
    _fields_ = _fields("u32 struct_size, p query_input, p key_input, p query_weight, p key_weight, p cosine, "
                       "p sine, p scores, u64 query_input_element_count, u64 key_input_element_count, "
                       "u64 query_weight_element_count, u64 key_weight_element_count, u64 cosine_element_count, "
                       "u64 sine_element_count, u64 score_element_count, u32 tokens, u32 query_heads, "
                       "u32 key_heads, u32 head_width, f32 epsilon, f32 scale, u32 preparation_order, "
                       "u64 query_input_generation, u64 key_input_generation, u64 query_weight_generation, "
                       "u64 key_weight_generation, u64 table_generation, u64 query_exact_source_hash, "
                       "u64 key_exact_source_hash")


class PrometheusGemma4E2BM1AttentionScoresResult(Structure):
    _fields_ = _fields("u32 struct_size, u32 stage, i32 detail_code, u32 score_written, "
                       "u32 positional_dispatch_count, u32 score_dispatch_count, u32 score_readback_count, "
                       "u32 host_detour_count, u32 query_slot_id, u32 query_slot_generation, u32 key_slot_id, "
                       "u32 key_slot_generation, u32 score_slot_id, u32 score_slot_generation, "
                       "u64 query_byte_range, u64 key_byte_range, u64 score_byte_range, u64 score_hash, "
                       "u64 buffer_allocation_count, u64 buffer_reuse_count, u64 descriptor_update_count, "
                       "u64 pipeline_create_count, u64 observed_weight_generation, u64 requested_weight_generation")


# ---- batched complex-fp32 FFT (reactor_api.h:329-380, 1251-1305) ----------
PROM_FFT_FLAG_FORWARD, PROM_FFT_FLAG_INVERSE, PROM_FFT_FLAG_INVERSE_NORMALIZE = 1, 2, 4
PROM_FFT_FLAG_BENCHMARK_ALLOW_NON_PRODUCTION_PATH = 8
PROM_FFT_PATH_NONE, PROM_FFT_PATH_UNAVAILABLE, PROM_FFT_PATH_VULKAN_RADIX2_RESERVED = 0, 1, 3
PROM_FFT_BENCHMARK_VARIANT_RADIX2 = 2
PROM_FFT_DETAIL = {
    "UNAVAILABLE": -6701, "INVALID_REQUEST": -6702, "NULL_INPUT": -6703, "NULL_OUTPUT": -6704,
    "ZERO_ELEMENT_COUNT": -6705, "NON_POWER_OF_TWO": -6706, "INVALID_DIRECTION_FLAGS": -6707,
    "INVALID_STRIDE": -6708, "SIZE_OVERFLOW": -6709, "ZERO_BATCH_COUNT": -6710,
    "INVERSE_NORMALIZE_REQUIRES_INVERSE": -6711, "VULKAN_UNAVAILABLE": -6712, "UNSUPPORTED_SIZE": -6713,
    "ALLOCATION_FAILED": -6714, "UPLOAD_FAILED": -6715, "DISPATCH_FAILED": -6716, "READBACK_FAILED": -6717,
    "PLAN_DISPATCH_DISAGREEMENT": -6719,
}


class PrometheusComplex32(Structure):
    _fields_ = _fields("f32 real, f32 imag")


class PrometheusFftRequest(Structure):
    _fields_ = _fields("u32 struct_size, p input, p output, u32 element_count, u32 batch_count, "
                       "u32 stride_elements, u32 flags")


class PrometheusFftDiagnostics(Structure):
    _fields_ = _fields(
        "u32 struct_size, u32 api_declared, u32 capability_reported, u32 production_enabled, u32 benchmark_enabled, "
        "u32 last_element_count, u32 last_batch_count, u32 last_stride_elements, u32 last_effective_stride_elements, "
        "u32 last_flags, u32 last_direction, u32 last_validation_status, i32 last_failure_detail, "
        "u32 requested_path_id, u32 executed_path_id, u32 requested_radix, u32 executed_radix, u32 fallback_reason, "
        "u32 plan_pass_count, u32 ping_pong_swap_count, u32 final_output_role, u64 ping_arena_reuse_count, "
        "u64 ping_arena_grow_count, u64 pong_arena_reuse_count, u64 pong_arena_grow_count, "
        "u64 twiddle_arena_reuse_count, u64 twiddle_arena_grow_count, u32 selector_cache_valid, u32 plan_valid, "
        "u32 plan_element_count, u32 plan_log2_element_count, u32 plan_first_span, u32 plan_last_span, "
        "u32 plan_radix_mask, u32 plan_bit_reversal_required, u32 plan_first_source_role, "
        "u32 plan_first_destination_role, u32 plan_direction, u32 plan_twiddle_mode, u64 selector_cache_reuse_count, "
        "u64 selector_cache_recompute_count, u64 selector_cache_invalidation_count, "
        "u64 selector_cache_last_dependency_mask")


# ---- resident model blocks and the compiled session (reactor_api.h:666-1249)
PROM_MODEL_BLOCK_MAX_WEIGHTS = 13
PROM_MODEL_BLOCK_MAX_STEPS = 7
PROM_ZIMAGE_TURBO_LOCK_ID = 0x71EF202B4E34B562
PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES = 47186176
# the lock's static-audit arenas (resolved_audit_schedule.h:5-11, 67-71)
PROM_ZIMAGE_TURBO_AUDIT_LOCK_ID = PROM_ZIMAGE_TURBO_LOCK_ID
PROM_ZIMAGE_TURBO_AUDIT_REQUIRED_BYTES = 189696
PROM_ZIMAGE_TURBO_AUDIT_TRANSIENT_ATTENTION_OFFSET = 189440
PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_ARENA_BYTES = 1048576
PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_REQUIRED_BYTES = 4352
PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_TRANSIENT_ATTENTION_OFFSET = 4096
PROM_MODEL_BLOCK_M1C_TRANSIENT_AUDIT_FLOATS = 64
# main attention routes and fallback reasons (reactor_api.h:37-53)
PROM_MAIN_ATTENTION_ROUTE_AUTO, PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL, PROM_MAIN_ATTENTION_ROUTE_SUBGROUP_OWNED32 = 1, 2, 3
PROM_MAIN_ATTENTION_FALLBACK_NONE, PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_SIZE = 0, 3
PROM_NOISE_REFINER_FAMILY = 1
PROM_CONTEXT_REFINER_FAMILY = 2
PROM_MAIN_TRANSFORMER_FAMILY = 3
PROM_MODEL_BLOCK_SHADER_RESIDENT = 23
PROM_MODEL_BLOCK_SHADER_NOISE = 24
NOISE_REFINER_AGGREGATES = (0xA1BA526898A2A752, 0x80C0CD75F44CC434)
PROM_MODEL_BLOCK_DETAIL = {
    "INVALID_REQUEST": -6901, "NOT_FOUND": -6902, "ALREADY_CREATED": -6903, "WEIGHT_MISMATCH": -6904,
    "RESOURCE_CREATE_FAILED": -6905, "PIPELINE_CREATE_FAILED": -6906, "UPLOAD_FAILED": -6907,
    "COMMAND_RECORD_FAILED": -6908, "QUEUE_SUBMIT_FAILED": -6909, "COMPLETION_UNCERTAIN": -6910,
    "AUDIT_FAILED": -6911, "STALE_OUTPUT": -6912, "PARAMETER_SET_MISMATCH": -6920, "REBIND_FAILED": -6921,
    "SESSION_INVALID_REQUEST": -6923, "SESSION_STALE_STREAM": -6924, "SESSION_STREAM_MISMATCH": -6925,
    "SESSION_COMPLETION_UNCERTAIN": -6926, "INGRESS_DISPATCH_FAILED": -6914, "INGRESS_INPUT_SIZE_MISMATCH": -6916,
    "INGRESS_TIMESTEP_SIZE_MISMATCH": -6917, "M1C_SOFTMAX_INVALID": -6918, "MAIN_ATTENTION_ROUTE_REJECTED": -6927,
}
PROM_REDUCTION_TESTCFG_FAIL_COMMAND_RECORD = 1 << 0
PROM_REDUCTION_TESTCFG_FAIL_QUEUE_SUBMIT = 1 << 1
PROM_REDUCTION_TESTCFG_FAIL_COMPLETION_OBSERVATION = 1 << 2


class PrometheusModelBlockWeightDeclaration(Structure):
    _fields_ = _fields("u64 content_identity, u64 layout_identity, u64 byte_count")


class PrometheusModelBlockCreateRequest(Structure):
    """reactor_api.h:806-826"""
    _fields_ = _fields("u32 struct_size, u32 assembly_family, u32 parameter_set, "
                       "u64 parameter_set_aggregate_identity, u64 model_contract_identity, u64 weight_identity, "
                       "u64 shader_portfolio_identity, u64 precision_policy_identity, u64 capability_route_identity, "
                       "u64 memory_ceiling_bytes, u64 external_input_bytes, u64 external_output_bytes, "
                       "u64 audit_bytes, u32 shader_id, u32 weight_count") + [
        ("weights", PrometheusModelBlockWeightDeclaration * PROM_MODEL_BLOCK_MAX_WEIGHTS),
        ("step_count", c_uint32), ("steps", c_uint32 * PROM_MODEL_BLOCK_MAX_STEPS)]


class PrometheusModelBlockWeightUpload(Structure):
    _fields_ = _fields("u32 binding_index, p bytes, u64 byte_count, u64 content_identity, u64 layout_identity")


class PrometheusNoiseRefinerRebindRequest(Structure):
    _fields_ = _fields("u32 struct_size, u32 model_local_block_id, u64 lock_identity, u32 upload_count, p uploads")


# ContextRefiner create/rebind and MainTransformer create/rebind share this layout.
PrometheusContextRefinerCreateRequest = PrometheusNoiseRefinerRebindRequest


class PrometheusMainTransformerExecuteRequest(Structure):
    _fields_ = _fields("u32 struct_size, u64 session_identity, u64 lock_identity, u32 model_local_block_id, "
                       "u32 audit_enabled, u32 resident_chain_mode, u32 reserved0, u64 required_image_generation, "
                       "u64 required_context_generation, u64 required_joint_generation, p timestep_bf16, "
                       "u64 timestep_bytes, u64 timestep_identity, u64 output_identity")


class PrometheusModelBlockExecuteRequest(Structure):
    _fields_ = _fields("u32 struct_size, p input, p output, u64 element_count, u64 input_identity, "
                       "u32 audit_enabled, p audit_output, u64 audit_element_capacity")


class PrometheusNoiseRefiner0ExecuteRequest(Structure):
    _fields_ = _fields("u32 struct_size, p model_input_bf16, p timestep_bf16, u64 model_input_bytes, "
                       "u64 timestep_bytes, u64 input_identity, u64 timestep_identity, u64 output_identity, "
                       "u32 audit_enabled")


class PrometheusNoiseRefinerResidentExecuteRequest(Structure):
    _fields_ = _fields("u32 struct_size, u64 input_generation, u64 output_identity, u32 audit_enabled, "
                       "u32 audit_family, u32 audit_stage, p audit_output, u64 audit_element_capacity")


class PrometheusContextRefiner0ExecuteRequest(Structure):
    _fields_ = _fields("u32 struct_size, p context_input, u64 context_input_bytes, u64 input_identity, "
                       "u64 output_identity, u32 audit_enabled")


class PrometheusContextRefinerResidentExecuteRequest(Structure):
    _fields_ = _fields("u32 struct_size, u64 input_generation, u64 output_identity, u32 audit_enabled")


class PrometheusNoiseRefinerFinalAuditRequest(Structure):
    _fields_ = _fields("u32 struct_size, u64 required_output_generation, u64 output_identity, p output, "
                       "u64 output_element_capacity")


class PrometheusModelBlockM1BExecuteRequest(Structure):
    """reactor_api.h:961-973"""
    _fields_ = _fields("u32 struct_size, p model_input_bf16, p timestep_bf16, u64 model_input_bytes, "
                       "u64 timestep_bytes, u64 input_identity, u64 timestep_identity, u32 audit_enabled, "
                       "u32 audit_stage, p audit_output, u64 audit_element_capacity")


class PrometheusModelBlockM1CExecuteRequest(Structure):
    """reactor_api.h:978-987"""
    _fields_ = _fields("u32 struct_size, u64 m1b_prefix_replay_identity, u64 output_identity, p output, "
                       "u64 output_element_capacity, u32 audit_stage, p transient_audit, "
                       "u64 transient_audit_element_capacity")


class PrometheusModelBlockM1DExecuteRequest(Structure):
    """reactor_api.h:1000-1007"""
    _fields_ = _fields("u32 struct_size, u64 m1c_prefix_replay_identity, u64 output_identity, p output, "
                       "u64 output_element_capacity, u32 audit_stage")


class PrometheusNoiseRefinerStaticAuditRequest(Structure):
    """reactor_api.h:1070-1081 (also the ContextRefiner request)"""
    _fields_ = _fields("u32 struct_size, u64 lock_identity, u64 input_generation, u64 output_identity, "
                       "p audit_arena, u64 audit_arena_capacity_bytes")


class PrometheusMainTransformerStaticAuditRequest(Structure):
    """reactor_api.h:1082-1093"""
    _fields_ = _fields("u32 struct_size, u64 session_identity, u64 lock_identity, u32 model_local_block_id, "
                       "u64 required_image_generation, u64 required_context_generation, "
                       "u64 required_joint_generation, u64 output_identity, p audit_arena, "
                       "u64 audit_arena_capacity_bytes")


class PrometheusModelBlockEvidence(Structure):
    """reactor_api.h:1103-1186"""
    _fields_ = _fields(
        "u32 struct_size, i32 detail_code, u32 created, u32 weights_uploaded, u32 quarantined, u32 output_valid, "
        "u32 audit_valid, u32 fixed_step_count, u32 weight_count, u64 persistent_bytes, u64 reusable_bytes, "
        "u64 audit_bytes, u64 external_bytes, u64 total_committed_bytes, u64 peak_plan_bytes, "
        "u64 cold_buffer_allocation_count, u64 warm_buffer_allocation_count, u64 pipeline_create_count, "
        "u64 descriptor_set_count, u64 weight_upload_count, u64 execution_count, u64 last_execution_ns, "
        "u64 execution_plan_identity, u64 replay_identity, u32 assembly_family, u32 parameter_set, "
        "u32 binding_state, u32 active_weight_window, u64 parameter_set_aggregate_identity, "
        "u64 binding_generation, u64 output_generation, u64 descriptor_generation") + [
        ("m1b_boundary_gpu_ns", c_uint64 * 6)] + _fields(
        "u64 gpu_total_begin_tick, u64 gpu_total_end_tick, u64 gpu_total_ns, u64 gpu_compute_begin_tick, "
        "u64 gpu_compute_end_tick, u64 gpu_compute_ns, u64 gpu_ingress_transfer_ns, u64 gpu_joint_copy_ns, "
        "u64 gpu_readback_ns") + [
        ("main_stage_gpu_begin_tick", c_uint64 * 13), ("main_stage_gpu_end_tick", c_uint64 * 13),
        ("main_stage_gpu_ns", c_uint64 * 13)] + _fields(
        "u64 last_active_target_validation_ns, u64 last_command_reset_ns, u64 last_command_begin_ns, "
        "u64 last_command_record_ns, u64 last_command_end_ns, u64 last_queue_submit_ns, u64 last_fence_wait_ns, "
        "u64 last_descriptor_update_ns, u64 last_staging_memcpy_ns, u64 last_output_readback_ns, "
        "u64 vk_create_buffer_count, u64 vk_destroy_buffer_count, u64 vk_allocate_memory_count, "
        "u64 vk_free_memory_count, u64 vk_create_shader_module_count, u64 vk_destroy_shader_module_count, "
        "u64 vk_create_compute_pipelines_count, u64 vk_allocate_descriptor_sets_count, "
        "u64 vk_update_descriptor_sets_count, u64 vk_create_command_pool_count, "
        "u64 vk_allocate_command_buffers_count, u64 vk_reset_command_buffer_count, u64 vk_queue_submit_count, "
        "u64 vk_fence_wait_count, u64 vk_timeline_wait_count, u64 vk_map_memory_count, u64 vk_unmap_memory_count, "
        "u64 vk_flush_count, u64 vk_invalidate_count, u64 m6a_activation_pack_gpu_ns, "
        "u64 m6a_cooperative_execute_gpu_ns, u64 m6a_w3_segment_repack_gpu_ns")


class PrometheusCompiledModelRetargetRequest(Structure):
    """reactor_api.h:1237-1249 (also the prefetch request)"""
    _fields_ = _fields("u32 struct_size, u64 session_identity, u64 lock_identity, u32 model_local_block_id, "
                       "u32 upload_count, p uploads")


class PrometheusCompiledModelSessionCreateRequest(Structure):
    _fields_ = _fields("u32 struct_size, u64 lock_identity, u32 execution_profile, u32 main_attention_route_policy")


class PrometheusCompiledModelSessionCaptureRequest(Structure):
    _fields_ = _fields("u32 struct_size, u64 source_output_generation")


class PrometheusCompiledModelSessionComposeRequest(Structure):
    _fields_ = _fields("u32 struct_size, u64 required_image_generation, u64 required_context_generation")


class PrometheusCompiledModelSessionEvidence(Structure):
    """reactor_api.h:1208-1236"""
    _fields_ = _fields(
        "u32 struct_size, i32 detail_code, u32 created, u32 quarantined, u64 session_identity, u64 lock_identity, "
        "u64 active_block_id, u64 binding_generation, u64 replay_identity, u64 prepared_image_generation, "
        "u64 prepared_context_generation, u64 joint_generation, u64 joint_image_generation, "
        "u64 joint_context_generation, u64 prepared_image_bytes, u64 prepared_context_bytes, u64 joint_bytes, "
        "u64 cold_buffer_allocation_count, u64 warm_buffer_allocation_count, u64 composition_count, "
        "u32 requested_execution_profile, u32 selected_execution_profile, u32 profile_fallback_reason, "
        "u32 requested_main_attention_route, u32 selected_main_attention_route, "
        "u32 main_attention_fallback_reason, u32 main_attention_shader_id")


# ---- errors and status (status.go, bridge.go) ------------------------------
class ReactorIssue(RuntimeError):
    """Structured reactor failure (reference ``ReactorIssue``, bridge.go:33-66)."""

    def __init__(self, code: str, message: str):
        super().__init__(f"{code}: {message}")
        self.code = code
        self.message = message


class StrictExecutionError(ReactorIssue):
    """strict.go:11-32's error.  Its text is the message alone
    ("PROMETHEUS requires GPU matrix execution: ..."), as the Go code's
    fmt.Errorf words it, so an interpreter can print it unchanged."""

    def __init__(self, message: str):
        RuntimeError.__init__(self, message)
        self.code = "strict"
        self.message = message


def stage_name(stage: int) -> str:
    """bridge.go:535-550 (stageFromNativeCode)."""
    return {1: "init", 2: "transfer_in", 3: "submit", 4: "transfer_out", 5: "cleanup"}.get(stage, "unknown")


@dataclass
class RunStatus:
    """status.go:30-59."""

    kind: str
    error_stage: str = ""
    error_code: int = 0
    fallback_reason: str = ""

    def __str__(self) -> str:
        if self.kind == "ok":
            return "ok"
        if self.kind == "fallback":
            return f"fallback({self.fallback_reason})"
        return f"error({self.error_stage},{self.error_code})"


@dataclass
class CallStatus:
    stage: int
    detail: int


# ---- library loading --------------------------------------------------------
_SIGNATURES = {
    "prometheus_reactor_abi_version": (c_uint32, []),
    "prometheus_reactor_runtime_create": (c_int, [c_void_p, POINTER(c_void_p)]),
    "prometheus_reactor_runtime_destroy": (c_int, [c_void_p]),
    "prometheus_reactor_runtime_probe": (c_int, [c_void_p, POINTER(PrometheusCaps)]),
    "prometheus_runtime_create": (c_int, [c_void_p, POINTER(c_void_p)]),
    "prometheus_runtime_destroy": (c_int, [c_void_p]),
    "prometheus_runtime_probe": (c_int, [c_void_p, POINTER(PrometheusCaps)]),
    "prometheus_reactor_sgemm_plan": (c_int, [c_uint32, c_uint32, c_uint32, POINTER(PrometheusSgemmPlanInfo)]),
    "prometheus_reactor_runtime_vulkan_device_diagnostics": (c_int, [c_void_p, POINTER(PrometheusVulkanDeviceDiagnostics)]),
    "prometheus_reactor_runtime_hip_device_diagnostics": (c_int, [c_void_p, POINTER(PrometheusHipDeviceDiagnostics)]),
    "prometheus_reactor_runtime_sgemm": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_sgemm_device": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_sgemm_device_variant": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_sgemm_device_noalloc": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_attention_bf16_device": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32,
                POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_gemm_bf16": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_gemm_bf16_device": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_reduction_plan": (
        c_int, [POINTER(PrometheusReductionRequest), POINTER(PrometheusReductionPlan)]),
    "prometheus_reactor_runtime_reduction": (
        c_int, [c_void_p, POINTER(PrometheusReductionRequest), POINTER(PrometheusReductionExecutionResult)]),
    "prometheus_reactor_runtime_reduction_v2": (
        c_int, [c_void_p, POINTER(PrometheusReductionRequest), POINTER(PrometheusReductionExecutionResult)]),
    "prometheus_reactor_runtime_reduction_device": (
        c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_row_wise_softmax": (
        c_int, [c_void_p, POINTER(PrometheusRowWiseSoftmaxRequest), POINTER(PrometheusRowWiseSoftmaxResult)]),
    "prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm": (
        c_int, [c_void_p, POINTER(PrometheusGemma4E2BM1InputRmsNormRequest),
                POINTER(PrometheusGemma4E2BM1InputRmsNormResult)]),
    "prometheus_reactor_runtime_rmsnorm": (
        c_int, [c_void_p, POINTER(PrometheusRmsNormRequest), POINTER(PrometheusRmsNormResult)]),
    "prometheus_reactor_runtime_rmsnorm_device": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_float,
                POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_decoder_layer_f32": (
        c_int, [c_void_p, POINTER(PrometheusDecoderLayerF32Request), POINTER(PrometheusBlockResult)]),
    "prometheus_reactor_runtime_decoder_layer_f32_device": (
        c_int, [c_void_p, POINTER(PrometheusDecoderLayerF32Request), POINTER(PrometheusBlockResult)]),
    "prometheus_reactor_runtime_dit_block_bf16": (
        c_int, [c_void_p, POINTER(PrometheusDitBlockBf16Request), POINTER(PrometheusBlockResult)]),
    "prometheus_reactor_runtime_dit_block_bf16_device": (
        c_int, [c_void_p, POINTER(PrometheusDitBlockBf16Request), POINTER(PrometheusBlockResult)]),
    "prometheus_reactor_runtime_device_alloc": (c_int, [c_void_p, c_uint64, POINTER(c_void_p)]),
    "prometheus_reactor_runtime_device_free": (c_int, [c_void_p, c_void_p]),
    "prometheus_reactor_runtime_device_upload": (c_int, [c_void_p, c_void_p, c_void_p, c_uint64]),
    "prometheus_reactor_runtime_device_download": (c_int, [c_void_p, c_void_p, c_void_p, c_uint64]),
    "prometheus_reactor_runtime_synchronize": (c_int, [c_void_p]),
    "prometheus_reactor_runtime_event_record": (c_int, [c_void_p, c_uint32]),
    "prometheus_reactor_runtime_event_elapsed_ms": (c_int, [c_void_p, c_uint32, c_uint32, POINTER(c_float)]),
    "prometheus_reactor_runtime_sgemm_submit_async": (
        c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, POINTER(c_int), POINTER(c_uint32),
                POINTER(c_int)]),
    "prometheus_reactor_runtime_sgemm_query_async": (c_int, [c_void_p, c_int, POINTER(PrometheusAsyncStatus)]),
    "prometheus_reactor_runtime_sgemm_async_diagnostics": (
        c_int, [c_void_p, POINTER(PrometheusSgemmAsyncDiagnostics)]),
    "prometheus_reactor_runtime_sgemm_consume_async": (
        c_int, [c_void_p, c_int, c_void_p, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_sgemm_abandon_async": (c_int, [c_void_p, c_int]),
    "prometheus_reactor_runtime_sgemm_batch": (
        c_int, [c_void_p, POINTER(PrometheusSgemmBatchEntry), c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_sgemm_batch_m31_test": (
        c_int, [c_void_p, POINTER(PrometheusSgemmBatchEntry), c_uint32, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_sgemm_batch_diagnostics": (
        c_int, [c_void_p, POINTER(PrometheusSgemmBatchDiagnostics)]),
    "prometheus_reactor_runtime_fft64": (
        c_int, [c_void_p, c_void_p, c_void_p, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_fft64_device": (
        c_int, [c_void_p, c_void_p, c_void_p, c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_reduction_diagnostics": (
        c_int, [c_void_p, POINTER(PrometheusReductionDiagnostics)]),
    "prometheus_reactor_runtime_reduction_benchmark": (
        c_int, [c_void_p, POINTER(PrometheusReductionBenchmarkRequest), POINTER(PrometheusReductionBenchmarkResult)]),
    "prometheus_reactor_runtime_fft": (
        c_int, [c_void_p, POINTER(PrometheusFftRequest), POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_fft_benchmark_variant": (
        c_int, [c_void_p, POINTER(PrometheusFftRequest), c_uint32, POINTER(c_uint32), POINTER(c_int)]),
    "prometheus_reactor_runtime_fft_diagnostics": (c_int, [c_void_p, POINTER(PrometheusFftDiagnostics)]),
    "prometheus_reactor_runtime_fft_diagnostics_sized": (
        c_int, [c_void_p, POINTER(PrometheusFftDiagnostics), c_uint32]),
    "prometheus_reactor_runtime_gemma4e2b_m1_projection_activation_rmsnorm": (
        c_int, [c_void_p, POINTER(PrometheusGemma4E2BM1InputRmsNormRequest),
                POINTER(PrometheusGemma4E2BM1InputRmsNormResult)]),
    "prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm": (
        c_int, [c_void_p, POINTER(PrometheusGemma4E2BM1InputRmsNormRequest),
                POINTER(PrometheusGemma4E2BM1InputRmsNormResult)]),
    "prometheus_reactor_runtime_gemma4e2b_m1_rope": (
        c_int, [c_void_p, POINTER(PrometheusGemma4E2BM1RopeRequest), POINTER(PrometheusGemma4E2BM1RopeResult)]),
    "prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm_rope": (
        c_int, [c_void_p, POINTER(PrometheusGemma4E2BM1HeadRmsNormRopeRequest),
                POINTER(PrometheusGemma4E2BM1HeadRmsNormRopeResult)]),
    "prometheus_reactor_runtime_gemma4e2b_m1_attention_scores": (
        c_int, [c_void_p, POINTER(PrometheusGemma4E2BM1AttentionScoresRequest),
                POINTER(PrometheusGemma4E2BM1AttentionScoresResult)]),
    # resident model blocks and the compiled session (reactor_api.h:2713-2808)
    "prometheus_reactor_runtime_model_block_create": (
        c_int, [c_void_p, POINTER(PrometheusModelBlockCreateRequest), POINTER(c_uint64),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_model_block_upload_weights": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusModelBlockWeightUpload), c_uint32,
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_model_block_execute": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusModelBlockExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_model_block_execute_m1b": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusModelBlockM1BExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_model_block_execute_m1c": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusModelBlockM1CExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_model_block_execute_m1d": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusModelBlockM1DExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_noise_refiner_execute_static_audit": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusNoiseRefinerStaticAuditRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_context_refiner_execute_static_audit": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusNoiseRefinerStaticAuditRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_main_transformer_execute_static_audit": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusMainTransformerStaticAuditRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_compiled_model_session_set_main_attention_route": (
        c_int, [c_void_p, c_uint64, c_uint32, POINTER(PrometheusCompiledModelSessionEvidence)]),
    "prometheus_reactor_runtime_noise_refiner0_execute": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusNoiseRefiner0ExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_noise_refiner1_execute": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusNoiseRefiner0ExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_noise_refiner_rebind": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusNoiseRefinerRebindRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_noise_refiner_execute_resident": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusNoiseRefinerResidentExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_noise_refiner_audit_final": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusNoiseRefinerFinalAuditRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_context_refiner_create": (
        c_int, [c_void_p, POINTER(PrometheusContextRefinerCreateRequest), POINTER(c_uint64),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_context_refiner_rebind": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusContextRefinerCreateRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_context_refiner0_execute": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusContextRefiner0ExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_context_refiner_execute_resident": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusContextRefinerResidentExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_context_refiner_audit_final": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusNoiseRefinerFinalAuditRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_main_transformer_create": (
        c_int, [c_void_p, POINTER(PrometheusContextRefinerCreateRequest), POINTER(c_uint64),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_main_transformer_rebind": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusContextRefinerCreateRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_main_transformer_execute": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusMainTransformerExecuteRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_main_transformer_audit_final": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusNoiseRefinerFinalAuditRequest),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_model_block_get_evidence": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_model_block_destroy": (c_int, [c_void_p, c_uint64]),
    "prometheus_reactor_runtime_compiled_model_session_create": (
        c_int, [c_void_p, POINTER(PrometheusCompiledModelSessionCreateRequest), POINTER(c_uint64),
                POINTER(PrometheusCompiledModelSessionEvidence)]),
    "prometheus_reactor_runtime_compiled_model_session_capture_completed": (
        c_int, [c_void_p, c_uint64, c_uint64, POINTER(PrometheusCompiledModelSessionCaptureRequest),
                POINTER(PrometheusCompiledModelSessionEvidence)]),
    "prometheus_reactor_runtime_compiled_model_session_compose_joint": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusCompiledModelSessionComposeRequest),
                POINTER(PrometheusCompiledModelSessionEvidence)]),
    "prometheus_reactor_runtime_compiled_model_session_get_evidence": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusCompiledModelSessionEvidence)]),
    "prometheus_reactor_runtime_compiled_model_session_destroy": (c_int, [c_void_p, c_uint64]),
    "prometheus_reactor_runtime_compiled_model_owner_create": (
        c_int, [c_void_p, POINTER(PrometheusNoiseRefinerRebindRequest), POINTER(c_uint64),
                POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_compiled_model_retarget": (
        c_int, [c_void_p, POINTER(PrometheusCompiledModelRetargetRequest), POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_compiled_model_prefetch": (
        c_int, [c_void_p, POINTER(PrometheusCompiledModelRetargetRequest), POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_compiled_model_activate_prefetch": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusModelBlockEvidence)]),
    "prometheus_reactor_runtime_compiled_model_evaluation_reset": (
        c_int, [c_void_p, c_uint64, POINTER(PrometheusCompiledModelSessionEvidence)]),
}

MANDATORY_SYMBOLS = (
    "prometheus_reactor_abi_version",
    "prometheus_reactor_runtime_create",
    "prometheus_reactor_runtime_destroy",
    "prometheus_reactor_runtime_probe",
    "prometheus_reactor_runtime_sgemm",
)


def discover_reactor_candidates() -> list:
    """bridge.go:552-582: $OCT_PROMETHEUS_REACTOR wins; else the package's build."""
    explicit = os.environ.get(REACTOR_ENV_VAR, "")
    if explicit:
        return [explicit]
    return [str(PACKAGE_DIR / LIBRARY_BASENAME)]


def load_library(path: Optional[str] = None) -> ctypes.CDLL:
    """dlopen the reactor and bind every known symbol (bridge.go:276-340)."""
    candidates = [path] if path else discover_reactor_candidates()
    last_err = None
    for cand in candidates:
        if not Path(cand).exists():
            continue
        try:
            lib = ctypes.CDLL(cand, mode=os.RTLD_NOW | os.RTLD_LOCAL)
        except OSError as exc:
            last_err = ReactorIssue("reactor_load_failed", f"{cand}: {exc}")
            continue
        for name in MANDATORY_SYMBOLS:
            if not hasattr(lib, name):
                raise ReactorIssue("symbol_missing", f"{name} missing from {cand}")
        for name, (restype, argtypes) in _SIGNATURES.items():
            if hasattr(lib, name):
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
        version = lib.prometheus_reactor_abi_version()
        if version != REACTOR_EXPECTED_ABI_VERSION:
            raise ReactorIssue("abi_mismatch", f"expected ABI {REACTOR_EXPECTED_ABI_VERSION}, got {version}")
        lib._oct_path = cand  # type: ignore[attr-defined]
        return lib
    # bridge.go:262-267: a candidate that failed to load wins over "not found".
    if last_err is not None:
        raise last_err
    raise ReactorIssue("reactor_not_found", "prometheus reactor not found")


_LOADED: dict = {}


def shared_library() -> ctypes.CDLL:
    """The reactor that discovery names now.  The reference resolves the path
    on every runtime open (bridge.go:552-582), so a changed
    $OCT_PROMETHEUS_REACTOR takes effect at the next open; each path is
    loaded and bound once per process, as a repeated dlopen of one path
    returns the same handle."""
    for cand in discover_reactor_candidates():
        lib = _LOADED.get(cand)
        if lib is not None:
            return lib
    lib = load_library()
    _LOADED[lib._oct_path] = lib
    return lib


def _ptr(arr: Optional[np.ndarray]) -> Optional[int]:
    return None if arr is None else arr.ctypes.data


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


class NativeRuntime:
    """A reactor runtime handle (reference ``nativeRuntime``, bridge.go:238-516).

    Unlike the reference's strict path, which opens a private runtime per call,
    a process-wide device context is shared by every handle; creating one is cheap.
    """

    def __init__(self, lib: Optional[ctypes.CDLL] = None, test_flags: Optional[int] = None,
                 reduction_test_flags: int = 0, batch_ring_depth: int = 0):
        self.lib = lib or shared_library()
        if test_flags is None:
            env = os.environ.get(REACTOR_TEST_FLAGS_ENV_VAR, "")
            test_flags = int(env, 0) if env else 0
        cfg = PrometheusReactorConfig()
        cfg.struct_size = ctypes.sizeof(cfg)
        cfg.test_flags = test_flags
        cfg.reduction_test_flags = reduction_test_flags
        cfg.batch_ring_depth = batch_ring_depth
        handle = c_void_p()
        rc = self.lib.prometheus_reactor_runtime_create(byref(cfg), byref(handle))
        if rc != PROM_OK or not handle.value:
            raise ReactorIssue("runtime_create_failed", f"runtime_create returned {rc}")
        self.handle = handle
        caps = PrometheusCaps()
        rc = self.lib.prometheus_reactor_runtime_probe(self.handle, byref(caps))
        if rc != PROM_OK:
            self.close()
            raise ReactorIssue("runtime_probe_unavailable", f"runtime_probe returned {rc}")
        self.caps = caps

    # -- lifecycle --------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.lib.prometheus_reactor_runtime_destroy(self.handle)
            self.handle = c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def available(self) -> bool:
        return bool(self.caps.available)

    def require_hardware_gpu(self) -> None:
        """internal/prometheus/fft.go:50-55: strict execution requires an
        available hardware device (backend 2), with the reference's error text."""
        if not self.caps.available or self.caps.backend_type != PROM_BACKEND_HARDWARE_GPU:
            raise ReactorIssue("unavailable", f"GPU execution requires hardware Vulkan; backend is {self.environment()}")

    def environment(self) -> str:
        """bridge.go:518-533, with this library's name for the hardware backend."""
        if self.caps.backend_type == PROM_BACKEND_HARDWARE_GPU:
            return "hardware_gpu_hip"
        if self.caps.backend_type == 3:
            return "software_vulkan_llvmpipe_or_cpu"
        return "unknown"

    def device_diagnostics(self) -> PrometheusHipDeviceDiagnostics:
        d = PrometheusHipDeviceDiagnostics()
        d.struct_size = ctypes.sizeof(d)
        rc = self.lib.prometheus_reactor_runtime_hip_device_diagnostics(self.handle, byref(d))
        if rc != PROM_OK:
            raise ReactorIssue("diagnostics_failed", f"hip_device_diagnostics returned {rc}")
        return d

    # -- host-pointer operations -------------------------------------------
    def sgemm_with_status(self, m: int, n: int, k: int, a, b) -> Tuple[Optional[np.ndarray], CallStatus, int]:
        a = _f32(a).reshape(-1)
        b = _f32(b).reshape(-1)
        if a.size != m * k or b.size != k * n:
            return None, CallStatus(STAGE_INIT, -2), PROM_ERROR
        out = np.empty(m * n, dtype=np.float32)
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_sgemm(self.handle, _ptr(a), _ptr(b), _ptr(out), m, n, k,
                                                       byref(stage), byref(detail))
        status = CallStatus(stage.value, detail.value)
        return (out if rc == PROM_OK else None), status, rc

    def sgemm(self, m: int, n: int, k: int, a, b) -> Tuple[np.ndarray, RunStatus]:
        """bridge.go:410-422 (nativeRuntime.SGEMM)."""
        out, st, rc = self.sgemm_with_status(m, n, k, a, b)
        if rc != PROM_OK:
            status = RunStatus("error", stage_name(st.stage), st.detail)
            raise ReactorIssue("runtime_sgemm_failed", f"native sgemm failed: {status}")
        return out, RunStatus("ok")

    def gemm_bf16(self, m: int, n: int, k: int, a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a_bits, dtype=np.uint16).reshape(-1)
        b = np.ascontiguousarray(b_bits, dtype=np.uint16).reshape(-1)
        if a.size != m * k or b.size != k * n:
            raise ValueError("invalid matrix lengths")
        out = np.empty(m * n, dtype=np.float32)
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_gemm_bf16(self.handle, _ptr(a), _ptr(b), _ptr(out), m, n, k,
                                                           byref(stage), byref(detail))
        if rc != PROM_OK:
            raise ReactorIssue("gemm_bf16_failed", f"error({stage_name(stage.value)},{detail.value})")
        return out

    def reduction(self, x, operation: int, flags: int = 0, lifted: bool = True, output=None):
        """Row reduction through ..._reduction_v2 (lifted limits) or the reference entry."""
        x = _f32(x)
        rows, width = x.shape
        req = PrometheusReductionRequest()
        req.struct_size = ctypes.sizeof(req)
        req.input = _ptr(x)
        out_count = rows * width if operation == OP_SOFTMAX else rows
        if output is None:
            output = np.empty((rows, width) if operation == OP_SOFTMAX else (rows,), dtype=np.float32)
        req.output = _ptr(output)
        req.row_count, req.elements_per_row = rows, width
        req.input_element_count, req.output_element_count = rows * width, out_count
        req.operation = operation
        req.finalization = FINALIZATION_STABLE_SOFTMAX if operation == OP_SOFTMAX else FINALIZATION_NONE
        req.flags = flags
        res = PrometheusReductionExecutionResult()
        fn = (self.lib.prometheus_reactor_runtime_reduction_v2 if lifted
              else self.lib.prometheus_reactor_runtime_reduction)
        rc = fn(self.handle, byref(req), byref(res))
        return rc, res, output

    def reduction_diagnostics(self):
        d = PrometheusReductionDiagnostics()
        rc = self.lib.prometheus_reactor_runtime_reduction_diagnostics(self.handle, byref(d))
        return rc, d

    def reduction_benchmark(self, x, operation: int, warmup: int = 2, measured: int = 10, request_patch=None):
        """reactor_api.h:2678-2681 on the reference envelope; returns (rc, result, output)."""
        x = _f32(x)
        rows, width = x.shape
        output = np.empty((rows, width) if operation == OP_SOFTMAX else (rows,), dtype=np.float32)
        b = PrometheusReductionBenchmarkRequest()
        b.struct_size = ctypes.sizeof(b)
        r = b.reduction
        r.struct_size = ctypes.sizeof(r)
        r.input, r.output = _ptr(x), _ptr(output)
        r.row_count, r.elements_per_row = rows, width
        r.input_element_count, r.output_element_count = rows * width, output.size
        r.operation = operation
        r.finalization = FINALIZATION_STABLE_SOFTMAX if operation == OP_SOFTMAX else FINALIZATION_NONE
        b.warmup_iterations, b.measured_iterations = warmup, measured
        if request_patch:
            request_patch(b)
        res = PrometheusReductionBenchmarkResult()
        rc = self.lib.prometheus_reactor_runtime_reduction_benchmark(self.handle, byref(b), byref(res))
        return rc, res, output

    def rmsnorm(self, x, weight, epsilon: float, stride: Optional[int] = None):
        x = _f32(x)
        w = _f32(weight)
        tokens = x.shape[0]
        width = w.size
        stride = stride or x.shape[1]
        out = np.empty((tokens, width), dtype=np.float32)
        inv = np.empty(tokens, dtype=np.float32)
        req = PrometheusRmsNormRequest()
        req.struct_size = ctypes.sizeof(req)
        req.input, req.weight, req.output, req.inv_rms_output = _ptr(x), _ptr(w), _ptr(out), _ptr(inv)
        req.tokens, req.width, req.input_row_stride, req.epsilon = tokens, width, stride, epsilon
        res = PrometheusRmsNormResult()
        rc = self.lib.prometheus_reactor_runtime_rmsnorm(self.handle, byref(req), byref(res))
        return rc, res, out, inv

    # -- transformer blocks ----------------------------------------------------
    def decoder_layer_request(self, tokens, hidden, q_heads, head_dim, ffn, ptrs: dict, eps=1e-6,
                              rope_base=10000.0, position_offset=0, kv_heads=1) -> PrometheusDecoderLayerF32Request:
        req = PrometheusDecoderLayerF32Request()
        req.struct_size = ctypes.sizeof(req)
        req.tokens, req.hidden, req.q_heads, req.kv_heads = tokens, hidden, q_heads, kv_heads
        req.head_dim, req.ffn_hidden, req.position_offset = head_dim, ffn, position_offset
        req.rms_epsilon, req.rope_base = eps, rope_base
        for name, ptr in ptrs.items():
            setattr(req, name, ptr)
        return req

    def decoder_layer_f32(self, x, w, q_heads: int, head_dim: int, eps=1e-6, rope_base=10000.0,
                          position_offset=0) -> Tuple[int, PrometheusBlockResult, np.ndarray]:
        """Host-pointer Gemma-style layer; ``w`` has attn_norm, w_qkv, w_o, ffn_norm, w_gate_up, w_down."""
        x = _f32(x)
        tokens, hidden = x.shape
        arrs = {"input": x, "attn_norm_weight": _f32(w.attn_norm), "w_qkv": _f32(w.w_qkv), "w_o": _f32(w.w_o),
                "ffn_norm_weight": _f32(w.ffn_norm), "w_gate_up": _f32(w.w_gate_up), "w_down": _f32(w.w_down)}
        out = np.empty_like(x)
        arrs["output"] = out
        req = self.decoder_layer_request(tokens, hidden, q_heads, head_dim, arrs["w_down"].shape[0],
                                         {k: _ptr(v) for k, v in arrs.items()}, eps, rope_base, position_offset)
        res = PrometheusBlockResult()
        rc = self.lib.prometheus_reactor_runtime_decoder_layer_f32(self.handle, byref(req), byref(res))
        return rc, res, out

    def dit_block_request(self, tokens, hidden, heads, ffn, cond_dim, ptrs: dict, eps=1e-5, theta=256.0,
                          axes=(32, 48, 48), head_dim=128) -> PrometheusDitBlockBf16Request:
        req = PrometheusDitBlockBf16Request()
        req.struct_size = ctypes.sizeof(req)
        req.tokens, req.hidden, req.heads, req.head_dim = tokens, hidden, heads, head_dim
        req.ffn_hidden, req.cond_dim = ffn, cond_dim
        req.rope_axes[0], req.rope_axes[1], req.rope_axes[2] = axes
        req.rope_theta, req.rms_epsilon = theta, eps
        for name, ptr in ptrs.items():
            setattr(req, name, ptr)
        return req

    def dit_block_bf16(self, x, coords, condition, w, heads: int, eps=1e-5, theta=256.0,
                       axes=(32, 48, 48)) -> Tuple[int, PrometheusBlockResult, np.ndarray]:
        """Host-pointer DiT block; ``w`` carries bf16 bit patterns for the projections."""
        x = _f32(x)
        tokens, hidden = x.shape
        u16 = lambda a: np.ascontiguousarray(a, dtype=np.uint16)
        arrs = {"input": x, "coordinates": _f32(coords), "condition": _f32(condition), "w_adaln": u16(w.w_adaln),
                "b_adaln": _f32(w.b_adaln), "attn_norm1": _f32(w.attn_norm1), "attn_norm2": _f32(w.attn_norm2),
                "ffn_norm1": _f32(w.ffn_norm1), "ffn_norm2": _f32(w.ffn_norm2), "q_norm": _f32(w.q_norm),
                "k_norm": _f32(w.k_norm), "w_qkv": u16(w.w_qkv), "w_out": u16(w.w_out), "w_13": u16(w.w_13),
                "w_2": u16(w.w_2)}
        out = np.empty_like(x)
        arrs["output"] = out
        req = self.dit_block_request(tokens, hidden, heads, arrs["w_2"].shape[0], arrs["condition"].size,
                                     {k: _ptr(v) for k, v in arrs.items()}, eps, theta, axes)
        res = PrometheusBlockResult()
        rc = self.lib.prometheus_reactor_runtime_dit_block_bf16(self.handle, byref(req), byref(res))
        return rc, res, out

    def decoder_layer_f32_device(self, req: PrometheusDecoderLayerF32Request) -> PrometheusBlockResult:
        res = PrometheusBlockResult()
        rc = self.lib.prometheus_reactor_runtime_decoder_layer_f32_device(self.handle, byref(req), byref(res))
        if rc != PROM_OK:
            raise ReactorIssue("decoder_layer_failed", f"error({stage_name(res.stage)},{res.detail_code})")
        return res

    def dit_block_bf16_device(self, req: PrometheusDitBlockBf16Request) -> PrometheusBlockResult:
        res = PrometheusBlockResult()
        rc = self.lib.prometheus_reactor_runtime_dit_block_bf16_device(self.handle, byref(req), byref(res))
        if rc != PROM_OK:
            raise ReactorIssue("dit_block_failed", f"error({stage_name(res.stage)},{res.detail_code})")
        return res

    def upload_new(self, arr: np.ndarray) -> int:
        """Allocates a device buffer holding a copy of ``arr``; returns its address."""
        arr = np.ascontiguousarray(arr)
        ptr = self.alloc(max(arr.nbytes, 1))
        self.upload(ptr, arr)
        return ptr

    # -- device-resident operations ----------------------------------------
    def alloc(self, nbytes: int) -> int:
        p = c_void_p()
        rc = self.lib.prometheus_reactor_runtime_device_alloc(self.handle, nbytes, byref(p))
        if rc != PROM_OK:
            raise ReactorIssue("alloc_failed", f"device_alloc({nbytes}) returned {rc}")
        return p.value

    def free(self, ptr: int) -> None:
        self.lib.prometheus_reactor_runtime_device_free(self.handle, c_void_p(ptr))

    def upload(self, dptr: int, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        rc = self.lib.prometheus_reactor_runtime_device_upload(self.handle, c_void_p(dptr), _ptr(arr), arr.nbytes)
        if rc != PROM_OK:
            raise ReactorIssue("upload_failed", f"device_upload returned {rc}")

    def download(self, arr: np.ndarray, dptr: int) -> np.ndarray:
        rc = self.lib.prometheus_reactor_runtime_device_download(self.handle, _ptr(arr), c_void_p(dptr), arr.nbytes)
        if rc != PROM_OK:
            raise ReactorIssue("download_failed", f"device_download returned {rc}")
        return arr

    def synchronize(self) -> None:
        rc = self.lib.prometheus_reactor_runtime_synchronize(self.handle)
        if rc != PROM_OK:
            raise ReactorIssue("sync_failed", f"synchronize returned {rc}")

    def event_record(self, slot: int) -> None:
        if self.lib.prometheus_reactor_runtime_event_record(self.handle, slot) != PROM_OK:
            raise ReactorIssue("event_failed", "event_record failed")

    def event_elapsed_ms(self, start: int, end: int) -> float:
        ms = c_float(0.0)
        if self.lib.prometheus_reactor_runtime_event_elapsed_ms(self.handle, start, end, byref(ms)) != PROM_OK:
            raise ReactorIssue("event_failed", "event_elapsed_ms failed")
        return ms.value

    def _check(self, rc: int, stage: c_uint32, detail: c_int, what: str) -> int:
        if rc != PROM_OK:
            raise ReactorIssue(f"{what}_failed", f"error({stage_name(stage.value)},{detail.value})")
        return detail.value

    def sgemm_device(self, da: int, db: int, dc: int, m: int, n: int, k: int) -> int:
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_sgemm_device(self.handle, c_void_p(da), c_void_p(db), c_void_p(dc),
                                                              m, n, k, byref(stage), byref(detail))
        return self._check(rc, stage, detail, "sgemm_device")

    def sgemm_device_variant(self, da: int, db: int, dc: int, m: int, n: int, k: int, tile: int,
                             k_slices: int) -> Tuple[int, CallStatus]:
        """One product with a chosen kernel variant: (rc, stage/detail); does not raise."""
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_sgemm_device_variant(self.handle, c_void_p(da), c_void_p(db),
                                                                       c_void_p(dc), m, n, k, tile, k_slices,
                                                                       byref(stage), byref(detail))
        return rc, CallStatus(stage.value, detail.value)

    def attention_bf16_device(self, dq: int, dk: int, dv: int, do: int, tokens: int, heads: int, ld: int,
                              variant: int = 0) -> Tuple[int, CallStatus]:
        """bf16 flash attention on device buffers [tokens, ld]: (rc, stage/detail); does not raise."""
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_attention_bf16_device(self.handle, c_void_p(dq), c_void_p(dk),
                                                                        c_void_p(dv), c_void_p(do), tokens, heads,
                                                                        ld, variant, byref(stage), byref(detail))
        return rc, CallStatus(stage.value, detail.value)

    def sgemm_device_noalloc(self, da: int, db: int, dc: int, m: int, n: int, k: int) -> Tuple[int, CallStatus]:
        """The allocation-free SGEMM entry: (rc, stage/detail); does not raise."""
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_sgemm_device_noalloc(self.handle, c_void_p(da), c_void_p(db),
                                                                       c_void_p(dc), m, n, k, byref(stage),
                                                                       byref(detail))
        return rc, CallStatus(stage.value, detail.value)

    def gemm_bf16_device(self, da: int, db: int, dc: int, m: int, n: int, k: int) -> int:
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_gemm_bf16_device(self.handle, c_void_p(da), c_void_p(db),
                                                                  c_void_p(dc), m, n, k, byref(stage), byref(detail))
        return self._check(rc, stage, detail, "gemm_bf16_device")

    def reduction_device(self, din: int, dout: int, rows: int, width: int, operation: int) -> int:
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_reduction_device(self.handle, c_void_p(din), c_void_p(dout), rows,
                                                                  width, operation, byref(stage), byref(detail))
        return self._check(rc, stage, detail, "reduction_device")

    def rmsnorm_device(self, din: int, dw: int, dout: int, dinv: Optional[int], tokens: int, width: int,
                       stride: int, eps: float) -> int:
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_rmsnorm_device(
            self.handle, c_void_p(din), c_void_p(dw), c_void_p(dout), c_void_p(dinv) if dinv else None,
            tokens, width, stride, eps, byref(stage), byref(detail))
        return self._check(rc, stage, detail, "rmsnorm_device")

    # -- asynchronous SGEMM (bridge.go:438-470) ------------------------------
    def submit_async(self, m: int, n: int, k: int, a, b) -> Tuple[int, int, CallStatus]:
        """Returns (rc, task_id, status); A and B may be reused as soon as this returns."""
        a, b = _f32(a), _f32(b)
        task, stage, detail = c_int(-1), c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_sgemm_submit_async(
            self.handle, _ptr(a), _ptr(b), m, n, k, byref(task), byref(stage), byref(detail))
        return rc, task.value, CallStatus(stage.value, detail.value)

    def query_async(self, task_id: int) -> Tuple[int, PrometheusAsyncStatus]:
        st = PrometheusAsyncStatus()
        rc = self.lib.prometheus_reactor_runtime_sgemm_query_async(self.handle, task_id, byref(st))
        return rc, st

    def wait_async(self, task_id: int, timeout_s: float = 30.0) -> PrometheusAsyncStatus:
        """Polls query_async until the task leaves SUBMITTED (bounded by timeout_s)."""
        import time

        deadline = time.monotonic() + timeout_s
        while True:
            rc, st = self.query_async(task_id)
            if rc != PROM_OK or st.lifecycle_state != ASYNC_SUBMITTED or time.monotonic() > deadline:
                return st
            time.sleep(0.0005)

    def consume_async(self, task_id: int, out: Optional[np.ndarray], c_len: Optional[int] = None):
        stage, detail = c_uint32(0), c_int(0)
        if c_len is None:
            c_len = out.size if out is not None else 0
        rc = self.lib.prometheus_reactor_runtime_sgemm_consume_async(
            self.handle, task_id, _ptr(out), c_len, byref(stage), byref(detail))
        return rc, CallStatus(stage.value, detail.value)

    def abandon_async(self, task_id: int) -> int:
        return self.lib.prometheus_reactor_runtime_sgemm_abandon_async(self.handle, task_id)

    def async_diagnostics(self) -> PrometheusSgemmAsyncDiagnostics:
        d = PrometheusSgemmAsyncDiagnostics()
        rc = self.lib.prometheus_reactor_runtime_sgemm_async_diagnostics(self.handle, byref(d))
        if rc != PROM_OK:
            raise ReactorIssue("diagnostics_failed", f"async_diagnostics returned {rc}")
        return d

    # -- batched SGEMM (reactor_api.h:2610-2622) -----------------------------
    def sgemm_batch(self, problems, flags: int = 0, test_entry: bool = False):
        """problems: list of (a[m,k], b[k,n]).  Outputs start at -1 so that a
        failed batch's untouched outputs are visible.  Returns (rc, status, outputs)."""
        entries = (PrometheusSgemmBatchEntry * max(1, len(problems)))()
        keep, outs = [], []
        for i, (a, b) in enumerate(problems):
            a, b = _f32(a), _f32(b)
            m, k = a.shape
            n = b.shape[1]
            c = np.full((m, n), -1.0, np.float32)
            keep.append((a, b))
            outs.append(c)
            entries[i] = PrometheusSgemmBatchEntry(_ptr(a), _ptr(b), _ptr(c), m, n, k)
        rc, status = self.sgemm_batch_raw(entries, len(problems), flags, test_entry)
        return rc, status, outs

    def sgemm_batch_raw(self, entries, count: int, flags: int = 0, test_entry: bool = False):
        stage, detail = c_uint32(0), c_int(0)
        fn = (self.lib.prometheus_reactor_runtime_sgemm_batch_m31_test if test_entry
              else self.lib.prometheus_reactor_runtime_sgemm_batch)
        rc = fn(self.handle, entries, count, flags, byref(stage), byref(detail))
        return rc, CallStatus(stage.value, detail.value)

    # -- binary64 FFT (fft.go:33-40, reactor_concept_fft.cpp:97-104) ----------
    def fft64(self, values, output: Optional[np.ndarray] = None):
        """Forward unnormalised FFT of complex128 values; returns (rc, status, spectrum)."""
        x = np.ascontiguousarray(values, dtype=np.complex128)
        out = np.empty_like(x) if output is None else output
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_fft64(self.handle, _ptr(x) if x.size else None,
                                                       _ptr(out) if out.size else None, x.size,
                                                       byref(stage), byref(detail))
        return rc, CallStatus(stage.value, detail.value), out

    # -- batched complex-fp32 FFT (reactor_api.h:2656-2670) -------------------
    def fft(self, values, count: int, batch: int = 1, stride: int = 0, flags: int = 0,
            output: Optional[np.ndarray] = None, variant: Optional[int] = None, request_patch=None):
        """complex64 ``values`` holding ``batch`` sequences of ``count`` points
        ``stride`` apart (0: contiguous); returns (rc, status, output)."""
        x = np.ascontiguousarray(values, dtype=np.complex64)
        out = np.zeros_like(x) if output is None else output
        r = PrometheusFftRequest()
        r.struct_size = ctypes.sizeof(r)
        r.input = _ptr(x) if x.size else None
        r.output = _ptr(out) if out.size else None
        r.element_count, r.batch_count, r.stride_elements, r.flags = count, batch, stride, flags
        if request_patch:
            request_patch(r)
        stage, detail = c_uint32(0), c_int(0)
        if variant is None:
            rc = self.lib.prometheus_reactor_runtime_fft(self.handle, byref(r), byref(stage), byref(detail))
        else:
            rc = self.lib.prometheus_reactor_runtime_fft_benchmark_variant(self.handle, byref(r), variant,
                                                                         byref(stage), byref(detail))
        return rc, CallStatus(stage.value, detail.value), out

    def fft_diagnostics(self, size: Optional[int] = None) -> PrometheusFftDiagnostics:
        d = PrometheusFftDiagnostics()
        rc = (self.lib.prometheus_reactor_runtime_fft_diagnostics(self.handle, byref(d)) if size is None else
              self.lib.prometheus_reactor_runtime_fft_diagnostics_sized(self.handle, byref(d), size))
        if rc != PROM_OK:
            raise ReactorIssue("fft_diagnostics_failed", f"rc={rc}")
        return d

    def fft64_device(self, din: int, dout: int, count: int) -> int:
        stage, detail = c_uint32(0), c_int(0)
        rc = self.lib.prometheus_reactor_runtime_fft64_device(self.handle, c_void_p(din), c_void_p(dout), count,
                                                              byref(stage), byref(detail))
        return self._check(rc, stage, detail, "fft64_device")

    def batch_diagnostics(self) -> PrometheusSgemmBatchDiagnostics:
        d = PrometheusSgemmBatchDiagnostics()
        rc = self.lib.prometheus_reactor_runtime_sgemm_batch_diagnostics(self.handle, byref(d))
        if rc != PROM_OK:
            raise ReactorIssue("diagnostics_failed", f"batch_diagnostics returned {rc}")
        return d


def sgemm_plan(m: int, n: int, k: int, lib: Optional[ctypes.CDLL] = None) -> Tuple[int, PrometheusSgemmPlanInfo]:
    """The launch plan of a contiguous m x n x k SGEMM (no device needed): (rc, plan)."""
    lib = lib or shared_library()
    info = PrometheusSgemmPlanInfo()
    info.struct_size = ctypes.sizeof(info)
    rc = lib.prometheus_reactor_sgemm_plan(m, n, k, byref(info))
    return rc, info


# ---- the strict `@` path (strict.go:11-32, runtime.go:251-317) -------------
def compiled_matmul_request(left: Sequence[Sequence[float]], right: Sequence[Sequence[float]]):
    """runtime.go:251-306: shape checks and float64 -> float32 (RNE) flattening."""
    if len(left) == 0 or len(right) == 0:
        raise ValueError("compiled Prometheus matmul requires non-empty matrices")
    k = len(left[0])
    if any(len(r) != k for r in left):
        raise ValueError("compiled Prometheus matmul requires rectangular matrices")
    if k == 0:
        raise ValueError("compiled Prometheus matmul requires matrices with at least one column")
    n = len(right[0])
    if any(len(r) != n for r in right):
        raise ValueError("compiled Prometheus matmul requires rectangular matrices")
    if n == 0:
        raise ValueError("compiled Prometheus matmul requires matrices with at least one column")
    if k != len(right):
        raise ValueError(f"compiled Prometheus matmul shape mismatch: left columns={k} right rows={len(right)}")
    a = np.asarray(left, dtype=np.float64).astype(np.float32)
    b = np.asarray(right, dtype=np.float64).astype(np.float32)
    return len(left), n, k, a, b


def run_compiled_matmul_mm_strict(left, right) -> Tuple[list, str]:
    """strict.go:11-32: GPU or error, never a CPU substitute."""
    m, n, k, a, b = compiled_matmul_request(left, right)
    try:
        rt = NativeRuntime()
    except ReactorIssue as exc:
        raise StrictExecutionError(f"PROMETHEUS requires GPU matrix execution: {exc.message}") from exc
    with rt:
        try:
            rt.require_hardware_gpu()
        except ReactorIssue as exc:
            raise StrictExecutionError(f"PROMETHEUS requires GPU matrix execution: {exc.message}") from exc
        try:
            out, status = rt.sgemm(m, n, k, a, b)
        except ReactorIssue as exc:
            raise StrictExecutionError(f"PROMETHEUS requires GPU matrix execution: {exc.message}") from exc
        env = rt.environment()
    return out.reshape(m, n).astype(np.float64).tolist(), env
