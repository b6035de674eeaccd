"""Host mirror of the resident model-block ABI (reactor_api.h:666-1249, 2713-2808).

Thin ctypes calls over ``libprometheus_reactor.so``; each returns
``(rc, evidence)`` with the reference's evidence struct, so callers check the
same detail codes the reference's Marionette tests do
(internal/prometheus/native/Marionette/reactor_model_block_tests.cpp).
Weights are passed as FP16 numpy arrays in the cache-manifest order of the
Z-Image Turbo layer (``oracle``-independent: ``ZIMAGE_TENSORS`` below).
"""
from __future__ import annotations

import ctypes
from ctypes import byref, c_uint64
from typing import Optional, Sequence

import numpy as np

from . import prometheus as p

ZIMAGE_TENSORS = ("adaln_b", "adaln_w", "k_norm", "w_out", "q_norm", "w_qkv", "attn_norm1", "attn_norm2",
                  "w1", "w2", "w3", "ffn_norm1", "ffn_norm2")
CONTEXT_TENSORS = ZIMAGE_TENSORS[2:]
STEPS = (1, 2, 3, 4, 5, 6, 7)
WIDTH, IMAGE_TOKENS, CONTEXT_TOKENS, JOINT_TOKENS = 3840, 1024, 32, 1056


class Uploads:
    """A PrometheusModelBlockWeightUpload array that keeps its byte buffers alive."""

    def __init__(self, arrays: Sequence[np.ndarray], content_base: int, layout_base: int = 0x6B00):
        self.arrays = [np.ascontiguousarray(a) for a in arrays]
        self.items = (p.PrometheusModelBlockWeightUpload * len(self.arrays))()
        for i, a in enumerate(self.arrays):
            u = self.items[i]
            u.binding_index = i
            u.bytes = a.ctypes.data
            u.byte_count = a.nbytes
            u.content_identity = content_base + i
            u.layout_identity = layout_base + i

    def __len__(self):
        return len(self.arrays)

    def pointer(self):
        return ctypes.cast(self.items, ctypes.POINTER(p.PrometheusModelBlockWeightUpload))


def zimage_uploads(weights: dict, content_base: int, names=ZIMAGE_TENSORS) -> Uploads:
    return Uploads([np.asarray(weights[n], dtype=np.float16) for n in names], content_base)


def create_request(uploads: Uploads, *, shader_id: int = 23, family: int = 0, parameter_set: int = 0,
                   aggregate: int = 0, external_input_bytes: int = 0, external_output_bytes: int = 0,
                   audit_bytes: int = 256, memory_ceiling: int = 1 << 40,
                   steps: Sequence[int] = STEPS) -> p.PrometheusModelBlockCreateRequest:
    r = p.PrometheusModelBlockCreateRequest()
    r.struct_size = ctypes.sizeof(r)
    r.assembly_family = family
    r.parameter_set = parameter_set
    r.parameter_set_aggregate_identity = aggregate
    r.model_contract_identity = 0x101
    r.weight_identity = 0x102
    r.shader_portfolio_identity = 0x103
    r.precision_policy_identity = 0x104
    r.capability_route_identity = 0x105
    r.memory_ceiling_bytes = memory_ceiling
    r.external_input_bytes = external_input_bytes
    r.external_output_bytes = external_output_bytes
    r.audit_bytes = audit_bytes
    r.shader_id = shader_id
    r.weight_count = len(uploads)
    for i, u in enumerate(uploads.items):
        r.weights[i].content_identity = u.content_identity
        r.weights[i].layout_identity = u.layout_identity
        r.weights[i].byte_count = u.byte_count
    r.step_count = len(steps)
    for i, s in enumerate(steps):
        r.steps[i] = s
    return r


class ResidentModel:
    """One runtime's model block and session, called through the C ABI."""

    def __init__(self, rt: p.NativeRuntime):
        self.rt = rt
        self.lib = rt.lib
        self.h = rt.handle

    # -- generic block -------------------------------------------------------
    def create(self, request: p.PrometheusModelBlockCreateRequest):
        ev = p.PrometheusModelBlockEvidence()
        bid = c_uint64(0)
        rc = self.lib.prometheus_reactor_runtime_model_block_create(self.h, byref(request), byref(bid), byref(ev))
        return rc, bid.value, ev

    def upload(self, block_id: int, uploads: Uploads, count: Optional[int] = None):
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_model_block_upload_weights(
            self.h, block_id, uploads.pointer(), len(uploads) if count is None else count, byref(ev))
        return rc, ev

    def execute(self, block_id: int, x: np.ndarray, out: np.ndarray, input_identity: int = 0x8ABC,
                audit: Optional[np.ndarray] = None, request_patch=None):
        r = p.PrometheusModelBlockExecuteRequest()
        r.struct_size = ctypes.sizeof(r)
        r.input = x.ctypes.data
        r.output = out.ctypes.data
        r.element_count = x.size
        r.input_identity = input_identity
        if audit is not None:
            r.audit_enabled = 1
            r.audit_output = audit.ctypes.data
            r.audit_element_capacity = audit.size
        if request_patch:
            request_patch(r)
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_model_block_execute(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    def evidence(self, block_id: int):
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_model_block_get_evidence(self.h, block_id, byref(ev))
        return rc, ev

    def destroy(self, block_id: int) -> int:
        return self.lib.prometheus_reactor_runtime_model_block_destroy(self.h, block_id)

    # -- NoiseRefiner ----------------------------------------------------------
    def noise_refiner_create(self, weights: dict, parameter_set: int = 1, content_base: int = 0x5A00,
                             audit_bytes: int = 65536 * 4):
        uploads = zimage_uploads(weights, content_base)
        req = create_request(uploads, shader_id=p.PROM_MODEL_BLOCK_SHADER_NOISE, family=p.PROM_NOISE_REFINER_FAMILY,
                             parameter_set=parameter_set, aggregate=p.NOISE_REFINER_AGGREGATES[parameter_set - 1],
                             external_input_bytes=IMAGE_TOKENS * WIDTH * 2, audit_bytes=audit_bytes,
                             memory_ceiling=512 << 20)
        rc, bid, ev = self.create(req)
        if rc != p.PROM_OK:
            return rc, bid, ev
        rc, ev = self.upload(bid, uploads)
        return rc, bid, ev

    def noise_refiner_execute(self, block_id: int, model_input_bf16: np.ndarray, timestep_bf16: np.ndarray,
                              parameter_set: int = 1, output_identity: int = 0x0E01, request_patch=None):
        r = p.PrometheusNoiseRefiner0ExecuteRequest()
        r.struct_size = ctypes.sizeof(r)
        r.model_input_bf16 = model_input_bf16.ctypes.data
        r.timestep_bf16 = timestep_bf16.ctypes.data
        r.model_input_bytes = model_input_bf16.nbytes
        r.timestep_bytes = timestep_bf16.nbytes
        r.input_identity = 0x1A01
        r.timestep_identity = 0x1B01
        r.output_identity = output_identity
        if request_patch:
            request_patch(r)
        ev = p.PrometheusModelBlockEvidence()
        fn = (self.lib.prometheus_reactor_runtime_noise_refiner0_execute if parameter_set == 1
              else self.lib.prometheus_reactor_runtime_noise_refiner1_execute)
        rc = fn(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    def noise_refiner_rebind(self, block_id: int, weights: dict, content_base: int = 0x7A00,
                             model_local_block_id: int = 1, lock: int = p.PROM_ZIMAGE_TURBO_LOCK_ID):
        uploads = zimage_uploads(weights, content_base)
        r = p.PrometheusNoiseRefinerRebindRequest()
        r.struct_size = ctypes.sizeof(r)
        r.model_local_block_id = model_local_block_id
        r.lock_identity = lock
        r.upload_count = len(uploads)
        r.uploads = ctypes.cast(uploads.items, ctypes.c_void_p)
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_noise_refiner_rebind(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    def noise_refiner_resident(self, block_id: int, input_generation: int, output_identity: int = 0x0E02,
                               audit_family: int = 0, audit_stage: int = 0, audit: Optional[np.ndarray] = None):
        r = p.PrometheusNoiseRefinerResidentExecuteRequest()
        r.struct_size = ctypes.sizeof(r)
        r.input_generation = input_generation
        r.output_identity = output_identity
        if audit is not None:
            r.audit_enabled = 1
            r.audit_family = audit_family
            r.audit_stage = audit_stage
            r.audit_output = audit.ctypes.data
            r.audit_element_capacity = audit.size
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_noise_refiner_execute_resident(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    # -- stage-split NoiseRefiner (reactor_api.h:957-1007, 2722-2730) -----------
    def execute_m1b(self, block_id: int, model_input_bf16: np.ndarray, timestep_bf16: np.ndarray,
                    audit_stage: int = 0, audit: Optional[np.ndarray] = None, input_identity: int = 0x51,
                    timestep_identity: int = 0x52, request_patch=None):
        r = p.PrometheusModelBlockM1BExecuteRequest()
        r.struct_size = ctypes.sizeof(r)
        r.model_input_bf16 = model_input_bf16.ctypes.data
        r.timestep_bf16 = timestep_bf16.ctypes.data
        r.model_input_bytes = model_input_bf16.nbytes
        r.timestep_bytes = timestep_bf16.nbytes
        r.input_identity = input_identity
        r.timestep_identity = timestep_identity
        if audit is not None:
            r.audit_enabled = 1
            r.audit_stage = audit_stage
            r.audit_output = audit.ctypes.data
            r.audit_element_capacity = audit.size
        if request_patch:
            request_patch(r)
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_model_block_execute_m1b(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    def execute_m1c(self, block_id: int, prefix: int, out: np.ndarray, audit_stage: int = 3,
                    transient: Optional[np.ndarray] = None, output_identity: int = 0x53, request_patch=None):
        r = p.PrometheusModelBlockM1CExecuteRequest()
        r.struct_size = ctypes.sizeof(r)
        r.m1b_prefix_replay_identity = prefix
        r.output_identity = output_identity
        r.output = out.ctypes.data
        r.output_element_capacity = out.size
        r.audit_stage = audit_stage
        if transient is not None:
            r.transient_audit = transient.ctypes.data
            r.transient_audit_element_capacity = transient.size
        if request_patch:
            request_patch(r)
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_model_block_execute_m1c(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    def execute_m1d(self, block_id: int, prefix: int, out: np.ndarray, audit_stage: int = 7,
                    output_identity: int = 0x54, request_patch=None):
        r = p.PrometheusModelBlockM1DExecuteRequest()
        r.struct_size = ctypes.sizeof(r)
        r.m1c_prefix_replay_identity = prefix
        r.output_identity = output_identity
        r.output = out.ctypes.data
        r.output_element_capacity = out.size
        r.audit_stage = audit_stage
        if request_patch:
            request_patch(r)
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_model_block_execute_m1d(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    # -- static audits (reactor_api.h:1070-1093, 2743-2778) ----------------------
    def static_audit(self, kind: str, block_id: int, input_generation: int, arena: np.ndarray,
                     output_identity: int = 0x57, lock: int = p.PROM_ZIMAGE_TURBO_AUDIT_LOCK_ID):
        """``kind`` "noise" or "context"; ``arena`` a uint8 array of the arena capacity."""
        r = p.PrometheusNoiseRefinerStaticAuditRequest()
        r.struct_size = ctypes.sizeof(r)
        r.lock_identity = lock
        r.input_generation = input_generation
        r.output_identity = output_identity
        r.audit_arena = arena.ctypes.data
        r.audit_arena_capacity_bytes = arena.nbytes
        ev = p.PrometheusModelBlockEvidence()
        fn = {"noise": self.lib.prometheus_reactor_runtime_noise_refiner_execute_static_audit,
              "context": self.lib.prometheus_reactor_runtime_context_refiner_execute_static_audit}[kind]
        rc = fn(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    def main_static_audit(self, block_id: int, session_id: int, image_gen: int, context_gen: int, joint_gen: int,
                          arena: np.ndarray, output_identity: int = 0x58, layer: int = 0):
        r = p.PrometheusMainTransformerStaticAuditRequest()
        r.struct_size = ctypes.sizeof(r)
        r.session_identity = session_id
        r.lock_identity = p.PROM_ZIMAGE_TURBO_AUDIT_LOCK_ID
        r.model_local_block_id = layer
        r.required_image_generation = image_gen
        r.required_context_generation = context_gen
        r.required_joint_generation = joint_gen
        r.output_identity = output_identity
        r.audit_arena = arena.ctypes.data
        r.audit_arena_capacity_bytes = arena.nbytes
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_main_transformer_execute_static_audit(self.h, block_id, byref(r),
                                                                                       byref(ev))
        return rc, ev

    def audit_final(self, kind: str, block_id: int, generation: int, out: np.ndarray, output_identity: int = 0xA0D1):
        r = p.PrometheusNoiseRefinerFinalAuditRequest()
        r.struct_size = ctypes.sizeof(r)
        r.required_output_generation = generation
        r.output_identity = output_identity
        r.output = out.ctypes.data
        r.output_element_capacity = out.size
        ev = p.PrometheusModelBlockEvidence()
        fn = {"noise": self.lib.prometheus_reactor_runtime_noise_refiner_audit_final,
              "context": self.lib.prometheus_reactor_runtime_context_refiner_audit_final,
              "main": self.lib.prometheus_reactor_runtime_main_transformer_audit_final}[kind]
        rc = fn(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    # -- ContextRefiner and MainTransformer facades -----------------------------
    def _lock_request(self, uploads: Uploads, model_local_block_id: int, lock: int):
        r = p.PrometheusContextRefinerCreateRequest()
        r.struct_size = ctypes.sizeof(r)
        r.model_local_block_id = model_local_block_id
        r.lock_identity = lock
        r.upload_count = len(uploads)
        r.uploads = ctypes.cast(uploads.items, ctypes.c_void_p)
        return r

    def context_refiner_create(self, weights: dict, content_base: int = 0x5C00, lock: int = p.PROM_ZIMAGE_TURBO_LOCK_ID):
        uploads = zimage_uploads(weights, content_base, CONTEXT_TENSORS)
        r = self._lock_request(uploads, 0, lock)
        ev = p.PrometheusModelBlockEvidence()
        bid = c_uint64(0)
        rc = self.lib.prometheus_reactor_runtime_context_refiner_create(self.h, byref(r), byref(bid), byref(ev))
        return rc, bid.value, ev

    def context_refiner_rebind(self, block_id: int, weights: dict, content_base: int = 0x7C00):
        uploads = zimage_uploads(weights, content_base, CONTEXT_TENSORS)
        r = self._lock_request(uploads, 1, p.PROM_ZIMAGE_TURBO_LOCK_ID)
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_context_refiner_rebind(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    def context_refiner0_execute(self, block_id: int, x: np.ndarray, output_identity: int = 0x0C01):
        r = p.PrometheusContextRefiner0ExecuteRequest()
        r.struct_size = ctypes.sizeof(r)
        r.context_input = x.ctypes.data
        r.context_input_bytes = x.nbytes
        r.input_identity = 0x1C01
        r.output_identity = output_identity
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_context_refiner0_execute(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    def context_refiner_resident(self, block_id: int, input_generation: int, output_identity: int = 0x0C02):
        r = p.PrometheusContextRefinerResidentExecuteRequest()
        r.struct_size = ctypes.sizeof(r)
        r.input_generation = input_generation
        r.output_identity = output_identity
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_context_refiner_execute_resident(self.h, block_id, byref(r),
                                                                                   byref(ev))
        return rc, ev

    def main_transformer_create(self, layer: int, weights: dict, content_base: int = 0x5D00):
        uploads = zimage_uploads(weights, content_base)
        r = self._lock_request(uploads, layer, p.PROM_ZIMAGE_TURBO_LOCK_ID)
        ev = p.PrometheusModelBlockEvidence()
        bid = c_uint64(0)
        rc = self.lib.prometheus_reactor_runtime_main_transformer_create(self.h, byref(r), byref(bid), byref(ev))
        return rc, bid.value, ev

    def main_transformer_rebind(self, block_id: int, layer: int, weights: dict, content_base: int = 0x7D00):
        uploads = zimage_uploads(weights, content_base)
        r = self._lock_request(uploads, layer, p.PROM_ZIMAGE_TURBO_LOCK_ID)
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_main_transformer_rebind(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    def main_transformer_execute(self, block_id: int, session_id: int, layer: int, timestep_bf16: np.ndarray,
                                 image_gen: int, context_gen: int, joint_gen: int, chain: bool = False,
                                 output_identity: int = 0x0D01):
        r = p.PrometheusMainTransformerExecuteRequest()
        r.struct_size = ctypes.sizeof(r)
        r.session_identity = session_id
        r.lock_identity = p.PROM_ZIMAGE_TURBO_LOCK_ID
        r.model_local_block_id = layer
        r.resident_chain_mode = 1 if chain else 0
        r.required_image_generation = image_gen
        r.required_context_generation = context_gen
        r.required_joint_generation = joint_gen
        r.timestep_bf16 = timestep_bf16.ctypes.data
        r.timestep_bytes = timestep_bf16.nbytes
        r.timestep_identity = 0x1B02
        r.output_identity = output_identity
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_main_transformer_execute(self.h, block_id, byref(r), byref(ev))
        return rc, ev

    # -- session -----------------------------------------------------------------
    def session_create(self, lock: int = p.PROM_ZIMAGE_TURBO_LOCK_ID, profile: int = 1, route: int = 1):
        r = p.PrometheusCompiledModelSessionCreateRequest()
        r.struct_size = ctypes.sizeof(r)
        r.lock_identity = lock
        r.execution_profile = profile
        r.main_attention_route_policy = route
        ev = p.PrometheusCompiledModelSessionEvidence()
        sid = c_uint64(0)
        rc = self.lib.prometheus_reactor_runtime_compiled_model_session_create(self.h, byref(r), byref(sid),
                                                                                byref(ev))
        return rc, sid.value, ev

    def session_capture(self, session_id: int, block_id: int, generation: int):
        r = p.PrometheusCompiledModelSessionCaptureRequest()
        r.struct_size = ctypes.sizeof(r)
        r.source_output_generation = generation
        ev = p.PrometheusCompiledModelSessionEvidence()
        rc = self.lib.prometheus_reactor_runtime_compiled_model_session_capture_completed(
            self.h, session_id, block_id, byref(r), byref(ev))
        return rc, ev

    def session_compose(self, session_id: int, image_gen: int, context_gen: int):
        r = p.PrometheusCompiledModelSessionComposeRequest()
        r.struct_size = ctypes.sizeof(r)
        r.required_image_generation = image_gen
        r.required_context_generation = context_gen
        ev = p.PrometheusCompiledModelSessionEvidence()
        rc = self.lib.prometheus_reactor_runtime_compiled_model_session_compose_joint(self.h, session_id, byref(r),
                                                                                      byref(ev))
        return rc, ev

    def session_evidence(self, session_id: int):
        ev = p.PrometheusCompiledModelSessionEvidence()
        rc = self.lib.prometheus_reactor_runtime_compiled_model_session_get_evidence(self.h, session_id, byref(ev))
        return rc, ev

    def set_main_attention_route(self, session_id: int, route: int, evidence: bool = True):
        ev = p.PrometheusCompiledModelSessionEvidence()
        rc = self.lib.prometheus_reactor_runtime_compiled_model_session_set_main_attention_route(
            self.h, session_id, route, byref(ev) if evidence else None)
        return rc, ev

    def session_destroy(self, session_id: int) -> int:
        return self.lib.prometheus_reactor_runtime_compiled_model_session_destroy(self.h, session_id)

    # -- the compiled-model owner (tools/prometheus_zimage_bridge/reactor_windows.go:190-238)
    def owner_create(self, weights: dict, content_base: int = 0x5E00):
        uploads = zimage_uploads(weights, content_base)
        r = self._lock_request(uploads, 0, p.PROM_ZIMAGE_TURBO_LOCK_ID)
        ev = p.PrometheusModelBlockEvidence()
        bid = c_uint64(0)
        rc = self.lib.prometheus_reactor_runtime_compiled_model_owner_create(self.h, byref(r), byref(bid), byref(ev))
        return rc, bid.value, ev

    def _retarget_request(self, session_id: int, local: int, uploads: Uploads):
        r = p.PrometheusCompiledModelRetargetRequest()
        r.struct_size = ctypes.sizeof(r)
        r.session_identity = session_id
        r.lock_identity = p.PROM_ZIMAGE_TURBO_LOCK_ID
        r.model_local_block_id = local
        r.upload_count = len(uploads)
        r.uploads = ctypes.cast(uploads.items, ctypes.c_void_p)
        return r

    def retarget(self, session_id: int, local: int, weights: dict, names=ZIMAGE_TENSORS, content_base: int = 0x5F00):
        uploads = zimage_uploads(weights, content_base, names)
        r = self._retarget_request(session_id, local, uploads)
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_compiled_model_retarget(self.h, byref(r), byref(ev))
        return rc, ev

    def prefetch(self, session_id: int, local: int, weights: dict, names=ZIMAGE_TENSORS):
        uploads = zimage_uploads(weights, 0x6F00, names)
        r = self._retarget_request(session_id, local, uploads)
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_compiled_model_prefetch(self.h, byref(r), byref(ev))
        return rc, ev

    def activate_prefetch(self, session_id: int):
        ev = p.PrometheusModelBlockEvidence()
        rc = self.lib.prometheus_reactor_runtime_compiled_model_activate_prefetch(self.h, session_id, byref(ev))
        return rc, ev

    def evaluation_reset(self, session_id: int):
        ev = p.PrometheusCompiledModelSessionEvidence()
        rc = self.lib.prometheus_reactor_runtime_compiled_model_evaluation_reset(self.h, session_id, byref(ev))
        return rc, ev
