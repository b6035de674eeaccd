"""GPU checks of the resident model-block ABI (reactor_api.h:2713-2808) and
parity of its fp32 Z-Image blocks with the binary64 oracle.

Lifecycle cases follow the reference's Marionette facts
(internal/prometheus/native/Marionette/reactor_model_block_tests.cpp:201-405):
the closed resident program stays warm (no allocation, upload or pipeline
creation after the cold start), faults are consumed in execution order and
recover, and stale generations are rejected.  Numerics use the reference's
accepted FP32 bound for a block against its canonical stage, relative L2
<= 5e-5 (reactor_model_block_tests.cpp:1945, 2236, 3679), on seeded random
FP16 weights and BF16 inputs at the lock's shapes (1024 image, 32 context,
1056 joint tokens; width 3840, 30 heads, FFN 10240).
"""
import json
import threading
import time
from pathlib import Path

import numpy as np
import pytest

import oracle
from oracle import blocks
from oct_amd import model_block as mb
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu

BAR = 5e-5
D = p.PROM_MODEL_BLOCK_DETAIL
W, T_IMG, T_CTX, T_JOINT = 3840, 1024, 32, 1056
ROWS_IMG = np.array([0, 1, 31, 32, 33, 511, 512, 1000, 1023])
ROWS_JOINT = np.concatenate((ROWS_IMG, np.arange(1024, 1056, 7), [1055]))


def rel_l2(got, ref):
    return float(np.linalg.norm(np.asarray(got, np.float64) - ref) / np.linalg.norm(ref))


@pytest.fixture
def model():
    rt = p.NativeRuntime()
    assert rt.available, "HIP device unavailable: GPU tests must run on the MI355X box"
    yield mb.ResidentModel(rt)
    rt.close()


def runtime_model(**kw):
    rt = p.NativeRuntime(**kw)
    assert rt.available
    return rt, mb.ResidentModel(rt)


@pytest.fixture(scope="module")
def weights():
    print("generating FP16 weights", flush=True)
    return {"nr0": blocks.make_zimage_weights(11), "nr1": blocks.make_zimage_weights(12),
            "cr0": blocks.make_zimage_weights(21, modulated=False), "cr1": blocks.make_zimage_weights(22, False),
            "main0": blocks.make_zimage_weights(31)}


@pytest.fixture(scope="module")
def inputs():
    rng = np.random.default_rng(5)
    x_bits = oracle.to_bf16(rng.standard_normal((T_IMG, W)).astype(np.float32))
    t_bits = oracle.to_bf16(rng.standard_normal(256).astype(np.float32))
    ctx = rng.standard_normal((T_CTX, W)).astype(np.float32)
    return x_bits, t_bits, ctx


# ------------------------------------------------------------ resident proof
def proof_uploads(content_base=0x200):
    return mb.Uploads([np.full(64, i, np.uint8) for i in range(13)], content_base, layout_base=0x300)


def proof_request(ups):
    return mb.create_request(ups, shader_id=23, external_input_bytes=4096, external_output_bytes=4096,
                             audit_bytes=256, memory_ceiling=1 << 20)


def test_resident_program_executes_and_stays_warm(model):
    """FACT PrometheusResidentModelBlockExecutesAClosedGpuProgramAndStaysWarm."""
    ups = proof_uploads()
    rc, bid, ev = model.create(proof_request(ups))
    assert rc == p.PROM_OK and bid != 0
    assert ev.fixed_step_count == 7 and ev.weight_count == 13 and ev.pipeline_create_count == 1
    # 13 weights + input, output, audit and upload staging, all at create
    assert ev.cold_buffer_allocation_count >= 17
    bad = proof_uploads()
    bad.items[0].content_identity = 0
    rc, ev = model.upload(bid, bad)
    assert rc == p.PROM_ERROR and ev.detail_code == D["WEIGHT_MISMATCH"]
    rc, ev = model.upload(bid, ups)
    assert rc == p.PROM_OK and ev.weights_uploaded == 1 and ev.weight_upload_count == 13
    assert ev.binding_state == 1 and ev.binding_generation == 1
    x = np.array([((i * 19) % 113 - 56) / 32.0 for i in range(1024)], np.float32)
    out = np.zeros(1024, np.float32)
    audit = np.zeros(64, np.float32)
    rc, ev = model.execute(bid, x, out, audit=audit)
    assert rc == p.PROM_OK and ev.output_valid == 1 and ev.audit_valid == 1
    np.testing.assert_array_equal(out, x)
    np.testing.assert_array_equal(audit, x[:64])
    replay, allocs, uploads = ev.replay_identity, ev.cold_buffer_allocation_count, ev.weight_upload_count
    for _ in range(10):
        out[:] = 0
        audit[:] = 0
        rc, ev = model.execute(bid, x, out, audit=audit)
        assert rc == p.PROM_OK
        assert ev.cold_buffer_allocation_count == allocs and ev.warm_buffer_allocation_count == 0
        assert ev.weight_upload_count == uploads and ev.pipeline_create_count == 1
        assert ev.replay_identity == replay
    np.testing.assert_array_equal(out, x)
    # a second upload of a bound set is a mismatch; the binding is untouched
    rc, ev = model.upload(bid, ups)
    assert rc == p.PROM_ERROR and ev.detail_code == D["WEIGHT_MISMATCH"]
    assert model.destroy(bid) == p.PROM_OK
    assert model.destroy(bid) == p.PROM_ERROR
    rc, bid2, ev = model.create(proof_request(ups))
    assert rc == p.PROM_OK and bid2 != bid
    rc, bid3, ev = model.create(proof_request(ups))
    assert rc == p.PROM_ERROR and ev.detail_code == D["ALREADY_CREATED"]
    assert model.destroy(bid2) == p.PROM_OK


def test_injected_phases_fail_in_order_and_recover():
    """FACT PrometheusConceptModelBlockOwnsResourcesAndRetiresQuarantineBeforeRootTeardown."""
    flags = (p.PROM_REDUCTION_TESTCFG_FAIL_COMMAND_RECORD | p.PROM_REDUCTION_TESTCFG_FAIL_QUEUE_SUBMIT
             | p.PROM_REDUCTION_TESTCFG_FAIL_COMPLETION_OBSERVATION)
    rt, model = runtime_model(reduction_test_flags=flags)
    try:
        ups = proof_uploads()
        rc, bid, ev = model.create(proof_request(ups))
        assert rc == p.PROM_OK
        assert model.upload(bid, ups)[0] == p.PROM_OK
        x = np.full(1024, 3.25, np.float32)
        out = np.full(1024, -99.0, np.float32)
        for expected in ("COMMAND_RECORD_FAILED", "QUEUE_SUBMIT_FAILED", "COMPLETION_UNCERTAIN"):
            rc, ev = model.execute(bid, x, out, input_identity=1)
            assert rc == p.PROM_ERROR and ev.detail_code == D[expected]
            assert out[0] == -99.0 and ev.output_valid == 0
        assert ev.quarantined == 1
        rc, ev = model.execute(bid, x, out, input_identity=1)
        assert rc == p.PROM_OK and ev.quarantined == 0 and out[0] == 3.25
        # the synchronous SGEMM shares the device with the block
        c, st, rc = rt.sgemm_with_status(1, 1, 1, np.array([2.0], np.float32), np.array([3.0], np.float32))
        assert rc == p.PROM_OK and c[0] == 6.0
    finally:
        rt.close()


def test_upload_and_readback_faults():
    rt, model = runtime_model(test_flags=p.TESTCFG_FAIL_UPLOAD)
    try:
        ups = proof_uploads()
        rc, bid, ev = model.create(proof_request(ups))
        assert rc == p.PROM_OK
        rc, ev = model.upload(bid, ups)
        assert rc == p.PROM_ERROR and ev.detail_code == D["UPLOAD_FAILED"] and ev.weights_uploaded == 0
        x = np.ones(1024, np.float32)
        rc, ev = model.execute(bid, x, np.zeros_like(x))
        assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]
    finally:
        rt.close()
    rt, model = runtime_model(test_flags=p.TESTCFG_FAIL_DOWNLOAD)
    try:
        ups = proof_uploads()
        rc, bid, ev = model.create(proof_request(ups))
        assert model.upload(bid, ups)[0] == p.PROM_OK
        x = np.ones(1024, np.float32)
        rc, ev = model.execute(bid, x, np.zeros_like(x))
        assert rc == p.PROM_ERROR and ev.detail_code == D["AUDIT_FAILED"] and ev.output_valid == 0
    finally:
        rt.close()


# ------------------------------------------------------------ NoiseRefiner
def test_noise_refiner_chain(model, weights, inputs):
    x_bits, t_bits, _ = inputs
    x = oracle.from_bf16(x_bits).astype(np.float64)
    cond = oracle.from_bf16(t_bits).astype(np.float64)
    coords = blocks.image_coordinates(T_IMG)
    print("noise refiner: create and upload", flush=True)
    rc, bid, ev = model.noise_refiner_create(weights["nr0"])
    assert rc == p.PROM_OK, ev.detail_code
    assert ev.binding_state == 1 and ev.binding_generation == 1 and ev.parameter_set == 1
    # the resident entry point belongs to parameter set 1
    rc, ev = model.noise_refiner_resident(bid, input_generation=1)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]
    rc, ev = model.noise_refiner_execute(bid, x_bits, t_bits, parameter_set=1)
    assert rc == p.PROM_OK, ev.detail_code
    assert ev.output_generation == 1 and ev.output_valid == 1 and ev.warm_buffer_allocation_count == 0
    print(f"noise refiner 0: gpu {ev.gpu_compute_ns / 1e6:.3f} ms", flush=True)
    out0 = np.zeros(T_IMG * W, np.float32)
    rc, ev = model.audit_final("noise", bid, 1, out0)
    assert rc == p.PROM_OK and ev.audit_valid == 1
    # a stale audit request fails and, as in the reference, invalidates the
    # published output; the resident chain still follows the generation
    rc, ev = model.audit_final("noise", bid, 2, np.zeros_like(out0))
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"] and ev.output_valid == 0
    out0 = out0.reshape(T_IMG, W)
    ref0 = blocks.zimage_block_f64(x, coords, weights["nr0"], cond, rows=ROWS_IMG)
    err0 = rel_l2(out0[ROWS_IMG], ref0)
    print(f"noise refiner 0 rel L2 {err0:.3e}", flush=True)
    assert err0 <= BAR

    rc, ev = model.noise_refiner_rebind(bid, weights["nr1"])
    assert rc == p.PROM_OK, ev.detail_code
    assert ev.parameter_set == 2 and ev.binding_generation == 2
    assert ev.parameter_set_aggregate_identity == p.NOISE_REFINER_AGGREGATES[1]
    rc, ev = model.noise_refiner_execute(bid, x_bits, t_bits, parameter_set=1)
    assert rc == p.PROM_ERROR and ev.detail_code == D["PARAMETER_SET_MISMATCH"]
    rc, ev = model.noise_refiner_resident(bid, input_generation=2)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]
    rc, ev = model.noise_refiner_resident(bid, input_generation=1)
    assert rc == p.PROM_OK and ev.output_generation == 2
    out1 = np.zeros(T_IMG * W, np.float32)
    assert model.audit_final("noise", bid, 2, out1)[0] == p.PROM_OK
    out1 = out1.reshape(T_IMG, W)
    stages = {}
    ref1 = blocks.zimage_block_f64(out0, coords, weights["nr1"], cond, rows=ROWS_IMG, stages=stages)
    err1 = rel_l2(out1[ROWS_IMG], ref1)
    print(f"noise refiner 1 (resident) rel L2 {err1:.3e}", flush=True)
    assert err1 <= BAR
    # the same resident boundary again: bit-identical
    rc, ev = model.noise_refiner_resident(bid, input_generation=1)
    assert rc == p.PROM_OK and ev.output_generation == 3
    again = np.zeros(T_IMG * W, np.float32)
    assert model.audit_final("noise", bid, 3, again)[0] == p.PROM_OK
    np.testing.assert_array_equal(again.reshape(T_IMG, W), out1)
    # stage audits of the resident block (reactor_api.h:776-797, 988-992, 1085-1093)
    cases = [(1, 3, "adaln_projection", None), (1, 14, "qkv", ROWS_IMG), (1, 20, "q_rope", ROWS_IMG),
             (1, 19, "k_norm", ROWS_IMG), (2, 1, "attention_aggregation", ROWS_IMG),
             (2, 3, "attention_residual", ROWS_IMG), (3, 1, "ffn_norm", ROWS_IMG),
             (3, 5, "ffn_gated_hidden", ROWS_IMG), (3, 7, "final_output", ROWS_IMG)]
    for fam, stage, name, rows in cases:
        n = mb_audit_elements(fam, stage)
        buf = np.zeros(n, np.float32)
        rc, ev = model.noise_refiner_resident(bid, 1, audit_family=fam, audit_stage=stage, audit=buf)
        assert rc == p.PROM_OK and ev.audit_valid == 1, (fam, stage, ev.detail_code)
        assert ev.output_valid == (1 if fam == 3 else 0)
        got = buf if rows is None else buf.reshape(T_IMG, -1)[rows]
        err = rel_l2(got, stages[name])
        assert err <= BAR, (name, err)
    assert model.destroy(bid) == p.PROM_OK


def mb_audit_elements(fam, stage):
    if fam == 1:
        return {3: 4 * W, 14: T_IMG * 3 * W, 2: 256}.get(stage, W if 4 <= stage <= 11 else T_IMG * W)
    if fam == 3 and stage in (3, 4, 5):
        return T_IMG * 10240
    return T_IMG * W


# ------------------------------------------------------------ ContextRefiner
def test_context_refiner_chain(model, weights, inputs):
    _, _, ctx = inputs
    coords = blocks.context_coordinates(T_CTX)
    rc, bid, ev = model.context_refiner_create(weights["cr0"])
    assert rc == p.PROM_OK, ev.detail_code
    assert ev.assembly_family == p.PROM_CONTEXT_REFINER_FAMILY and ev.weight_count == 11 and ev.binding_state == 1
    rc, ev = model.context_refiner0_execute(bid, ctx)
    assert rc == p.PROM_OK and ev.output_generation == 1
    out0 = np.zeros(T_CTX * W, np.float32)
    assert model.audit_final("context", bid, 1, out0)[0] == p.PROM_OK
    out0 = out0.reshape(T_CTX, W)
    err0 = rel_l2(out0, blocks.zimage_block_f64(ctx, coords, weights["cr0"], None))
    print(f"context refiner 0 rel L2 {err0:.3e}", flush=True)
    assert err0 <= BAR
    rc, ev = model.context_refiner_resident(bid, 1)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]  # still parameter set 1
    rc, ev = model.context_refiner_rebind(bid, weights["cr1"])
    assert rc == p.PROM_OK and ev.parameter_set == 2
    rc, ev = model.context_refiner_resident(bid, 1)
    assert rc == p.PROM_OK and ev.output_generation == 2
    out1 = np.zeros(T_CTX * W, np.float32)
    assert model.audit_final("context", bid, 2, out1)[0] == p.PROM_OK
    err1 = rel_l2(out1.reshape(T_CTX, W), blocks.zimage_block_f64(out0, coords, weights["cr1"], None))
    print(f"context refiner 1 (resident) rel L2 {err1:.3e}", flush=True)
    assert err1 <= BAR
    assert model.destroy(bid) == p.PROM_OK


def test_closed_form_refiners(model):
    """The NoiseRefiner and ContextRefiner on the closed-form weights of
    tests/closed_forms.py (scaled selections, period-4 channel classes,
    identical tokens): every row of the output is known from the stage
    recurrences there, and tests/test_oracle_closed_forms.py shows that each
    named misreading of the block wiring misses it by more than 0.2."""
    from tests import closed_forms as cf

    x = np.tile(cf.tile(cf.X, W), (T_IMG, 1)).astype(np.float32)
    t_bits = oracle.to_bf16(np.random.default_rng(9).standard_normal(256).astype(np.float32))
    print("closed-form noise refiner: create and upload", flush=True)
    rc, bid, ev = model.noise_refiner_create(cf.zimage_case(True))
    assert rc == p.PROM_OK, ev.detail_code
    rc, ev = model.noise_refiner_execute(bid, oracle.to_bf16(x), t_bits, parameter_set=1)
    assert rc == p.PROM_OK, ev.detail_code
    out = np.zeros(T_IMG * W, np.float32)
    assert model.audit_final("noise", bid, 1, out)[0] == p.PROM_OK
    err = rel_l2(out.reshape(T_IMG, W), cf.zimage_expected(T_IMG, True))
    print(f"closed-form noise refiner rel L2 {err:.3e} over all {T_IMG} rows", flush=True)
    assert err <= BAR
    assert model.destroy(bid) == p.PROM_OK
    rc, bid, ev = model.context_refiner_create(cf.zimage_case(False))
    assert rc == p.PROM_OK, ev.detail_code
    rc, ev = model.context_refiner0_execute(bid, x[:T_CTX])
    assert rc == p.PROM_OK, ev.detail_code
    out = np.zeros(T_CTX * W, np.float32)
    assert model.audit_final("context", bid, 1, out)[0] == p.PROM_OK
    err = rel_l2(out.reshape(T_CTX, W), cf.zimage_expected(T_CTX, False))
    print(f"closed-form context refiner rel L2 {err:.3e}", flush=True)
    assert err <= BAR
    assert model.destroy(bid) == p.PROM_OK


# ------------------------------------------------------------ session and MainTransformer
def check_stage_timing(ev):
    """The 13 per-stage GPU timings of a MainTransformer execution tile its
    compute interval (reactor_vulkan_model_block.c:3545-3562): stage s runs
    from boundary s+1 to s+2, ingress precedes the compute, the joint copy
    follows it."""
    ns = list(ev.main_stage_gpu_ns)
    begin, end = list(ev.main_stage_gpu_begin_tick), list(ev.main_stage_gpu_end_tick)
    # Stage 5 (0-based 4) is the fused flash attention; the softmax and P.V
    # stages that follow it close immediately, so only they may be empty.
    assert all(n > 0 for i, n in enumerate(ns) if i not in (5, 6)), ns
    assert all(n >= 0 for n in ns), ns
    assert [e - b for b, e in zip(begin, end)] == ns
    assert begin[1:] == end[:-1]
    assert begin[0] == ev.gpu_compute_begin_tick and end[-1] == ev.gpu_compute_end_tick
    assert sum(ns) == ev.gpu_compute_ns
    assert ev.gpu_total_begin_tick > 0
    assert ev.gpu_total_begin_tick + ev.gpu_ingress_transfer_ns == ev.gpu_compute_begin_tick
    assert ev.gpu_compute_end_tick + ev.gpu_joint_copy_ns == ev.gpu_total_end_tick
    assert ev.gpu_total_ns == ev.gpu_total_end_tick - ev.gpu_total_begin_tick
    print("main stages (us): " + " ".join(f"{n / 1e3:.1f}" for n in ns), flush=True)


def test_session_main_transformer_chain(model, weights, inputs):
    x_bits, t_bits, ctx = inputs
    cond = oracle.from_bf16(t_bits).astype(np.float64)
    rc, sid, sev = model.session_create()
    assert rc == p.PROM_OK and sid != 0 and sev.prepared_image_bytes == T_IMG * W * 4
    rc, sid2, sev = model.session_create()
    assert rc == p.PROM_ERROR  # one session per runtime

    # PreparedImage: NoiseRefiner 0 -> 1, then capture
    rc, bid, ev = model.noise_refiner_create(weights["nr0"])
    assert rc == p.PROM_OK
    assert model.noise_refiner_execute(bid, x_bits, t_bits)[0] == p.PROM_OK
    rc, sev = model.session_capture(sid, bid, 1)
    assert rc == p.PROM_ERROR and sev.detail_code == D["SESSION_STREAM_MISMATCH"]  # set 1 is not PreparedImage
    assert model.noise_refiner_rebind(bid, weights["nr1"])[0] == p.PROM_OK
    assert model.noise_refiner_resident(bid, 1)[0] == p.PROM_OK
    rc, sev = model.session_capture(sid, bid, 1)
    assert rc == p.PROM_ERROR and sev.detail_code == D["SESSION_STALE_STREAM"]  # generation 2 is current
    rc, sev = model.session_capture(sid, bid, 2)
    assert rc == p.PROM_OK and sev.prepared_image_generation == 1
    image = np.zeros(T_IMG * W, np.float32)
    assert model.audit_final("noise", bid, 2, image)[0] == p.PROM_OK
    assert model.destroy(bid) == p.PROM_OK

    # PreparedContext: ContextRefiner 0 -> 1, then capture
    rc, bid, ev = model.context_refiner_create(weights["cr0"])
    assert rc == p.PROM_OK
    assert model.context_refiner0_execute(bid, ctx)[0] == p.PROM_OK
    assert model.context_refiner_rebind(bid, weights["cr1"])[0] == p.PROM_OK
    assert model.context_refiner_resident(bid, 1)[0] == p.PROM_OK
    rc, sev = model.session_capture(sid, bid, 2)
    assert rc == p.PROM_OK and sev.prepared_context_generation == 1
    context = np.zeros(T_CTX * W, np.float32)
    assert model.audit_final("context", bid, 2, context)[0] == p.PROM_OK
    assert model.destroy(bid) == p.PROM_OK

    # MainTransformer layer 0 over JointWorking
    rc, mid, ev = model.main_transformer_create(0, weights["main0"])
    assert rc == p.PROM_OK, ev.detail_code
    assert ev.assembly_family == p.PROM_MAIN_TRANSFORMER_FAMILY and ev.parameter_set == 1
    rc, ev = model.main_transformer_execute(mid, sid, 0, t_bits, 1, 1, 1)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]  # nothing composed yet
    rc, sev = model.session_compose(sid, 1, 2)
    assert rc == p.PROM_ERROR and sev.detail_code == D["SESSION_STALE_STREAM"]
    rc, sev = model.session_compose(sid, 1, 1)
    assert rc == p.PROM_OK and sev.joint_generation == 1 and sev.composition_count == 1
    joint = np.concatenate((image.reshape(T_IMG, W), context.reshape(T_CTX, W)), axis=0)
    coords = blocks.joint_coordinates(32, 32, 32)
    rc, ev = model.main_transformer_execute(mid, sid, 0, t_bits, 1, 1, 1, chain=False)
    assert rc == p.PROM_OK and ev.output_generation == 1
    print(f"main transformer layer 0: gpu {ev.gpu_compute_ns / 1e6:.3f} ms", flush=True)
    check_stage_timing(ev)
    first_end = ev.gpu_total_end_tick
    assert model.session_evidence(sid)[1].joint_generation == 1  # audit mode leaves the joint alone
    out = np.zeros(T_JOINT * W, np.float32)
    assert model.audit_final("main", mid, 1, out)[0] == p.PROM_OK
    out = out.reshape(T_JOINT, W)
    ref = blocks.zimage_block_f64(joint, coords, weights["main0"], cond, rows=ROWS_JOINT)
    err = rel_l2(out[ROWS_JOINT], ref)
    print(f"main transformer 0 rel L2 {err:.3e}", flush=True)
    assert err <= BAR
    # the route the create decided: AUTO falls back to serial-canonical on 64-lane wavefronts
    sev = model.session_evidence(sid)[1]
    assert sev.requested_main_attention_route == p.PROM_MAIN_ATTENTION_ROUTE_AUTO
    assert sev.selected_main_attention_route == p.PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL
    assert sev.main_attention_fallback_reason == p.PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_SIZE
    assert sev.main_attention_shader_id == 41
    assert model.set_main_attention_route(sid, p.PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL)[0] == p.PROM_ERROR
    # the static audit re-runs layer 0 on the same JointWorking stream and the
    # timestep it last took; the arena holds that output, the rest is zeroed
    out_bytes = T_JOINT * W * 4
    arena = np.full(out_bytes + 4096, 0xCD, np.uint8)
    rc, ev = model.main_static_audit(mid, sid, 1, 1, 2, arena)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]
    rc, ev = model.main_static_audit(mid, sid, 1, 1, 1, arena)
    assert rc == p.PROM_OK and ev.output_generation == 2 and ev.audit_valid == 1 and ev.output_valid == 1
    np.testing.assert_array_equal(arena[:out_bytes].view(np.float32).reshape(T_JOINT, W), out)
    assert not arena[out_bytes:].any()
    assert model.session_evidence(sid)[1].joint_generation == 1
    # chain mode writes the output back into JointWorking (generation 2)
    rc, ev = model.main_transformer_execute(mid, sid, 0, t_bits, 1, 1, 1, chain=True)
    assert rc == p.PROM_OK and ev.output_generation == 3
    check_stage_timing(ev)
    assert ev.gpu_total_begin_tick > first_end and ev.gpu_joint_copy_ns > 0
    sev = model.session_evidence(sid)[1]
    assert sev.joint_generation == 2 and sev.active_block_id == mid
    chained = np.zeros(T_JOINT * W, np.float32)
    assert model.audit_final("main", mid, 3, chained)[0] == p.PROM_OK
    np.testing.assert_array_equal(chained.reshape(T_JOINT, W), out)
    rc, ev = model.main_transformer_execute(mid, sid, 0, t_bits, 1, 1, 1, chain=True)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]  # joint generation moved on
    # layer 1 is the only legal successor
    rc, ev = model.main_transformer_rebind(mid, 2, weights["nr1"])
    assert rc == p.PROM_ERROR and ev.detail_code == D["REBIND_FAILED"]
    rc, ev = model.main_transformer_rebind(mid, 1, weights["nr1"])
    assert rc == p.PROM_OK and ev.parameter_set == 2
    rc, ev = model.main_transformer_execute(mid, sid, 1, t_bits, 1, 1, 2, chain=True)
    assert rc == p.PROM_OK
    assert model.session_evidence(sid)[1].joint_generation == 3
    out2 = np.zeros(T_JOINT * W, np.float32)
    assert model.audit_final("main", mid, ev.output_generation, out2)[0] == p.PROM_OK
    ref2 = blocks.zimage_block_f64(out, coords, weights["nr1"], cond, rows=ROWS_JOINT)
    err2 = rel_l2(out2.reshape(T_JOINT, W)[ROWS_JOINT], ref2)
    print(f"main transformer 1 (chained) rel L2 {err2:.3e}", flush=True)
    assert err2 <= BAR
    assert model.destroy(mid) == p.PROM_OK
    assert model.session_destroy(sid) == p.PROM_OK
    assert model.session_destroy(sid) == p.PROM_ERROR


# ------------------------------------------------------------ compiled-model owner
def test_compiled_owner_drives_the_bridge_sequence(model, weights, inputs):
    """The call sequence of tools/prometheus_zimage_bridge/reactor_windows.go:805-1000
    (MINIMUM_MEMORY profile): one owner retargeted through NoiseRefiner 0/1,
    ContextRefiner 0/1 and MainTransformer layers, then a reset evaluation."""
    x_bits, t_bits, ctx = inputs
    cond = oracle.from_bf16(t_bits).astype(np.float64)
    rc, sid, sev = model.session_create(profile=1)  # MINIMUM_MEMORY
    assert rc == p.PROM_OK
    rc, oid, ev = model.owner_create(weights["nr0"])
    assert rc == p.PROM_OK and oid != 0, ev.detail_code
    sev = model.session_evidence(sid)[1]
    assert sev.selected_execution_profile == 1 and sev.profile_fallback_reason == 0
    # prefetch belongs to the PREFETCH profile only
    assert model.prefetch(sid, 1, weights["nr1"])[1].detail_code == D["REBIND_FAILED"]
    assert model.activate_prefetch(sid)[1].detail_code == D["REBIND_FAILED"]
    rc, ev = model.noise_refiner_execute(oid, x_bits, t_bits)
    assert rc == p.PROM_OK
    first_nr0 = np.zeros(T_IMG * W, np.float32)
    assert model.audit_final("noise", oid, ev.output_generation, first_nr0)[0] == p.PROM_OK
    # the position names the next block: ContextRefiner weights are refused here
    rc, ev = model.retarget(sid, 0, weights["cr0"], mb.CONTEXT_TENSORS)
    assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]
    rc, ev = model.retarget(sid, 1, weights["nr1"])
    assert rc == p.PROM_OK and ev.parameter_set == 2
    gen = ev.output_generation
    rc, ev = model.noise_refiner_resident(oid, gen)
    assert rc == p.PROM_OK
    rc, sev = model.session_capture(sid, oid, ev.output_generation)
    assert rc == p.PROM_OK and sev.prepared_image_generation == 1
    image = np.zeros(T_IMG * W, np.float32)
    assert model.audit_final("noise", oid, ev.output_generation, image)[0] == p.PROM_OK
    # ContextRefiner 0 -> 1 on the same owner
    rc, ev = model.retarget(sid, 0, weights["cr0"], mb.CONTEXT_TENSORS)
    assert rc == p.PROM_OK and ev.assembly_family == p.PROM_CONTEXT_REFINER_FAMILY and ev.weight_count == 11
    rc, ev = model.context_refiner0_execute(oid, ctx)
    assert rc == p.PROM_OK
    rc, ev = model.retarget(sid, 1, weights["cr1"], mb.CONTEXT_TENSORS)
    assert rc == p.PROM_OK
    rc, ev = model.context_refiner_resident(oid, ev.output_generation)
    assert rc == p.PROM_OK
    rc, sev = model.session_capture(sid, oid, ev.output_generation)
    assert rc == p.PROM_OK and sev.prepared_context_generation == 1
    context = np.zeros(T_CTX * W, np.float32)
    assert model.audit_final("context", oid, ev.output_generation, context)[0] == p.PROM_OK
    np.testing.assert_allclose(context.reshape(T_CTX, W)[:2],
                               blocks.zimage_block_f64(
                                   blocks.zimage_block_f64(ctx, blocks.context_coordinates(), weights["cr0"], None),
                                   blocks.context_coordinates(), weights["cr1"], None)[:2], rtol=0, atol=1e-3)
    rc, sev = model.session_compose(sid, 1, 1)
    assert rc == p.PROM_OK
    joint_gen = sev.joint_generation
    # MainTransformer layers 0 and 1 in chain mode
    for layer, name in ((0, "main0"), (1, "nr1")):
        rc, ev = model.retarget(sid, layer, weights[name])
        assert rc == p.PROM_OK and ev.parameter_set == layer + 1, (layer, ev.detail_code)
        rc, ev = model.main_transformer_execute(oid, sid, layer, t_bits, 1, 1, joint_gen, chain=True)
        assert rc == p.PROM_OK, (layer, ev.detail_code)
        joint_gen += 1
    out = np.zeros(T_JOINT * W, np.float32)
    assert model.audit_final("main", oid, ev.output_generation, out)[0] == p.PROM_OK
    joint = np.concatenate((image.reshape(T_IMG, W), context.reshape(T_CTX, W)), axis=0)
    coords = blocks.joint_coordinates(32, 32, 32)
    mid = blocks.zimage_block_f64(joint, coords, weights["main0"], cond)
    ref = blocks.zimage_block_f64(mid, coords, weights["nr1"], cond, rows=ROWS_JOINT)
    err = rel_l2(out.reshape(T_JOINT, W)[ROWS_JOINT], ref)
    print(f"owner chain: main layers 0..1 rel L2 {err:.3e}", flush=True)
    assert err <= BAR
    # a new evaluation starts again at NoiseRefiner 0 and reproduces it exactly
    rc, sev = model.evaluation_reset(sid)
    assert rc == p.PROM_OK and sev.joint_generation == joint_gen
    rc, ev = model.retarget(sid, 1, weights["nr1"])
    assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]
    rc, ev = model.retarget(sid, 0, weights["nr0"])
    assert rc == p.PROM_OK and ev.parameter_set == 1
    rc, ev = model.noise_refiner_execute(oid, x_bits, t_bits)
    assert rc == p.PROM_OK
    again = np.zeros(T_IMG * W, np.float32)
    assert model.audit_final("noise", oid, ev.output_generation, again)[0] == p.PROM_OK
    np.testing.assert_array_equal(again, first_nr0)
    assert model.destroy(oid) == p.PROM_OK
    assert model.session_destroy(sid) == p.PROM_OK


# ------------------------------------------------------------ PREFETCH profile
# Device bytes of one fp32 Z-Image weight set (13 slots, w1 and w3 sharing W13).
SET_BYTES = 4 * (15360 + 256 * 15360 + 128 + W * W + 128 + W * 3 * W + 2 * W + W * 2 * 10240 + 10240 * W + 2 * W)
CHAIN = [(1, "nr1", mb.ZIMAGE_TENSORS), (0, "cr0", mb.CONTEXT_TENSORS), (1, "cr1", mb.CONTEXT_TENSORS),
         (0, "main0", mb.ZIMAGE_TENSORS), (1, "nr1", mb.ZIMAGE_TENSORS)]


class Advance:
    """Moves the owner to CHAIN[i]: with prefetch, the upload starts on a
    second thread (the bridge's goroutine, reactor_windows.go:510-545) before
    the caller executes the current block and is activated afterwards;
    otherwise the owner is retargeted in place."""

    def __init__(self, model, sid, weights, prefetch):
        self.model, self.sid, self.weights, self.prefetch = model, sid, weights, prefetch
        self.thread, self.result, self.windows = None, None, []

    def start(self, i):
        if not self.prefetch:
            return
        local, name, names = CHAIN[i]

        def run():
            t0 = time.perf_counter()
            self.result = self.model.prefetch(self.sid, local, self.weights[name], names), time.perf_counter() - t0

        self.thread = threading.Thread(target=run)
        self.thread.start()

    def finish(self, i):
        local, name, names = CHAIN[i]
        if self.prefetch:
            self.thread.join(timeout=100)
            assert not self.thread.is_alive(), "prefetch did not return"
            (rc, ev), seconds = self.result
            assert rc == p.PROM_OK and ev.created == 1, (i, ev.detail_code)
            print(f"prefetch {name}: {seconds * 1e3:.1f} ms on its thread", flush=True)
            if i == 0:  # a prepared window is not begun again
                rc, ev = self.model.prefetch(self.sid, local, self.weights[name], names)
                assert rc == p.PROM_ERROR and ev.detail_code == D["REBIND_FAILED"]
            t0 = time.perf_counter()
            rc, ev = self.model.activate_prefetch(self.sid)
            self.windows.append(ev.active_weight_window)
        else:
            t0 = time.perf_counter()
            rc, ev = self.model.retarget(self.sid, local, self.weights[name], names)
        print(f"{'activate' if self.prefetch else 'retarget'} {name}: {(time.perf_counter() - t0) * 1e3:.1f} ms "
              "on the executing thread", flush=True)
        assert rc == p.PROM_OK, (i, ev.detail_code)
        assert ev.weight_count == len(names) and ev.output_valid == 0
        return ev


def owner_evaluation(model, sid, oid, weights, inputs, prefetch):
    """NoiseRefiner 0/1, ContextRefiner 0/1 and MainTransformer layers 0/1 on
    the owner, which is bound to NoiseRefiner 0 on entry; returns the prepared
    image, the prepared context and the final joint output."""
    x_bits, t_bits, ctx = inputs
    adv = Advance(model, sid, weights, prefetch)
    adv.start(0)
    rc, ev = model.noise_refiner_execute(oid, x_bits, t_bits)
    assert rc == p.PROM_OK, ev.detail_code
    gen = ev.output_generation
    adv.finish(0)
    adv.start(1)
    rc, ev = model.noise_refiner_resident(oid, gen)
    assert rc == p.PROM_OK, ev.detail_code
    rc, sev = model.session_capture(sid, oid, ev.output_generation)
    assert rc == p.PROM_OK
    image_gen = sev.prepared_image_generation
    image = np.zeros(T_IMG * W, np.float32)
    assert model.audit_final("noise", oid, ev.output_generation, image)[0] == p.PROM_OK
    adv.finish(1)
    assert model.session_evidence(sid)[1].active_block_id == oid
    adv.start(2)
    rc, ev = model.context_refiner0_execute(oid, ctx)
    assert rc == p.PROM_OK, ev.detail_code
    gen = ev.output_generation
    adv.finish(2)
    adv.start(3)
    rc, ev = model.context_refiner_resident(oid, gen)
    assert rc == p.PROM_OK, ev.detail_code
    rc, sev = model.session_capture(sid, oid, ev.output_generation)
    assert rc == p.PROM_OK
    context_gen = sev.prepared_context_generation
    context = np.zeros(T_CTX * W, np.float32)
    assert model.audit_final("context", oid, ev.output_generation, context)[0] == p.PROM_OK
    adv.finish(3)
    rc, sev = model.session_compose(sid, image_gen, context_gen)
    assert rc == p.PROM_OK
    joint_gen = sev.joint_generation
    adv.start(4)
    rc, ev = model.main_transformer_execute(oid, sid, 0, t_bits, image_gen, context_gen, joint_gen, chain=True)
    assert rc == p.PROM_OK, ev.detail_code
    ev_layer1 = adv.finish(4)
    assert ev_layer1.parameter_set == 2 and ev_layer1.assembly_family == p.PROM_MAIN_TRANSFORMER_FAMILY
    rc, ev = model.main_transformer_execute(oid, sid, 1, t_bits, image_gen, context_gen, joint_gen + 1, chain=True)
    assert rc == p.PROM_OK, ev.detail_code
    out = np.zeros(T_JOINT * W, np.float32)
    assert model.audit_final("main", oid, ev.output_generation, out)[0] == p.PROM_OK
    if prefetch:  # the two windows alternate at every activation
        assert adv.windows == [1, 0, 1, 0, 1]
    return image, context, out


def test_compiled_owner_prefetch_profile(model, weights, inputs):
    """The PREFETCH profile (reactor_vulkan_model_block.c:4364-4380, 4545-4715):
    every next block is uploaded into the owner's second window on another
    thread while the current block executes, then activated.  The evaluation
    equals the one the same session then runs by in-place retargets bit for
    bit, and its prepared image equals the binary64 NoiseRefiner 0 -> 1 chain."""
    x_bits, t_bits, ctx = inputs
    rc, sid, sev = model.session_create(profile=2)
    assert rc == p.PROM_OK
    rc, oid, ev = model.owner_create(weights["nr0"])
    assert rc == p.PROM_OK and oid != 0, ev.detail_code
    assert ev.persistent_bytes == 2 * SET_BYTES, (ev.persistent_bytes, SET_BYTES)
    sev = model.session_evidence(sid)[1]
    assert sev.selected_execution_profile == 2 and sev.profile_fallback_reason == 0
    # refusals before any transfer: nothing prepared, the wrong block, the wrong session
    assert model.activate_prefetch(sid)[1].detail_code == D["REBIND_FAILED"]
    assert model.prefetch(sid, 0, weights["nr1"])[1].detail_code == D["INVALID_REQUEST"]
    assert model.prefetch(sid, 1, weights["cr0"], mb.CONTEXT_TENSORS)[1].detail_code == D["INVALID_REQUEST"]
    assert model.prefetch(sid + 1, 1, weights["nr1"])[1].detail_code == D["REBIND_FAILED"]

    image_a, context_a, out_a = owner_evaluation(model, sid, oid, weights, inputs, prefetch=True)
    cond = oracle.from_bf16(t_bits).astype(np.float64)
    coords = blocks.image_coordinates(T_IMG)
    nr0 = blocks.zimage_block_f64(oracle.from_bf16(x_bits).astype(np.float64), coords, weights["nr0"], cond)
    ref = blocks.zimage_block_f64(nr0, coords, weights["nr1"], cond, rows=ROWS_IMG)
    err = rel_l2(image_a.reshape(T_IMG, W)[ROWS_IMG], ref)
    print(f"prefetched NoiseRefiner 0 -> 1 rel L2 {err:.3e}", flush=True)
    assert err <= BAR

    rc, sev = model.evaluation_reset(sid)
    assert rc == p.PROM_OK
    assert model.prefetch(sid, 0, weights["nr0"])[1].detail_code == D["INVALID_REQUEST"]  # position 0 is retargeted
    rc, ev = model.retarget(sid, 0, weights["nr0"])
    assert rc == p.PROM_OK
    image_b, context_b, out_b = owner_evaluation(model, sid, oid, weights, inputs, prefetch=False)
    np.testing.assert_array_equal(image_a, image_b)
    np.testing.assert_array_equal(context_a, context_b)
    np.testing.assert_array_equal(out_a, out_b)

    # a reset drops a prepared window
    rc, sev = model.evaluation_reset(sid)
    assert rc == p.PROM_OK
    assert model.retarget(sid, 0, weights["nr0"])[0] == p.PROM_OK
    assert model.prefetch(sid, 1, weights["nr1"])[0] == p.PROM_OK
    assert model.evaluation_reset(sid)[0] == p.PROM_OK
    assert model.retarget(sid, 0, weights["nr0"])[0] == p.PROM_OK
    assert model.activate_prefetch(sid)[1].detail_code == D["REBIND_FAILED"]
    # destroying the owner waits for a transfer in flight on another thread
    box = {}
    th = threading.Thread(target=lambda: box.update(r=model.prefetch(sid, 1, weights["nr1"])))
    th.start()
    assert model.destroy(oid) == p.PROM_OK
    th.join(timeout=100)
    assert not th.is_alive()
    rc, ev = box["r"]
    assert (rc, ev.detail_code) in ((p.PROM_OK, 0), (p.PROM_ERROR, D["REBIND_FAILED"])), (rc, ev.detail_code)
    assert model.session_destroy(sid) == p.PROM_OK


# ------------------------------------------------------------ stage-split NoiseRefiner (M1B, M1C, M1D)
ROWS_SPLIT = np.array([0, 1, 31, 32, 341, 512, 682, 1000, 1023])
ARENA = p.PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES
SCHEDULE = json.loads((Path(__file__).resolve().parent / "golden" / "zimage_audit_schedule.json").read_text())


def close(got, ref, tol):
    return abs(float(got) - float(ref)) <= tol * max(1.0, abs(float(ref)))


def logits(q_rope, k_rope_all, t_index, h, hd=128):
    """Scaled scores and probabilities of one (token, head) row in binary64."""
    s = np.asarray(k_rope_all, np.float64)[:, h * hd:(h + 1) * hd] @ np.asarray(q_rope, np.float64)[
        t_index, h * hd:(h + 1) * hd] / np.sqrt(hd)
    e = np.exp(s - s.max())
    return s, e / e.sum()


def check_image_witness(w, q_rope, k_rope_all, v_all, aggregation, t_rows):
    """The NoiseRefiner witness (nr0_attention_streaming.sdslv:24-116): per
    selected row, keys 0, 1, 512, 1023 as (raw, scaled, shifted, exp,
    probability), then max, sum, row sum, p0 * v0 and the head output."""
    T = 1024
    for base, (t, h) in ((0, (0, 0)), (32, (T - 1, 29))):
        ti = int(np.where(t_rows == t)[0][0])
        s, prob = logits(q_rope, k_rope_all, ti, h)
        assert w[base + 30] == 1.0 and abs(w[base + 22] - 1.0) <= 2e-5, base
        assert close(w[base + 20], s.max(), 1e-4)
        for i, key in enumerate((0, 1, T // 2, T - 1)):
            assert close(w[base + 5 * i + 1], s[key], 1e-4), (base, key)
            assert close(w[base + 5 * i], s[key] * np.sqrt(128.0), 1e-4), (base, key)
            assert close(w[base + 5 * i + 2], s[key] - s.max(), 1e-4), (base, key)
            assert abs(w[base + 5 * i + 4] - prob[key]) <= 2e-6, (base, key)
            assert close(w[base + 5 * i + 3], prob[key] * w[base + 21], 1e-4), (base, key)
        assert close(w[base + 23], prob[0] * float(v_all[0, h * 128]), 1e-4)
        assert close(w[base + 24], aggregation[ti, h * 128], 1e-4)


def test_stage_split_noise_refiner(model, weights, inputs):
    """M1B -> M1C -> M1D on the resident workspace (reactor_vulkan_model_block.c:
    1955-2199) against the binary64 block, the witness against the same
    oracle, and the split chain against the whole block bit for bit."""
    x_bits, t_bits, _ = inputs
    x = oracle.from_bf16(x_bits).astype(np.float64)
    cond = oracle.from_bf16(t_bits).astype(np.float64)
    stages = {}
    blocks.zimage_block_f64(x, blocks.image_coordinates(T_IMG), weights["nr0"], cond, rows=ROWS_SPLIT, stages=stages)
    out = np.zeros(T_IMG * W, np.float32)
    # a block declaring a 256 KiB audit refuses large stage audits and M1C
    rc, bid, ev = model.noise_refiner_create(weights["nr0"])
    assert rc == p.PROM_OK
    rc, ev = model.execute_m1b(bid, x_bits, t_bits, audit_stage=14, audit=np.zeros(T_IMG * 3 * W, np.float32))
    assert rc == p.PROM_ERROR and ev.detail_code == D["AUDIT_FAILED"]
    rc, ev = model.execute_m1b(bid, x_bits[:-1], t_bits)
    assert rc == p.PROM_ERROR and ev.detail_code == D["INGRESS_INPUT_SIZE_MISMATCH"]
    rc, ev = model.execute_m1b(bid, x_bits, t_bits[:-1])
    assert rc == p.PROM_ERROR and ev.detail_code == D["INGRESS_TIMESTEP_SIZE_MISMATCH"]
    rc, ev = model.execute_m1b(bid, x_bits, t_bits)
    assert rc == p.PROM_OK and ev.output_valid == 1 and ev.audit_valid == 0
    rc, ev2 = model.execute_m1c(bid, ev.replay_identity, out)
    assert rc == p.PROM_ERROR and ev2.detail_code == D["STALE_OUTPUT"]
    assert model.destroy(bid) == p.PROM_OK

    print("stage split: create with the lock's audit arena", flush=True)
    rc, bid, ev = model.noise_refiner_create(weights["nr0"], audit_bytes=ARENA)
    assert rc == p.PROM_OK
    allocs = ev.cold_buffer_allocation_count
    for stage, name, width in ((14, "qkv", 3 * W), (12, "attention_norm", W), (13, "attention_modulated", W),
                               (20, "q_rope", W), (19, "k_norm", W), (3, "adaln_projection", None)):
        buf = np.zeros(mb_audit_elements(1, stage), np.float32)
        rc, ev = model.execute_m1b(bid, x_bits, t_bits, audit_stage=stage, audit=buf)
        assert rc == p.PROM_OK and ev.audit_valid == 1 and ev.output_valid == 1, (stage, ev.detail_code)
        got = buf if width is None else buf.reshape(T_IMG, width)[ROWS_SPLIT]
        err = rel_l2(got, stages[name])
        assert err <= BAR, (name, err)
    rc, ev = model.execute_m1b(bid, x_bits, t_bits)
    prefix = ev.replay_identity
    rc, ev = model.execute_m1b(bid, x_bits, t_bits)
    assert rc == p.PROM_OK and ev.replay_identity == prefix  # identical requests replay identically
    rc, ev = model.execute_m1c(bid, prefix ^ 1, out)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]
    transient = np.zeros(p.PROM_MODEL_BLOCK_M1C_TRANSIENT_AUDIT_FLOATS, np.float32)
    for stage, name in ((1, "attention_aggregation"), (2, "attention_projection"), (3, "attention_residual")):
        transient[:] = 0
        rc, ev = model.execute_m1c(bid, prefix, out, audit_stage=stage, transient=transient)
        assert rc == p.PROM_OK and ev.output_valid == 1, (stage, ev.detail_code)
        err = rel_l2(out.reshape(T_IMG, W)[ROWS_SPLIT], stages[name])
        print(f"M1C {name} rel L2 {err:.3e}", flush=True)
        assert err <= BAR
        check_image_witness(transient, stages["q_rope"], stages["k_rope_all"], stages["v_all"],
                            stages["attention_aggregation"], ROWS_SPLIT)
    m1c = ev.replay_identity
    final = np.zeros(T_IMG * W, np.float32)
    rc, ev = model.execute_m1d(bid, m1c, final, audit_stage=7)
    assert rc == p.PROM_OK and ev.output_valid == 1 and ev.audit_valid == 1
    err = rel_l2(final.reshape(T_IMG, W)[ROWS_SPLIT], stages["final_output"])
    print(f"M1D final_output rel L2 {err:.3e}", flush=True)
    assert err <= BAR
    rc, ev = model.execute_m1d(bid, m1c, final, audit_stage=7)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]  # the chain moved on
    rc, ev = model.execute_m1c(bid, prefix, out, audit_stage=3)
    assert rc == p.PROM_OK and ev.replay_identity == m1c
    hidden = np.zeros(T_IMG * 10240, np.float32)
    rc, ev = model.execute_m1d(bid, m1c, hidden, audit_stage=5)
    assert rc == p.PROM_OK
    assert rel_l2(hidden.reshape(T_IMG, 10240)[ROWS_SPLIT], stages["ffn_gated_hidden"]) <= BAR
    # the whole block on the same ingress reproduces the split chain bit for bit
    rc, ev = model.noise_refiner_execute(bid, x_bits, t_bits)
    assert rc == p.PROM_OK and ev.cold_buffer_allocation_count == allocs
    whole = np.zeros(T_IMG * W, np.float32)
    assert model.audit_final("noise", bid, ev.output_generation, whole)[0] == p.PROM_OK
    np.testing.assert_array_equal(whole, final)
    rc, ev = model.execute_m1c(bid, prefix, out)  # a full execution replaced the M1B state
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]
    assert model.destroy(bid) == p.PROM_OK


# ------------------------------------------------------------ static audits
def check_record(rec, entry, data, generation):
    """One 256-byte summary record (nr0_persistent_audit_summary.sdslv:56-217)
    against the fp32 stage it summarises: counts, keys and key values exact,
    min and max exact, the sum of squares and RMS to fp32 summation accuracy."""
    data = np.asarray(data, np.float32).ravel()
    keys = entry["keys"]
    fl = rec.view(np.float32)
    assert rec[0] == entry["stage"] and rec[1] == generation and rec[2] == entry["count"] == data.size, entry["stage"]
    assert rec[3] == 1 and rec[4] == 0 and rec[5] == 0 and rec[6] == data.size and rec[7] == len(keys)
    assert fl[8] == data.min() and fl[9] == data.max(), entry["stage"]
    ss = float(np.sum(np.square(data, dtype=np.float64)))
    assert abs(fl[10] - ss) <= 2e-4 * ss, (entry["stage"], fl[10], ss)
    assert abs(fl[11] - np.sqrt(ss / data.size)) <= 1e-4 * np.sqrt(ss / data.size)
    assert rec[12] == 1 and rec[13] == 0 and rec[14] == 0 and rec[15] == 0
    for i, k in enumerate(keys):
        assert rec[16 + 2 * i] == k and fl[17 + 2 * i] == data[k], (entry["stage"], k)
    assert not rec[16 + 2 * len(keys):].any()


# NoiseRefiner schedule stage -> (audit family, stage) of the resident stage audits
NOISE_AUDIT_SOURCE = {1: (1, 3), 2: (1, 4), 3: (1, 5), 4: (1, 6), 5: (1, 7), 6: (1, 8), 7: (1, 9), 8: (1, 10),
                      9: (1, 11), 10: (1, 12), 11: (1, 13), 12: (1, 14), 13: (1, 15), 14: (1, 16), 15: (1, 17),
                      16: (1, 18), 17: (1, 19), 18: (1, 20), 19: (1, 21), 20: (2, 1), 21: (2, 2), 22: (2, 3),
                      23: (3, 1), 24: (3, 2), 25: (3, 3), 26: (3, 4), 27: (3, 5), 28: (3, 6), 29: (3, 7)}


def test_noise_refiner_static_audit(model, weights, inputs):
    """reactor_vulkan_model_block.c:3212-3272: one resident NoiseRefiner 1
    execution fills the lock's arena; every record is checked against the
    same stage fetched through the resident stage audits (a re-run of the
    same boundary, bit-identical), the witness against those stages."""
    x_bits, t_bits, _ = inputs
    sched = SCHEDULE["noise"]
    rc, bid, ev = model.noise_refiner_create(weights["nr0"], audit_bytes=ARENA)
    assert rc == p.PROM_OK
    assert model.noise_refiner_execute(bid, x_bits, t_bits)[0] == p.PROM_OK
    arena = np.full(ARENA, 0xCD, np.uint8)
    rc, ev = model.static_audit("noise", bid, 1, arena)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]  # parameter set 0
    assert model.noise_refiner_rebind(bid, weights["nr1"])[0] == p.PROM_OK
    rc, ev = model.static_audit("noise", bid, 2, arena)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]
    print("noise refiner static audit", flush=True)
    rc, ev = model.static_audit("noise", bid, 1, arena)
    assert rc == p.PROM_OK and ev.output_generation == 2 and ev.audit_valid == 1 and ev.output_valid == 1
    req = sched["required_bytes"]
    assert not arena[req:].any()
    words, floats = arena[:req].view(np.uint32), arena[:req].view(np.float32)
    out = np.zeros(T_IMG * W, np.float32)  # the published output is the resident one of generation 2
    assert model.audit_final("noise", bid, 2, out)[0] == p.PROM_OK
    fetched = {}
    for entry in sched["stages"]:
        fam, stage = NOISE_AUDIT_SOURCE[entry["stage"]]
        buf = np.zeros(mb_audit_elements(fam, stage), np.float32)
        rc, ev = model.noise_refiner_resident(bid, 1, audit_family=fam, audit_stage=stage, audit=buf)
        assert rc == p.PROM_OK, (entry["stage"], ev.detail_code)
        d0 = entry["dest"] // 4
        if entry["policy"] == 1:
            np.testing.assert_array_equal(floats[d0:d0 + entry["count"]], buf[:entry["count"]])
        else:
            check_record(words[d0:d0 + 64], entry, buf, generation=2)
        if entry["stage"] in (18, 19, 20):
            fetched[entry["stage"]] = buf.reshape(T_IMG, W)
        if entry["stage"] == 15:
            fetched["v"] = buf.reshape(T_IMG, W)
        if entry["stage"] == 29:
            np.testing.assert_array_equal(buf, out)  # the same boundary re-run: bit-identical
    w0 = sched["witness_offset"] // 4
    check_image_witness(floats[w0:w0 + 64], fetched[18], fetched[19], fetched["v"], fetched[20], np.arange(T_IMG))
    generation = model.evidence(bid)[1].output_generation
    rc, ev = model.static_audit("noise", bid, 1, arena)  # the same boundary again
    assert rc == p.PROM_OK and ev.output_generation == generation + 1
    assert model.destroy(bid) == p.PROM_OK


CONTEXT_STAGE_NAMES = {2: "attention_norm", 3: "qkv", 4: "q_norm", 5: "k_norm", 6: "q_rope", 7: "k_rope",
                       8: "attention_aggregation", 9: "attention_projection", 10: "attention_residual",
                       11: "ffn_modulated", 12: "w1", 13: "w3", 14: "ffn_gated_hidden", 15: "w2", 16: "final_output"}


def test_context_refiner_static_audit(model, weights, inputs):
    """reactor_vulkan_model_block.c:2671-2735 on parameter set 0: the arena's
    records against the binary64 ContextRefiner (32 tokens, every row)."""
    _, _, ctx = inputs
    sched = SCHEDULE["context"]
    stages = {}
    ref = blocks.zimage_block_f64(ctx, blocks.context_coordinates(T_CTX), weights["cr0"], None, stages=stages)
    stages["input"] = ctx
    rc, bid, ev = model.context_refiner_create(weights["cr0"])
    assert rc == p.PROM_OK
    assert model.context_refiner0_execute(bid, ctx)[0] == p.PROM_OK
    cap = p.PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_ARENA_BYTES + 512
    arena = np.full(cap, 0xCD, np.uint8)
    rc, ev = model.static_audit("context", bid, 2, arena)
    assert rc == p.PROM_ERROR and ev.detail_code == D["STALE_OUTPUT"]
    rc, ev = model.static_audit("context", bid, 1, arena)
    assert rc == p.PROM_OK and ev.output_generation == 2 and ev.audit_valid == 1
    req = sched["required_bytes"]
    assert not arena[req:].any()  # the whole capacity past the records is cleared
    words, floats = arena[:req].view(np.uint32), arena[:req].view(np.float32)
    for entry in sched["stages"]:
        r = stages[CONTEXT_STAGE_NAMES.get(entry["stage"], "input")]
        r = np.asarray(r, np.float64).ravel()
        rec = words[entry["dest"] // 4:entry["dest"] // 4 + 64]
        fl = rec.view(np.float32)
        scale = np.abs(r).max()
        assert rec[0] == entry["stage"] and rec[1] == 2 and rec[2] == entry["count"] == r.size
        assert rec[3] == 1 and rec[6] == r.size and rec[7] == len(entry["keys"]) and rec[12] == 1 and rec[13] == 0
        assert abs(fl[8] - r.min()) <= 1e-4 * scale and abs(fl[9] - r.max()) <= 1e-4 * scale, entry["stage"]
        ss = float(np.sum(r * r))
        assert abs(fl[10] - ss) <= 2e-4 * ss and abs(fl[11] - np.sqrt(ss / r.size)) <= 1e-4 * np.sqrt(ss / r.size)
        for i, k in enumerate(entry["keys"]):
            assert rec[16 + 2 * i] == k and abs(fl[17 + 2 * i] - r[k]) <= 1e-4 * scale, (entry["stage"], k)
    # the witness (context_refiner_attention_streaming.sdslv:44-73): key 0 of
    # (token 0, head 0) and (token 31, head 29)
    w = floats[sched["witness_offset"] // 4:sched["witness_offset"] // 4 + 64]
    for base, (t, h) in ((0, (0, 0)), (32, (T_CTX - 1, 29))):
        s, prob = logits(stages["q_rope"], stages["k_rope_all"], t, h)
        assert w[base + 30] == 1.0 and abs(w[base + 4] - 1.0) <= 2e-5
        assert close(w[base + 1], s[0], 1e-4) and close(w[base], s[0] * np.sqrt(128.0), 1e-4)
        assert close(w[base + 2], s[0] - s.max(), 1e-4) and abs(w[base + 3] - prob[0]) <= 2e-6
    out = np.zeros(T_CTX * W, np.float32)
    assert model.audit_final("context", bid, 2, out)[0] == p.PROM_OK
    assert rel_l2(out.reshape(T_CTX, W), ref) <= BAR
    assert model.destroy(bid) == p.PROM_OK


# ------------------------------------------------------------ main attention route
def test_main_attention_route(model, weights):
    """reactor_sgemm.cpp:1479-1516 and reactor_vulkan_model_block.c:2419-2430,
    4381-4408, 4229-4251 on 64-lane wavefronts."""
    rc, sid, sev = model.session_create(route=p.PROM_MAIN_ATTENTION_ROUTE_SUBGROUP_OWNED32)
    assert rc == p.PROM_OK
    assert sev.selected_main_attention_route == p.PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL
    assert sev.main_attention_shader_id == 41 and sev.main_attention_fallback_reason == 0
    rc, mid, ev = model.main_transformer_create(0, weights["main0"])
    assert rc == p.PROM_ERROR and ev.detail_code == D["RESOURCE_CREATE_FAILED"]
    rc, oid, ev = model.owner_create(weights["nr0"])
    assert rc == p.PROM_ERROR and ev.detail_code == D["MAIN_ATTENTION_ROUTE_REJECTED"]
    sev = model.session_evidence(sid)[1]
    assert sev.selected_main_attention_route == 0 and sev.main_attention_shader_id == 0
    assert sev.main_attention_fallback_reason == p.PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_SIZE
    rc, sev = model.set_main_attention_route(sid, p.PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL)
    assert rc == p.PROM_OK and sev.requested_main_attention_route == p.PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL
    assert sev.selected_main_attention_route == p.PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL
    rc, mid, ev = model.main_transformer_create(0, weights["main0"])
    assert rc == p.PROM_OK, ev.detail_code
    sev = model.session_evidence(sid)[1]
    assert sev.main_attention_fallback_reason == 0 and sev.main_attention_shader_id == 41
    assert model.set_main_attention_route(sid, p.PROM_MAIN_ATTENTION_ROUTE_AUTO)[0] == p.PROM_ERROR
    assert model.destroy(mid) == p.PROM_OK
    rc, sev = model.set_main_attention_route(sid, p.PROM_MAIN_ATTENTION_ROUTE_AUTO)
    assert rc == p.PROM_OK
    rc, oid, ev = model.owner_create(weights["nr0"])
    assert rc == p.PROM_OK
    sev = model.session_evidence(sid)[1]
    assert sev.selected_main_attention_route == p.PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL
    assert sev.main_attention_fallback_reason == p.PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_SIZE
    assert model.destroy(oid) == p.PROM_OK
    assert model.session_destroy(sid) == p.PROM_OK
