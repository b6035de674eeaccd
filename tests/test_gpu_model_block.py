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


# ------------------------------------------------------------ session and MainTransformer
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
    assert model.session_evidence(sid)[1].joint_generation == 1  # audit mode leaves the joint alone
    out = np.zeros(T_JOINT * W, np.float32)
    assert model.audit_final("main", mid, 1, out)[0] == p.PROM_OK
    out = out.reshape(T_JOINT, W)
    ref = blocks.zimage_block_f64(joint, coords, weights["main0"], cond, rows=ROWS_JOINT)
    err = rel_l2(out[ROWS_JOINT], ref)
    print(f"main transformer 0 rel L2 {err:.3e}", flush=True)
    assert err <= BAR
    # chain mode writes the output back into JointWorking (generation 2)
    rc, ev = model.main_transformer_execute(mid, sid, 0, t_bits, 1, 1, 1, chain=True)
    assert rc == p.PROM_OK and ev.output_generation == 2
    sev = model.session_evidence(sid)[1]
    assert sev.joint_generation == 2 and sev.active_block_id == mid
    chained = np.zeros(T_JOINT * W, np.float32)
    assert model.audit_final("main", mid, 2, chained)[0] == p.PROM_OK
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
    rc, sid, sev = model.session_create(profile=2)  # PREFETCH requested
    assert rc == p.PROM_OK
    rc, oid, ev = model.owner_create(weights["nr0"])
    assert rc == p.PROM_OK and oid != 0, ev.detail_code
    sev = model.session_evidence(sid)[1]
    assert sev.selected_execution_profile == 1 and sev.profile_fallback_reason == 1
    assert model.prefetch(sid, 1, weights["nr1"])[1].detail_code == D["REBIND_FAILED"]
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
