"""CPU checks of the resident model-block ABI: the closed create-request
validation (reactor_vulkan_model_block.c:393-493), not-found handling, the
lock-bound facades and the session's argument checks.  No device is needed:
every case below is decided before any allocation, and a valid request on a
device-less runtime reports RESOURCE_CREATE_FAILED."""
import ctypes

import pytest

from oct_amd import model_block as mb
from oct_amd import prometheus as p

D = p.PROM_MODEL_BLOCK_DETAIL
NOISE_BYTES = (30720, 7864320, 256, 29491200, 256, 88473600, 7680, 7680, 78643200, 78643200, 78643200, 7680, 7680)
CONTEXT_BYTES = NOISE_BYTES[2:]


class FakeUploads:
    """Upload descriptors whose byte pointers are never read (creation fails first)."""

    def __init__(self, sizes, content_base=0x200):
        self._anchor = (ctypes.c_uint8 * 16)()
        self.items = (p.PrometheusModelBlockWeightUpload * len(sizes))()
        for i, n in enumerate(sizes):
            self.items[i].binding_index = i
            self.items[i].bytes = ctypes.addressof(self._anchor)
            self.items[i].byte_count = n
            self.items[i].content_identity = content_base + i
            self.items[i].layout_identity = 0x300 + i

    def __len__(self):
        return len(self.items)

    def pointer(self):
        return ctypes.cast(self.items, ctypes.POINTER(p.PrometheusModelBlockWeightUpload))


@pytest.fixture
def model():
    rt = p.NativeRuntime(test_flags=0)
    yield mb.ResidentModel(rt)
    rt.close()


def proof_request(**kw):
    ups = FakeUploads([64] * 13)
    args = dict(shader_id=23, external_input_bytes=4096, external_output_bytes=4096, audit_bytes=256,
                memory_ceiling=1 << 20)
    args.update(kw)
    return mb.create_request(ups, **args)


def noise_request(**kw):
    ups = FakeUploads(NOISE_BYTES, 0x5A00)
    args = dict(shader_id=24, family=1, parameter_set=1, aggregate=p.NOISE_REFINER_AGGREGATES[0],
                external_input_bytes=1024 * 3840 * 2, audit_bytes=65536 * 4, memory_ceiling=512 << 20)
    args.update(kw)
    return mb.create_request(ups, **args)


def device_less_code():
    """What a valid request returns here: no device means no resources."""
    return D["RESOURCE_CREATE_FAILED"]


def test_valid_requests_reach_resource_creation(model):
    for req in (proof_request(), noise_request(), noise_request(parameter_set=2,
                                                                aggregate=p.NOISE_REFINER_AGGREGATES[1])):
        rc, bid, ev = model.create(req)
        expect_ok = model.rt.available
        assert (rc == p.PROM_OK) == expect_ok
        if not expect_ok:
            assert bid == 0 and ev.detail_code == device_less_code() and ev.created == 0
        else:
            model.destroy(bid)


def _set(req, **fields):
    for k, v in fields.items():
        setattr(req, k, v)
    return req


@pytest.mark.parametrize("mutate", [
    lambda r: _set(r, struct_size=r.struct_size - 8),
    lambda r: _set(r, model_contract_identity=0),
    lambda r: _set(r, weight_identity=0),
    lambda r: _set(r, shader_portfolio_identity=0),
    lambda r: _set(r, precision_policy_identity=0),
    lambda r: _set(r, capability_route_identity=0),
    lambda r: _set(r, memory_ceiling_bytes=0),
    lambda r: _set(r, shader_id=22),
    lambda r: _set(r, weight_count=0),
    lambda r: _set(r, weight_count=14),
    lambda r: _set(r, audit_bytes=0),
    lambda r: _set(r, audit_bytes=6),
    lambda r: _set(r, external_input_bytes=4097),
    lambda r: _set(r, external_output_bytes=0),       # shader 23 needs an output
    lambda r: _set(r, external_input_bytes=0),
    lambda r: _set(r, step_count=6),
    lambda r: (r.steps.__setitem__(3, 5), r)[1],      # the seven steps in their fixed order
    lambda r: _set(r, parameter_set=1),                # family 0 carries no parameter set
    lambda r: _set(r, parameter_set_aggregate_identity=7),
    lambda r: _set(r, assembly_family=4),
    lambda r: _set(r, memory_ceiling_bytes=13 * 64 * 2 + 4096 * 4 + 256 * 2 - 4),  # below the plan total
    lambda r: (setattr(r.weights[2], "content_identity", 0), r)[1],
    lambda r: (setattr(r.weights[0], "byte_count", 0), r)[1],
])
def test_malformed_program_is_invalid_request(model, mutate):
    """reactor_vulkan_model_block.c:393-493 and Marionette FACT
    PrometheusResidentModelBlockRejectsMalformedProgramAndPipelineFault."""
    rc, bid, ev = model.create(mutate(proof_request()))
    assert rc == p.PROM_ERROR and bid == 0
    assert ev.detail_code == D["INVALID_REQUEST"] and ev.struct_size == ctypes.sizeof(ev)


@pytest.mark.parametrize("mutate", [
    lambda r: _set(r, parameter_set=3),
    lambda r: _set(r, parameter_set_aggregate_identity=p.NOISE_REFINER_AGGREGATES[1]),  # set 1 with set 2's identity
    lambda r: _set(r, shader_id=23),
    lambda r: _set(r, external_input_bytes=1024 * 3840 * 4),   # the BF16 ingress size is fixed
    lambda r: _set(r, external_output_bytes=4),
    lambda r: _set(r, audit_bytes=p.PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES + 4),
    lambda r: _set(r, weight_count=12),
    lambda r: (setattr(r.weights[5], "byte_count", 88473600 - 2), r)[1],  # the lock's tensor sizes
    lambda r: _set(r, memory_ceiling_bytes=sum(NOISE_BYTES) + (128 << 20) - 1),
])
def test_noise_refiner_create_is_lock_bound(model, mutate):
    rc, bid, ev = model.create(mutate(noise_request()))
    assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]


def test_unknown_block_is_not_found(model):
    ups = FakeUploads([64] * 13)
    rc, ev = model.upload(99, ups)
    assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]
    rc, ev = model.evidence(99)
    assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]
    assert model.destroy(99) == p.PROM_ERROR
    rc, ev = model.noise_refiner_resident(99, input_generation=1)
    assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]
    out = __import__("numpy").zeros(1056 * 3840, dtype="float32")
    for kind in ("noise", "context", "main"):
        rc, ev = model.audit_final(kind, 99, 1, out)
        assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]


def test_execute_request_shape_checks(model):
    import numpy as np

    x = np.zeros(1024, np.float32)
    y = np.zeros(1024, np.float32)
    for patch in (lambda r: setattr(r, "struct_size", 8), lambda r: setattr(r, "input_identity", 0),
                  lambda r: setattr(r, "audit_enabled", 2), lambda r: setattr(r, "element_count", 0),
                  lambda r: setattr(r, "input", None)):
        rc, ev = model.execute(1, x, y, request_patch=patch)
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]


def test_noise_refiner_execute_requires_the_fixed_payload(model):
    import numpy as np

    xb = np.zeros(1024 * 3840, np.uint16)
    tb = np.zeros(256, np.uint16)
    for patch in (lambda r: setattr(r, "model_input_bytes", r.model_input_bytes - 2),
                  lambda r: setattr(r, "timestep_bytes", 510), lambda r: setattr(r, "input_identity", 0),
                  lambda r: setattr(r, "timestep_identity", 0), lambda r: setattr(r, "output_identity", 0),
                  lambda r: setattr(r, "audit_enabled", 1)):
        rc, ev = model.noise_refiner_execute(1, xb, tb, request_patch=patch)
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]
    # a well-formed request for a block that does not exist: parameter-set mismatch (facade check)
    rc, ev = model.noise_refiner_execute(1, xb, tb)
    assert rc == p.PROM_ERROR and ev.detail_code == D["PARAMETER_SET_MISMATCH"]


def test_resident_audit_request_checks(model):
    import numpy as np

    audit = np.zeros(16, np.float32)
    # unknown family, stage out of range, capacity below the stage's element count
    r_cases = [(1, 0, audit), (4, 1, audit), (1, 22, audit), (2, 4, audit), (3, 8, audit), (1, 3, audit)]
    for fam, stage, buf in r_cases:
        rc, ev = model.noise_refiner_resident(1, 1, audit_family=fam, audit_stage=stage, audit=buf)
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"], (fam, stage)
    rc, ev = model.noise_refiner_resident(1, 0)
    assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]


def test_lock_bound_facades_validate_before_creating(model):
    ctx_ups = FakeUploads(CONTEXT_BYTES)
    for count, lock, local in ((10, p.PROM_ZIMAGE_TURBO_LOCK_ID, 0), (11, 0x1234, 0), (11, p.PROM_ZIMAGE_TURBO_LOCK_ID, 1)):
        r = model._lock_request(ctx_ups, local, lock)
        r.upload_count = count
        ev = p.PrometheusModelBlockEvidence()
        bid = ctypes.c_uint64(7)
        rc = model.lib.prometheus_reactor_runtime_context_refiner_create(model.h, ctypes.byref(r), ctypes.byref(bid),
                                                                         ctypes.byref(ev))
        assert rc == p.PROM_ERROR and bid.value == 0 and ev.detail_code == D["INVALID_REQUEST"]
    # a valid ContextRefiner payload on a device-less runtime: no resources
    r = model._lock_request(ctx_ups, 0, p.PROM_ZIMAGE_TURBO_LOCK_ID)
    ev = p.PrometheusModelBlockEvidence()
    bid = ctypes.c_uint64(0)
    rc = model.lib.prometheus_reactor_runtime_context_refiner_create(model.h, ctypes.byref(r), ctypes.byref(bid),
                                                                     ctypes.byref(ev))
    if not model.rt.available:
        assert rc == p.PROM_ERROR and ev.detail_code == D["RESOURCE_CREATE_FAILED"]
    # MainTransformer: layer ids are 0..29 and a session of the lock must exist
    main_ups = FakeUploads(NOISE_BYTES)
    for local in (30, 31):
        r = model._lock_request(main_ups, local, p.PROM_ZIMAGE_TURBO_LOCK_ID)
        rc = model.lib.prometheus_reactor_runtime_main_transformer_create(model.h, ctypes.byref(r), ctypes.byref(bid),
                                                                          ctypes.byref(ev))
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]
    r = model._lock_request(main_ups, 0, p.PROM_ZIMAGE_TURBO_LOCK_ID)
    rc = model.lib.prometheus_reactor_runtime_main_transformer_create(model.h, ctypes.byref(r), ctypes.byref(bid),
                                                                      ctypes.byref(ev))
    assert rc == p.PROM_ERROR and ev.detail_code == D["RESOURCE_CREATE_FAILED"]  # no session


def test_session_argument_checks(model):
    for lock, profile, route in ((0x1, 1, 1), (p.PROM_ZIMAGE_TURBO_LOCK_ID, 3, 1),
                                 (p.PROM_ZIMAGE_TURBO_LOCK_ID, 1, 4), (p.PROM_ZIMAGE_TURBO_LOCK_ID, 0, 1)):
        rc, sid, ev = model.session_create(lock, profile, route)
        assert rc == p.PROM_ERROR and sid == 0 and ev.detail_code == D["SESSION_INVALID_REQUEST"]
    rc, ev = model.session_evidence(5)
    assert rc == p.PROM_ERROR and ev.detail_code == D["SESSION_INVALID_REQUEST"]
    rc, ev = model.session_compose(5, 1, 1)
    assert rc == p.PROM_ERROR
    rc, ev = model.session_capture(5, 1, 1)
    assert rc == p.PROM_ERROR
    assert model.session_destroy(5) == p.PROM_ERROR


def test_reference_struct_sizes():
    # x86-64 sizes of reactor_api.h:800-1249 (also compared field by field in test_abi.py)
    assert ctypes.sizeof(p.PrometheusModelBlockCreateRequest) == 448
    assert ctypes.sizeof(p.PrometheusModelBlockEvidence) == 896
    assert ctypes.sizeof(p.PrometheusCompiledModelSessionEvidence) == 176
    assert ctypes.sizeof(p.PrometheusModelBlockWeightUpload) == 40
    assert ctypes.sizeof(p.PrometheusMainTransformerExecuteRequest) == 96


def test_owner_entries_validate_before_any_work(model):
    import numpy as np

    ups = FakeUploads(NOISE_BYTES)
    r = model._lock_request(ups, 0, p.PROM_ZIMAGE_TURBO_LOCK_ID)
    ev = p.PrometheusModelBlockEvidence()
    bid = ctypes.c_uint64(5)
    # no session: the owner needs one of the same lock
    rc = model.lib.prometheus_reactor_runtime_compiled_model_owner_create(model.h, ctypes.byref(r), ctypes.byref(bid),
                                                                          ctypes.byref(ev))
    assert rc == p.PROM_ERROR and bid.value == 0 and ev.detail_code == D["INVALID_REQUEST"]
    for local, count in ((1, 13), (0, 12)):
        r = model._lock_request(ups, local, p.PROM_ZIMAGE_TURBO_LOCK_ID)
        r.upload_count = count
        rc = model.lib.prometheus_reactor_runtime_compiled_model_owner_create(model.h, ctypes.byref(r),
                                                                              ctypes.byref(bid), ctypes.byref(ev))
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]
    rr = model._retarget_request(1, 0, ups)
    rr.lock_identity = 0x77
    rc = model.lib.prometheus_reactor_runtime_compiled_model_retarget(model.h, ctypes.byref(rr), ctypes.byref(ev))
    assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]
    rr = model._retarget_request(1, 0, ups)
    rc = model.lib.prometheus_reactor_runtime_compiled_model_retarget(model.h, ctypes.byref(rr), ctypes.byref(ev))
    assert rc == p.PROM_ERROR  # no owner
    rc = model.lib.prometheus_reactor_runtime_compiled_model_prefetch(model.h, ctypes.byref(rr), ctypes.byref(ev))
    assert rc == p.PROM_ERROR and ev.detail_code == D["REBIND_FAILED"]
    rc, ev = model.activate_prefetch(1)
    assert rc == p.PROM_ERROR and ev.detail_code == D["REBIND_FAILED"]
    rc, sev = model.evaluation_reset(1)
    assert rc == p.PROM_ERROR and sev.detail_code == D["SESSION_INVALID_REQUEST"]
    assert ctypes.sizeof(p.PrometheusCompiledModelRetargetRequest) == 40


def test_stage_split_request_checks(model):
    """M1B/M1C/M1D argument validation (reactor_vulkan_model_block.c:1964-1980,
    2068-2079, 2141-2158): malformed requests are INVALID_REQUEST before the
    block lookup; well-formed ones for an unknown block are NOT_FOUND."""
    import numpy as np

    xb = np.zeros(1024 * 3840, np.uint16)
    tb = np.zeros(256, np.uint16)
    audit = np.zeros(4 * 3840, np.float32)
    for stage, patch in ((0, lambda r: setattr(r, "struct_size", 8)), (0, lambda r: setattr(r, "input_identity", 0)),
                         (0, lambda r: setattr(r, "timestep_identity", 0)),
                         (0, lambda r: setattr(r, "model_input_bf16", None)),
                         (0, lambda r: setattr(r, "audit_enabled", 2)),
                         (0, lambda r: setattr(r, "audit_stage", 3)),   # a stage without auditing
                         (22, None), (0, None)):                         # audited stage out of 1..21
        audited = stage != 0 or patch is None
        rc, ev = model.execute_m1b(1, xb, tb, audit_stage=stage, audit=audit if audited else None,
                                   request_patch=patch)
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"], (stage, patch)
    rc, ev = model.execute_m1b(1, xb, tb, audit_stage=3, audit=audit)
    assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]
    # M1B sizes the ingress only after it has found the block
    rc, ev = model.execute_m1b(1, xb[:-1], tb)
    assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]

    out = np.zeros(1024 * 3840, np.float32)
    for patch in (lambda r: setattr(r, "struct_size", 8), lambda r: setattr(r, "output", None),
                  lambda r: setattr(r, "output_identity", 0), lambda r: setattr(r, "m1b_prefix_replay_identity", 0),
                  lambda r: setattr(r, "output_element_capacity", 1024 * 3840 - 1),
                  lambda r: setattr(r, "audit_stage", 0), lambda r: setattr(r, "audit_stage", 4)):
        rc, ev = model.execute_m1c(1, 0x77, out, request_patch=patch)
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]
    rc, ev = model.execute_m1c(1, 0x77, out)
    assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]

    for stage, n in ((3, 1024 * 10240 - 1), (4, 1024 * 10240 - 1), (5, 1024 * 10240 - 1), (7, 1024 * 3840 - 1),
                     (0, 1024 * 3840), (8, 1024 * 3840)):
        rc, ev = model.execute_m1d(1, 0x78, np.zeros(n, np.float32), audit_stage=stage)
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"], stage
    for patch in (lambda r: setattr(r, "m1c_prefix_replay_identity", 0), lambda r: setattr(r, "output_identity", 0),
                  lambda r: setattr(r, "struct_size", 8)):
        rc, ev = model.execute_m1d(1, 0x78, out, request_patch=patch)
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"]
    rc, ev = model.execute_m1d(1, 0x78, out, audit_stage=6)
    assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]


def test_static_audit_request_checks(model):
    """Static-audit argument validation (reactor_vulkan_model_block.c:2681-2684,
    3221-3227, 4041-4049): the lock, generations, identities and the arena
    capacity come first; a well-formed request for an unknown block is NOT_FOUND."""
    import numpy as np

    arena = np.zeros(p.PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES, np.uint8)
    for kind, cap in (("noise", p.PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES),
                      ("context", p.PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_ARENA_BYTES)):
        short = arena[:cap - 4]
        for args in (dict(input_generation=0, arena=arena[:cap]), dict(input_generation=1, arena=short),
                     dict(input_generation=1, arena=arena[:cap], output_identity=0),
                     dict(input_generation=1, arena=arena[:cap], lock=0x1234)):
            rc, ev = model.static_audit(kind, 1, **args)
            assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"], (kind, args)
        rc, ev = model.static_audit(kind, 1, 1, arena[:cap])
        assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]
    out_bytes = 1056 * 3840 * 4
    for args in (dict(layer=1), dict(session_id=0), dict(image_gen=0), dict(joint_gen=0),
                 dict(arena=arena[:out_bytes - 4]), dict(output_identity=0)):
        call = dict(block_id=1, session_id=1, image_gen=1, context_gen=1, joint_gen=1, arena=arena[:out_bytes])
        call.update(args)
        rc, ev = model.main_static_audit(**call)
        assert rc == p.PROM_ERROR and ev.detail_code == D["INVALID_REQUEST"], args
    rc, ev = model.main_static_audit(1, 1, 1, 1, 1, arena[:out_bytes])
    assert rc == p.PROM_ERROR and ev.detail_code == D["NOT_FOUND"]


def test_set_main_attention_route_argument_checks(model):
    """reactor_vulkan_model_block.c:4229-4251: no evidence pointer or an unknown
    route fails without touching anything; an unknown session fails with the
    session evidence."""
    for route in (0, 4):
        rc, _ = model.set_main_attention_route(1, route)
        assert rc == p.PROM_ERROR
    rc, _ = model.set_main_attention_route(1, p.PROM_MAIN_ATTENTION_ROUTE_AUTO, evidence=False)
    assert rc == p.PROM_ERROR
    rc, ev = model.set_main_attention_route(7, p.PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL)
    assert rc == p.PROM_ERROR and ev.created == 0
