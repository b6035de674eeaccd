"""CPU-side checks of the C ABI: exports, struct layouts, validation semantics.

These run without a GPU: the library loads, every declared entry point is
exported, ctypes layouts equal the C header's, and the reference's
device-less and argument-validation behaviour is reproduced
(Marionette/reactor_stub_tests.cpp:144-203; reactor_reduction_tests.cpp:206-364).
"""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oct_amd import prometheus as p

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "prometheus_reactor.h"
LIB = REPO / "oct_amd" / "libprometheus_reactor.so"


def declared_entry_points():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"PROM_REACTOR_API\s+[\w\s\*]+?\b(prometheus_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_entry_points()
    assert len(names) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    # nothing beyond the declared ABI leaks out
    extra = sorted(e for e in exported if e.startswith("prometheus_") and e not in names)
    assert not extra, extra
    lib = ctypes.CDLL(str(LIB))
    for n in names:
        assert hasattr(lib, n)


def test_library_has_gfx950_code_object():
    # The HIP fat binary embedded in our own build names its offload target.
    data = LIB.read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


STRUCTS = {
    "PrometheusCaps": p.PrometheusCaps,
    "PrometheusReactorConfig": p.PrometheusReactorConfig,
    "PrometheusVulkanDeviceDiagnostics": p.PrometheusVulkanDeviceDiagnostics,
    "PrometheusHipDeviceDiagnostics": p.PrometheusHipDeviceDiagnostics,
    "PrometheusReductionRequest": p.PrometheusReductionRequest,
    "PrometheusReductionStageDispatch": p.PrometheusReductionStageDispatch,
    "PrometheusReductionPlan": p.PrometheusReductionPlan,
    "PrometheusReductionExecutionResult": p.PrometheusReductionExecutionResult,
    "PrometheusRowWiseSoftmaxRequest": p.PrometheusRowWiseSoftmaxRequest,
    "PrometheusRowWiseSoftmaxResult": p.PrometheusRowWiseSoftmaxResult,
    "PrometheusGemma4E2BM1InputRmsNormRequest": p.PrometheusGemma4E2BM1InputRmsNormRequest,
    "PrometheusGemma4E2BM1InputRmsNormResult": p.PrometheusGemma4E2BM1InputRmsNormResult,
    "PrometheusRmsNormRequest": p.PrometheusRmsNormRequest,
    "PrometheusRmsNormResult": p.PrometheusRmsNormResult,
    "PrometheusDecoderLayerF32Request": p.PrometheusDecoderLayerF32Request,
    "PrometheusDitBlockBf16Request": p.PrometheusDitBlockBf16Request,
    "PrometheusBlockResult": p.PrometheusBlockResult,
    "PrometheusAsyncStatus": p.PrometheusAsyncStatus,
    "PrometheusSgemmBatchEntry": p.PrometheusSgemmBatchEntry,
    "PrometheusSgemmBatchDiagnostics": p.PrometheusSgemmBatchDiagnostics,
    "PrometheusSgemmAsyncTaskDiagnostics": p.PrometheusSgemmAsyncTaskDiagnostics,
    "PrometheusSgemmAsyncDiagnostics": p.PrometheusSgemmAsyncDiagnostics,
    "PrometheusGemma4E2BM1RopeRequest": p.PrometheusGemma4E2BM1RopeRequest,
    "PrometheusGemma4E2BM1RopeResult": p.PrometheusGemma4E2BM1RopeResult,
    "PrometheusGemma4E2BM1HeadRmsNormRopeRequest": p.PrometheusGemma4E2BM1HeadRmsNormRopeRequest,
    "PrometheusGemma4E2BM1HeadRmsNormRopeResult": p.PrometheusGemma4E2BM1HeadRmsNormRopeResult,
    "PrometheusGemma4E2BM1AttentionScoresRequest": p.PrometheusGemma4E2BM1AttentionScoresRequest,
    "PrometheusGemma4E2BM1AttentionScoresResult": p.PrometheusGemma4E2BM1AttentionScoresResult,
    "PrometheusModelBlockWeightDeclaration": p.PrometheusModelBlockWeightDeclaration,
    "PrometheusModelBlockCreateRequest": p.PrometheusModelBlockCreateRequest,
    "PrometheusModelBlockWeightUpload": p.PrometheusModelBlockWeightUpload,
    "PrometheusNoiseRefinerRebindRequest": p.PrometheusNoiseRefinerRebindRequest,
    "PrometheusContextRefinerCreateRequest": p.PrometheusContextRefinerCreateRequest,
    "PrometheusMainTransformerCreateRequest": p.PrometheusContextRefinerCreateRequest,
    "PrometheusMainTransformerExecuteRequest": p.PrometheusMainTransformerExecuteRequest,
    "PrometheusModelBlockExecuteRequest": p.PrometheusModelBlockExecuteRequest,
    "PrometheusNoiseRefiner0ExecuteRequest": p.PrometheusNoiseRefiner0ExecuteRequest,
    "PrometheusNoiseRefiner1ExecuteRequest": p.PrometheusNoiseRefiner0ExecuteRequest,
    "PrometheusNoiseRefinerResidentExecuteRequest": p.PrometheusNoiseRefinerResidentExecuteRequest,
    "PrometheusContextRefiner0ExecuteRequest": p.PrometheusContextRefiner0ExecuteRequest,
    "PrometheusContextRefinerResidentExecuteRequest": p.PrometheusContextRefinerResidentExecuteRequest,
    "PrometheusNoiseRefinerFinalAuditRequest": p.PrometheusNoiseRefinerFinalAuditRequest,
    "PrometheusModelBlockEvidence": p.PrometheusModelBlockEvidence,
    "PrometheusCompiledModelSessionCreateRequest": p.PrometheusCompiledModelSessionCreateRequest,
    "PrometheusCompiledModelSessionCaptureRequest": p.PrometheusCompiledModelSessionCaptureRequest,
    "PrometheusCompiledModelSessionComposeRequest": p.PrometheusCompiledModelSessionComposeRequest,
    "PrometheusCompiledModelSessionEvidence": p.PrometheusCompiledModelSessionEvidence,
    "PrometheusCompiledModelRetargetRequest": p.PrometheusCompiledModelRetargetRequest,
    "PrometheusCompiledModelPrefetchRequest": p.PrometheusCompiledModelRetargetRequest,
    "PrometheusModelBlockM1BExecuteRequest": p.PrometheusModelBlockM1BExecuteRequest,
    "PrometheusModelBlockM1CExecuteRequest": p.PrometheusModelBlockM1CExecuteRequest,
    "PrometheusModelBlockM1DExecuteRequest": p.PrometheusModelBlockM1DExecuteRequest,
    "PrometheusNoiseRefinerStaticAuditRequest": p.PrometheusNoiseRefinerStaticAuditRequest,
    "PrometheusContextRefinerStaticAuditRequest": p.PrometheusNoiseRefinerStaticAuditRequest,
    "PrometheusMainTransformerStaticAuditRequest": p.PrometheusMainTransformerStaticAuditRequest,
    "PrometheusComplex32": p.PrometheusComplex32,
    "PrometheusFftRequest": p.PrometheusFftRequest,
    "PrometheusFftDiagnostics": p.PrometheusFftDiagnostics,
    "PrometheusReductionDiagnostics": p.PrometheusReductionDiagnostics,
    "PrometheusReductionBenchmarkRequest": p.PrometheusReductionBenchmarkRequest,
    "PrometheusReductionBenchmarkResult": p.PrometheusReductionBenchmarkResult,
}
MODEL_BLOCK_STRUCTS = tuple(n for n in STRUCTS if "ModelBlock" in n or "Refiner" in n or "MainTransformer" in n
                            or "CompiledModel" in n)

# Structs whose layout the reference header fixes (a drop-in caller compiled
# against it must read the same bytes).
REFERENCE_STRUCTS = (
    "PrometheusCaps", "PrometheusReactorConfig", "PrometheusVulkanDeviceDiagnostics", "PrometheusReductionRequest",
    "PrometheusReductionStageDispatch", "PrometheusReductionPlan", "PrometheusReductionExecutionResult",
    "PrometheusRowWiseSoftmaxRequest", "PrometheusRowWiseSoftmaxResult", "PrometheusGemma4E2BM1InputRmsNormRequest",
    "PrometheusGemma4E2BM1InputRmsNormResult", "PrometheusAsyncStatus", "PrometheusSgemmBatchEntry",
    "PrometheusSgemmBatchDiagnostics", "PrometheusSgemmAsyncTaskDiagnostics", "PrometheusSgemmAsyncDiagnostics",
    "PrometheusGemma4E2BM1RopeRequest", "PrometheusGemma4E2BM1RopeResult", "PrometheusGemma4E2BM1HeadRmsNormRopeRequest",
    "PrometheusGemma4E2BM1HeadRmsNormRopeResult", "PrometheusGemma4E2BM1AttentionScoresRequest",
    "PrometheusGemma4E2BM1AttentionScoresResult", "PrometheusComplex32", "PrometheusFftRequest",
    "PrometheusFftDiagnostics", "PrometheusReductionDiagnostics", "PrometheusReductionBenchmarkRequest",
    "PrometheusReductionBenchmarkResult",
) + MODEL_BLOCK_STRUCTS
REFERENCE_HEADER = Path("/root/reference/internal/prometheus/native/reactor_api.h")


def _layout(tmp_path, header: Path, names, tag: str) -> dict:
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{header}"', "int main(void){"]
    for name in names:
        cls = STRUCTS[name]
        lines.append(f'printf("{name} %zu\\n", sizeof({name}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{name}.{field} %zu\\n", offsetof({name}, {field}));')
    lines.append("return 0;}")
    src = tmp_path / f"layout_{tag}.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / f"layout_{tag}"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    return dict(line.rsplit(" ", 1) for line in out.splitlines())


@pytest.mark.skipif(not REFERENCE_HEADER.exists(), reason="reference tree not present on this machine")
def test_layouts_equal_the_reference_header(tmp_path):
    """Every shared struct has the reference's size and field offsets
    (compiled against internal/prometheus/native/reactor_api.h itself)."""
    ours = _layout(tmp_path, HEADER, REFERENCE_STRUCTS, "ours")
    ref = _layout(tmp_path, REFERENCE_HEADER, REFERENCE_STRUCTS, "ref")
    diff = {k: (ours[k], ref[k]) for k in ours if ours[k] != ref[k]}
    assert not diff, diff


def _constant_values(tmp_path, header: Path, names, tag: str) -> dict:
    lines = ["#include <stdio.h>", f'#include "{header}"', "int main(void){"]
    lines += [f'printf("{n} %lld\\n", (long long)({n}));' for n in names]
    lines.append("return 0;}")
    src = tmp_path / f"const_{tag}.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / f"const_{tag}"
    subprocess.run(["gcc", "-std=c11", "-w", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    return dict(line.rsplit(" ", 1) for line in out.splitlines())


@pytest.mark.skipif(not REFERENCE_HEADER.exists(), reason="reference tree not present on this machine")
def test_constants_equal_the_reference_header(tmp_path):
    """Every enum value and macro this header shares by name with the
    reference's (status, stage and detail codes, fault-injection bits, limits)
    has the reference's value, evaluated by the C compiler in both headers."""
    pattern = re.compile(r"^\s*(PROM_[A-Z0-9_]+)\s*=|^#define\s+(PROM_[A-Z0-9_]+)\s+\S", re.M)

    def names(text):
        return {a or b for a, b in pattern.findall(text)}

    ours_text = HEADER.read_text()
    ref_text = REFERENCE_HEADER.read_text()
    shared = sorted((names(ours_text) & names(ref_text)) - {"PROM_REACTOR_API"})  # the export attribute
    assert len(shared) > 100
    ours = _constant_values(tmp_path, HEADER, shared, "ours")
    ref = _constant_values(tmp_path, REFERENCE_HEADER, shared, "ref")
    diff = {k: (ours[k], ref[k]) for k in shared if ours[k] != ref[k]}
    assert not diff, diff


def test_ctypes_layouts_match_c_header(tmp_path):
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){"]
    for name, cls in STRUCTS.items():
        lines.append(f'printf("{name} %zu\\n", sizeof({name}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{name}.{field} %zu\\n", offsetof({name}, {field}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    c_layout = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                                    check=True).stdout.splitlines())
    for name, cls in STRUCTS.items():
        assert int(c_layout[name]) == ctypes.sizeof(cls), name
        for field, _ in cls._fields_:
            assert int(c_layout[f"{name}.{field}"]) == getattr(cls, field).offset, f"{name}.{field}"


def test_reference_struct_sizes_unchanged():
    # Layouts fixed by the reference header (x86-64): reactor_api.h:512-598, 1582-1586, 1751-1769.
    assert ctypes.sizeof(p.PrometheusCaps) == 12
    assert ctypes.sizeof(p.PrometheusReductionRequest) == 64
    assert ctypes.sizeof(p.PrometheusReactorConfig) == 40
    assert ctypes.sizeof(p.PrometheusRowWiseSoftmaxRequest) == 48
    assert ctypes.sizeof(p.PrometheusGemma4E2BM1InputRmsNormRequest) == 112
    # reactor_api.h:1307-1447, 1771-1779, 1987-2032
    assert ctypes.sizeof(p.PrometheusSgemmBatchEntry) == 40
    assert ctypes.sizeof(p.PrometheusSgemmBatchDiagnostics) == 3984
    assert ctypes.sizeof(p.PrometheusAsyncStatus) == 28
    assert ctypes.sizeof(p.PrometheusSgemmAsyncTaskDiagnostics) == 88
    assert ctypes.sizeof(p.PrometheusSgemmAsyncDiagnostics) == 488
    # reactor_api.h:1837-1985
    assert ctypes.sizeof(p.PrometheusGemma4E2BM1RopeRequest) == 104
    assert ctypes.sizeof(p.PrometheusGemma4E2BM1HeadRmsNormRopeRequest) == 144
    assert ctypes.sizeof(p.PrometheusGemma4E2BM1AttentionScoresRequest) == 208
    assert ctypes.sizeof(p.PrometheusGemma4E2BM1AttentionScoresResult) == 136


@pytest.fixture
def lib():
    return p.load_library(str(LIB))


def test_abi_version(lib):
    assert lib.prometheus_reactor_abi_version() == 1


def test_create_destroy_lifecycle(lib):
    h = ctypes.c_void_p()
    assert lib.prometheus_reactor_runtime_create(None, ctypes.byref(h)) == p.PROM_OK
    assert h.value
    assert lib.prometheus_reactor_runtime_destroy(h) == p.PROM_OK
    assert lib.prometheus_reactor_runtime_destroy(h) == p.PROM_INVALID_HANDLE


def test_invalid_usage(lib):
    assert lib.prometheus_reactor_runtime_create(None, None) == p.PROM_ERROR
    caps = p.PrometheusCaps()
    assert lib.prometheus_reactor_runtime_probe(None, ctypes.byref(caps)) == p.PROM_INVALID_HANDLE
    h = ctypes.c_void_p()
    assert lib.prometheus_reactor_runtime_create(None, ctypes.byref(h)) == p.PROM_OK
    assert lib.prometheus_reactor_runtime_probe(h, None) == p.PROM_ERROR
    lib.prometheus_reactor_runtime_destroy(h)


def test_forced_unavailable_runtime_reports_reference_caps():
    # PROM_TESTCFG_SKIP_VULKAN_INIT forces the device-less runtime on any machine.
    with p.NativeRuntime(test_flags=p.TESTCFG_SKIP_VULKAN_INIT) as rt:
        assert rt.caps.available == 0
        assert rt.caps.backend_type == p.PROM_BACKEND_UNKNOWN
        assert rt.caps.reason_code == p.PROM_REASON_VULKAN_UNAVAILABLE
        out, st, rc = rt.sgemm_with_status(1, 1, 1, [1.0], [1.0])
        assert rc == p.PROM_ERROR and st.stage == p.STAGE_INIT and out is None
        with pytest.raises(p.ReactorIssue):
            rt.require_hardware_gpu()


def test_sgemm_argument_validation_order(lib):
    h = ctypes.c_void_p()
    lib.prometheus_reactor_runtime_create(None, ctypes.byref(h))
    st, d = ctypes.c_uint32(), ctypes.c_int()
    a = np.ones(4, np.float32)
    ptr = a.ctypes.data
    # invalid handle -> INIT / PROM_INVALID_HANDLE (reactor_sgemm.cpp:4152-4155)
    assert lib.prometheus_reactor_runtime_sgemm(None, ptr, ptr, ptr, 1, 1, 1, ctypes.byref(st), ctypes.byref(d)) == 2
    assert (st.value, d.value) == (p.STAGE_INIT, p.PROM_INVALID_HANDLE)
    # NULL operand -> TRANSFER_IN / PROM_ERROR
    assert lib.prometheus_reactor_runtime_sgemm(h, None, ptr, ptr, 1, 1, 1, ctypes.byref(st), ctypes.byref(d)) == 1
    assert (st.value, d.value) == (p.STAGE_TRANSFER_IN, p.PROM_ERROR)
    # zero dimension -> INIT / PROM_ERROR
    assert lib.prometheus_reactor_runtime_sgemm(h, ptr, ptr, ptr, 0, 1, 1, ctypes.byref(st), ctypes.byref(d)) == 1
    assert (st.value, d.value) == (p.STAGE_INIT, p.PROM_ERROR)
    lib.prometheus_reactor_runtime_destroy(h)


def _request(rows, width, op, flags=0, fin=None, in_count=None, out_count=None):
    r = p.PrometheusReductionRequest()
    r.struct_size = ctypes.sizeof(r)
    r.row_count, r.elements_per_row = rows, width
    r.operation = op
    r.finalization = (1 if op == p.OP_SOFTMAX else 0) if fin is None else fin
    r.flags = flags
    r.input_element_count = rows * width if in_count is None else in_count
    r.output_element_count = (rows * width if op == p.OP_SOFTMAX else rows) if out_count is None else out_count
    return r


def _plan(lib, req):
    plan = p.PrometheusReductionPlan()
    rc = lib.prometheus_reactor_reduction_plan(ctypes.byref(req), ctypes.byref(plan))
    return rc, plan


def test_reduction_plan_reference_schedule(lib):
    # PrometheusReduction.concept:128-164 via reactor_vulkan_fused_reduction.c:101-148
    rc, plan = _plan(lib, _request(128, 4096, p.OP_SUM))
    assert rc == 0 and plan.strategy == 2 and plan.partial_count == 4 and plan.stage_count == 2
    assert [plan.stages[i].stage_role for i in range(2)] == [1, 1]
    assert plan.stages[0].groups_x == 128 * 4 and plan.stages[0].temporary_role == 1
    assert plan.temporary_bytes == 128 * 4 * 4
    rc, plan = _plan(lib, _request(16, 4096, p.OP_SOFTMAX))
    assert rc == 0 and plan.stage_count == 5
    assert [plan.stages[i].stage_role for i in range(5)] == [2, 2, 3, 1, 4]
    assert plan.stages[4].groups_x == (16 * 4096 + 255) // 256
    assert plan.temporary_bytes == 16 * 4 * 4 + 2 * 16 * 4
    rc, plan = _plan(lib, _request(1024, 512, p.OP_SOFTMAX))
    assert rc == 0 and plan.strategy == 1 and plan.stage_count == 1 and plan.stages[0].stage_role == 5
    rc, plan = _plan(lib, _request(4, 64, p.OP_SOFTMAX))
    assert plan.strategy == 3 and plan.stages[0].stage_role == 7 and plan.stages[0].groups_x == 1
    rc, plan = _plan(lib, _request(1024, 100, p.OP_SUM))
    assert plan.strategy == 3 and plan.stages[0].stage_role == 6
    rc, plan = _plan(lib, _request(1024, 100, p.OP_MAX))
    assert plan.strategy == 2
    # forced composed softmax at narrow width
    rc, plan = _plan(lib, _request(8, 512, p.OP_SOFTMAX, flags=2))
    assert plan.strategy == 2 and plan.stage_count == 3
    # replay ids distinguish plans and are stable
    a = _plan(lib, _request(8, 512, p.OP_SOFTMAX))[1].replay_id
    assert a == _plan(lib, _request(8, 512, p.OP_SOFTMAX))[1].replay_id
    assert a != _plan(lib, _request(8, 513, p.OP_SOFTMAX))[1].replay_id


@pytest.mark.parametrize("req,detail", [
    (dict(rows=0, width=4, op=1), -6804),
    (dict(rows=4, width=0, op=1), -6805),
    (dict(rows=1025, width=4, op=1), -6811),
    (dict(rows=1, width=1048577, op=1), -6812),
    (dict(rows=1024, width=16385, op=1), -6813),
    (dict(rows=4, width=4, op=4), -6806),
    (dict(rows=4, width=4, op=1, fin=1), -6807),
    (dict(rows=4, width=4, op=3, fin=0), -6807),
    (dict(rows=4, width=4, op=1, flags=1), -6815),
    (dict(rows=4, width=1057, op=3, flags=1), -6815),
    (dict(rows=4, width=4, op=1, in_count=15), -6809),
    (dict(rows=4, width=4, op=1, out_count=16), -6810),
])
def test_reduction_validation_codes(lib, req, detail):
    r = _request(req["rows"], req["width"], req["op"], req.get("flags", 0), req.get("fin"), req.get("in_count"),
                 req.get("out_count"))
    x = np.zeros(max(1, req["rows"] * req["width"]), np.float32)
    r.input = x.ctypes.data
    r.output = x.ctypes.data
    assert _plan(lib, r)[0] == p.PROM_ERROR
    with p.NativeRuntime(lib=lib, test_flags=p.TESTCFG_SKIP_VULKAN_INIT) as rt:
        res = p.PrometheusReductionExecutionResult()
        rc = lib.prometheus_reactor_runtime_reduction(rt.handle, ctypes.byref(r), ctypes.byref(res))
        assert rc == p.PROM_ERROR and res.stage == p.STAGE_INIT and res.detail_code == detail


def test_reduction_v2_lifts_the_envelope_but_keeps_codes(lib):
    with p.NativeRuntime(lib=lib, test_flags=p.TESTCFG_SKIP_VULKAN_INIT) as rt:
        x = np.ones((8192, 4), np.float32)
        rc, res, _ = rt.reduction(x, p.OP_SUM, lifted=False)
        assert rc == 1 and res.detail_code == -6811
        rc, res, _ = rt.reduction(x, p.OP_SUM, lifted=True)
        # admitted, then refused only because this runtime has no device
        assert rc == 1 and res.detail_code == -6825 and res.stage == p.STAGE_INIT


def test_reduction_nonfinite_is_transfer_in(lib):
    with p.NativeRuntime(lib=lib, test_flags=p.TESTCFG_SKIP_VULKAN_INIT) as rt:
        x = np.ones((3, 5), np.float32)
        x[2, 1] = np.nan
        rc, res, _ = rt.reduction(x, p.OP_MAX)
        assert rc == 1 and res.stage == p.STAGE_TRANSFER_IN and res.detail_code == -6814
        assert res.first_nonfinite_index == 11


def test_row_wise_softmax_validation(lib):
    with p.NativeRuntime(lib=lib, test_flags=p.TESTCFG_SKIP_VULKAN_INIT) as rt:
        x = np.zeros(64, np.float32)
        req = p.PrometheusRowWiseSoftmaxRequest()
        req.struct_size = ctypes.sizeof(req)
        res = p.PrometheusRowWiseSoftmaxResult()
        call = lambda: lib.prometheus_reactor_runtime_row_wise_softmax(rt.handle, ctypes.byref(req), ctypes.byref(res))
        # zero rows, zero counts: synchronous no-op
        assert call() == 0 and res.stage == 0
        req.row_count, req.elements_per_row, req.input_element_count, req.output_element_count = 2, 4, 8, 7
        assert call() == 1 and res.detail_code == -6854
        req.output_element_count = 8
        assert call() == 1 and res.detail_code == -6852
        req.input = x.ctypes.data
        req.output = x.ctypes.data + 4  # partial overlap
        assert call() == 1 and res.detail_code == -6859
        req.output = x.ctypes.data  # exact in-place is allowed -> reaches the device check
        assert call() == 1 and res.detail_code == -6861
        req.row_count, req.input_element_count, req.output_element_count = 1025, 1025 * 4, 1025 * 4
        assert call() == 1 and res.detail_code == -6856
        req.row_count, req.elements_per_row = 1, 1057
        req.input_element_count = req.output_element_count = 1057
        assert call() == 1 and res.detail_code == -6857


def test_gemma_rmsnorm_validation(lib):
    # reactor_api.c:250-275 then reactor_concept_rmsnorm.cpp:85-95: malformed requests and a
    # runtime without a device both end at INIT / -7401 with PROM_ERROR
    with p.NativeRuntime(lib=lib, test_flags=p.TESTCFG_SKIP_VULKAN_INIT) as rt:
        x = np.ones((2, 8), np.float32)
        w = np.ones(8, np.float32)
        y = np.zeros((2, 8), np.float32)
        inv = np.zeros(2, np.float32)
        req = p.PrometheusGemma4E2BM1InputRmsNormRequest()
        req.struct_size = ctypes.sizeof(req)
        res = p.PrometheusGemma4E2BM1InputRmsNormResult()
        for fn in (lib.prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm,
                   lib.prometheus_reactor_runtime_gemma4e2b_m1_projection_activation_rmsnorm):
            call = lambda: fn(rt.handle, ctypes.byref(req), ctypes.byref(res))
            assert call() == 1 and (res.stage, res.detail_code) == (p.STAGE_INIT, -7401)
            req.input, req.weight, req.output, req.inv_rms_output = (x.ctypes.data, w.ctypes.data, y.ctypes.data,
                                                                     inv.ctypes.data)
            req.input_element_count, req.weight_element_count, req.output_element_count = 16, 8, 16
            req.inv_rms_output_element_count = 2
            req.tokens, req.model_width, req.input_row_stride, req.epsilon = 2, 8, 8, 1e-6
            req.input_generation = req.weight_generation = req.exact_source_hash = 1
            assert call() == 1 and (res.stage, res.detail_code) == (p.STAGE_INIT, -7401)
            assert res.weight_hash != 0  # the weight was hashed before the device check
            w[3] = np.nan
            assert call() == 1 and (res.stage, res.detail_code) == (p.STAGE_INIT, p.DETAIL_M46_NONFINITE_INPUT)
            w[3] = 1.0
            req.input_generation = 0
            assert call() == 1 and res.detail_code == -7401
            req.input_generation = 1
        # an invalid handle is reported through the weight step: PROM_ERROR, INIT / -7401
        assert lib.prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm(None, ctypes.byref(req), ctypes.byref(res)) == 1
        assert (res.stage, res.detail_code) == (p.STAGE_INIT, -7401)


def _head_request(x, w, y, inv, rows):
    r = p.PrometheusGemma4E2BM1InputRmsNormRequest()
    r.struct_size = ctypes.sizeof(r)
    r.input, r.weight, r.output, r.inv_rms_output = x.ctypes.data, w.ctypes.data, y.ctypes.data, inv.ctypes.data
    r.input_element_count = r.output_element_count = rows * 256
    r.weight_element_count, r.inv_rms_output_element_count = 256, rows
    r.tokens, r.model_width, r.input_row_stride, r.epsilon = rows, 256, 256, 1e-6
    r.input_generation = r.weight_generation = r.exact_source_hash = 1
    return r


def test_gemma_head_rmsnorm_shape_lock(lib):
    # reactor_api.c:373-392: rows <= 120, width and stride 256, exact counts, epsilon exactly 1e-6
    with p.NativeRuntime(lib=lib, test_flags=p.TESTCFG_SKIP_VULKAN_INIT) as rt:
        x, w = np.ones((121, 256), np.float32), np.ones(256, np.float32)
        y, inv = np.zeros_like(x), np.zeros(121, np.float32)
        res = p.PrometheusGemma4E2BM1InputRmsNormResult()
        fn = lib.prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm
        for mutate in (lambda r: setattr(r, "tokens", 121), lambda r: setattr(r, "epsilon", 1e-5),
                       lambda r: setattr(r, "input_row_stride", 257), lambda r: setattr(r, "model_width", 128),
                       lambda r: setattr(r, "output_element_count", 120 * 256 + 1)):
            req = _head_request(x, w, y, inv, 120)
            mutate(req)
            assert fn(rt.handle, ctypes.byref(req), ctypes.byref(res)) == 1
            assert (res.stage, res.detail_code) == (p.STAGE_INIT, -7401)


def test_gemma_rope_and_scores_validation(lib):
    with p.NativeRuntime(lib=lib, test_flags=p.TESTCFG_SKIP_VULKAN_INIT) as rt:
        src, out = np.ones(15 * 8 * 256, np.float32), np.zeros(15 * 8 * 256, np.float32)
        cos, sin = np.ones(3840, np.float32), np.zeros(3840, np.float32)
        r = p.PrometheusGemma4E2BM1RopeRequest()
        r.struct_size = ctypes.sizeof(r)
        r.source, r.cosine, r.sine, r.output = src.ctypes.data, cos.ctypes.data, sin.ctypes.data, out.ctypes.data
        r.source_element_count = r.output_element_count = src.size
        r.cosine_element_count = r.sine_element_count = 3840
        r.tokens, r.heads, r.head_width = 15, 8, 256
        r.source_generation = r.table_generation = 1
        res = p.PrometheusGemma4E2BM1RopeResult()
        rope = lambda h: lib.prometheus_reactor_runtime_gemma4e2b_m1_rope(h, ctypes.byref(r), ctypes.byref(res))
        # reactor_concept_rmsnorm.cpp:157-172: handle first, then the request
        assert rope(None) == p.PROM_INVALID_HANDLE
        # no device: the request is valid, inputs hashed, then RESOURCE at INIT
        assert rope(rt.handle) == 1 and (res.stage, res.detail_code) == (p.STAGE_INIT, p.DETAIL_M46_RESOURCE)
        assert res.source_hash != 0 and res.cosine_hash != res.sine_hash
        r.output = src.ctypes.data  # in place is refused
        assert rope(rt.handle) == 1 and res.detail_code == -7401
        r.output, r.heads = out.ctypes.data, 2
        assert rope(rt.handle) == 1 and res.detail_code == -7401
        r.heads = 8
        src[5] = np.inf
        assert rope(rt.handle) == 1 and res.detail_code == p.DETAIL_M46_NONFINITE_INPUT
        # attention scores: the closed 15 x 8 x 1 x 256 geometry and scale 0.0625
        a = p.PrometheusGemma4E2BM1AttentionScoresRequest()
        a.struct_size = ctypes.sizeof(a)
        scores = np.full(1800, -99, np.float32)
        a.query_input = a.key_input = a.query_weight = a.key_weight = src.ctypes.data
        a.cosine, a.sine, a.scores = cos.ctypes.data, sin.ctypes.data, scores.ctypes.data
        a.query_input_element_count, a.key_input_element_count = 15 * 8 * 256, 15 * 256
        a.query_weight_element_count = a.key_weight_element_count = 256
        a.cosine_element_count = a.sine_element_count = 3840
        a.score_element_count = 1800
        a.tokens, a.query_heads, a.key_heads, a.head_width, a.epsilon, a.scale = 15, 8, 1, 256, 1e-6, 0.125
        for f in ("query_input_generation", "key_input_generation", "query_weight_generation",
                  "key_weight_generation", "table_generation", "query_exact_source_hash", "key_exact_source_hash"):
            setattr(a, f, 1)
        ares = p.PrometheusGemma4E2BM1AttentionScoresResult()
        call = lambda: lib.prometheus_reactor_runtime_gemma4e2b_m1_attention_scores(rt.handle, ctypes.byref(a),
                                                                                    ctypes.byref(ares))
        assert call() == 1 and (ares.stage, ares.detail_code) == (p.STAGE_INIT, -7401)
        a.scale, a.preparation_order = 0.0625, 2
        assert call() == 1 and ares.detail_code == -7401
        assert np.all(scores == -99)


def test_strict_path_raises_without_device(monkeypatch):
    monkeypatch.setenv(p.REACTOR_TEST_FLAGS_ENV_VAR, str(p.TESTCFG_SKIP_VULKAN_INIT))
    with pytest.raises(p.ReactorIssue, match="PROMETHEUS requires GPU matrix execution"):
        p.run_compiled_matmul_mm_strict([[1.0, 2.0], [3.0, 4.0]], [[1.0, 2.0], [3.0, 4.0]])


def test_strict_path_missing_library_is_an_error(monkeypatch, tmp_path):
    # Language/Prometheus/unavailable/matrix.octfail: no CPU substitute when the reactor is absent
    monkeypatch.setenv(p.REACTOR_ENV_VAR, str(tmp_path / "missing" / p.LIBRARY_BASENAME))
    with pytest.raises(p.ReactorIssue, match="PROMETHEUS requires GPU matrix execution"):
        p.run_compiled_matmul_mm_strict([[1.0]], [[1.0]])


def test_compiled_matmul_request_shape_checks():
    with pytest.raises(ValueError, match="shape mismatch"):
        p.compiled_matmul_request([[1.0, 2.0]], [[1.0, 2.0]])
    with pytest.raises(ValueError, match="rectangular"):
        p.compiled_matmul_request([[1.0, 2.0], [1.0]], [[1.0], [2.0]])
    m, n, k, a, b = p.compiled_matmul_request([[0.1, 2.0]], [[1.0], [3.0]])
    assert (m, n, k) == (1, 1, 2) and a.dtype == np.float32 and a[0, 0] == np.float32(0.1)


def test_reduction_diagnostics_and_benchmark_without_device():
    """reactor_concept_reduction.cpp:96-115 and reactor_vulkan_fused_reduction.c:
    1122-1146: argument checks, and the counters a device-less runtime keeps."""
    rt = p.NativeRuntime(test_flags=0)
    try:
        rc, d = rt.reduction_diagnostics()
        assert rc == p.PROM_OK and d.struct_size == ctypes.sizeof(d) and d.total_requests == 0
        assert rt.lib.prometheus_reactor_runtime_reduction_diagnostics(rt.handle, None) == p.PROM_ERROR
        assert rt.lib.prometheus_reactor_runtime_reduction_diagnostics(None, ctypes.byref(d)) == p.PROM_INVALID_HANDLE
        x = np.ones((4, 8), np.float32)
        for patch in (lambda b: setattr(b, "measured_iterations", 0),
                      lambda b: setattr(b, "measured_iterations", 10001),
                      lambda b: setattr(b, "struct_size", 4)):
            rc, res, _ = rt.reduction_benchmark(x, p.OP_SUM, request_patch=patch)
            assert rc == p.PROM_ERROR and res.detail_code == p.REDUCTION_DETAIL["INVALID_REQUEST"]
            assert res.first_mismatch_row == 0xFFFFFFFF and res.completed_iterations == 0
        assert rt.lib.prometheus_reactor_runtime_reduction_benchmark(rt.handle, None, None) == p.PROM_ERROR
        if not rt.available:
            rc, res, _ = rt.reduction_benchmark(x, p.OP_SUM)
            assert rc == p.PROM_ERROR and res.detail_code == p.REDUCTION_DETAIL["RUNTIME_UNAVAILABLE"]
            rc, d = rt.reduction_diagnostics()
            assert d.total_requests == 1 and d.logical_failure_count == 1 and d.initialized == 0
            assert d.last_detail_code == p.REDUCTION_DETAIL["RUNTIME_UNAVAILABLE"]
    finally:
        rt.close()


def test_attention_entry_validates_before_the_device():
    """prometheus_reactor_runtime_attention_bf16_device: argument checks come
    first (INIT, PROM_DETAIL_INVALID_ARGUMENT); valid arguments on a runtime
    without a device stop at INIT with the runtime's unavailability detail."""
    rt = p.NativeRuntime(test_flags=p.TESTCFG_SKIP_VULKAN_INIT)
    try:
        ok = 1 << 20  # an aligned address; nothing is dereferenced on these paths
        for args in ((ok, ok, ok, ok, 64, 2, 128, 0), (ok, ok, ok, ok, 64, 1, 129, 0), (ok, ok, ok, ok, 0, 1, 128, 0),
                     (ok, ok, ok, ok, 64, 1, 128, 2), (ok, ok, ok, ok, 64, 0, 128, 0), (ok, ok, ok, ok, 1, 1, 1 << 24, 0), (ok + 2, ok, ok, ok, 64, 1, 128, 0),
                     (0, ok, ok, ok, 64, 1, 128, 0), (ok, ok, ok, ok, 1 << 20, 8, 1024, 0)):
            rc, st = rt.attention_bf16_device(*args)
            assert rc == p.PROM_ERROR and st.stage == p.STAGE_INIT and st.detail == p.DETAIL_INVALID_ARGUMENT, args
        rc, st = rt.attention_bf16_device(ok, ok, ok, ok, 64, 1, 128, 0)
        assert rc == p.PROM_ERROR and st.stage == p.STAGE_INIT and st.detail == p.DETAIL_HIP_UNAVAILABLE
    finally:
        rt.close()
