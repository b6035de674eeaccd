"""The non-strict SGEMM path of Oct's Prometheus package.

Mirrors ``internal/prometheus/runtime.go:12-658``: ``RunSGEMM``,
``RunCompiledMatMulMM`` and ``RunStarterCorpus`` over ``runSGEMMWithOutput``,
the async hardware validation ``ValidateAsyncSGEMMOnHardware``, and the
Octagon reports of both (``WriteOctagonReport``,
``WriteAsyncValidationOctagon``; the writer is ``oct_amd.octagon``).
Unlike the strict ``@`` (``run_compiled_matmul_mm_strict`` in
``oct_amd.prometheus``), this path always computes the fp32 CPU reference
first, then runs the reactor and gates its output against that reference with
``compareAgainstOracle`` (abs 1e-4 and rel 1e-4, non-finite values fail).  When
the reactor cannot be opened (library missing or unloadable, a symbol missing,
ABI mismatch, create failure, or a probe that reports no device) it returns the
CPU result with status ``fallback(prometheus_unavailable)`` and says so; any
other reactor failure is an error, never a silent substitute.

The CPU reference here is this package's own loop (``cpuSGEMM``,
``runtime.go:319-331``: fp32 products added in k order to an fp32 sum starting
at zero); it is part of the reference's contract for this path, not the
library's compute path.  The reactor library itself never falls back.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import numpy as np

from . import octagon
from . import prometheus as p

# runtime.go:12-15
DEFAULT_ABS_TOLERANCE = 1e-4
DEFAULT_REL_TOLERANCE = 1e-4

BACKEND_CPU = "cpu"
BACKEND_PROMETHEUS = "prometheus"

# bridge.go:33-42 codes that make the non-strict path fall back (runtime.go:208-219)
_UNAVAILABLE_CODES = ("reactor_not_found", "reactor_load_failed", "symbol_missing", "abi_mismatch",
                      "runtime_create_failed", "runtime_probe_unavailable")
# runtime.go:221-240
_BRIDGE_STATUS = {"reactor_load_failed": -10, "symbol_missing": -11, "abi_mismatch": -12,
                  "runtime_create_failed": -13, "runtime_probe_unavailable": -14}


@dataclass(frozen=True)
class Shape:
    """runtime.go:17-21."""

    m: int
    n: int
    k: int


# runtime.go:83-89
STARTER_CORPUS: Tuple[Shape, ...] = (Shape(1, 1, 1), Shape(4, 4, 4), Shape(16, 16, 16), Shape(32, 32, 32),
                                     Shape(3, 5, 7))


@dataclass
class SGEMMRequest:
    """runtime.go:23-28: A [m*k] and B [k*n] row-major float32."""

    backend: str
    shape: Shape
    a: np.ndarray
    b: np.ndarray


@dataclass
class CorrectnessResult:
    """runtime.go:30-38.  The zero value, as Go's, has not passed: a run that
    stopped before the gate reports CorrectnessPass false."""

    passed: bool = False
    max_abs_error: float = 0.0
    max_rel_error: float = 0.0
    failing_count: int = 0
    first_failing_index: int = -1
    first_expected_value: float = 0.0
    first_actual_value: float = 0.0


@dataclass
class SGEMMRunResult:
    """runtime.go:40-54 (``VulkanTimeNs``/``VulkanEnv`` keep the reference's names)."""

    requested_backend: str = ""
    used_backend: str = ""
    shape: Shape = Shape(0, 0, 0)
    status: p.RunStatus = field(default_factory=lambda: p.RunStatus("error", "unknown", -1))
    detail_code: int = 0
    detail_name: str = "not_applicable"
    correctness: CorrectnessResult = field(default_factory=CorrectnessResult)
    cpu_time_ns: int = 0
    vulkan_time_ns: int = 0
    vulkan_env: str = "not_applicable"
    timing_mode: str = "end_to_end"
    wall_time_ns: int = 0
    notes: str = ""


class SGEMMError(RuntimeError):
    """An error return of runSGEMMWithOutput; ``result`` carries the run record."""

    def __init__(self, message: str, result: SGEMMRunResult, output: Optional[np.ndarray] = None):
        super().__init__(message)
        self.result = result
        self.output = output


def deterministic_matrix(rows: int, cols: int) -> np.ndarray:
    """runtime.go:242-249: element i is float32((i % 23) - 11) / 7."""
    i = np.arange(rows * cols, dtype=np.int64)
    return (((i % 23) - 11).astype(np.float32) / np.float32(7.0)).astype(np.float32)


def cpu_sgemm(m: int, n: int, k: int, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """runtime.go:319-331: c[r,c] = fp32 sum over kk in order of fp32 a[r,kk]*b[kk,c], from +0.

    Every output's sum takes the same sequence of fp32 roundings as the Go
    loop (one rounded product, one rounded add per kk); the loop over kk is
    explicit and the m x n outputs advance together."""
    a2 = np.ascontiguousarray(a, dtype=np.float32).reshape(m, k)
    b2 = np.ascontiguousarray(b, dtype=np.float32).reshape(k, n)
    c = np.zeros((m, n), dtype=np.float32)
    prod = np.empty((m, n), dtype=np.float32)
    for kk in range(k):
        np.multiply(a2[:, kk:kk + 1], b2[kk:kk + 1, :], out=prod)
        np.add(c, prod, out=c)
    return c.reshape(-1)


def _timed_cpu_sgemm(m, n, k, a, b):
    t0 = time.perf_counter_ns()
    out = cpu_sgemm(m, n, k, a, b)
    return out, time.perf_counter_ns() - t0


def compare_against_oracle(expected: np.ndarray, actual: np.ndarray) -> CorrectnessResult:
    """runtime.go:339-372: an element fails when it or its reference is not finite, or
    when |e - a| (an fp32 difference) exceeds both the absolute and relative tolerance."""
    e = np.ascontiguousarray(expected, dtype=np.float32).reshape(-1)
    a = np.ascontiguousarray(actual, dtype=np.float32).reshape(-1)
    res = CorrectnessResult(passed=True)
    finite = np.isfinite(e) & np.isfinite(a)
    with np.errstate(over="ignore", invalid="ignore"):
        diff = np.where(finite, e - a, np.float32(0)).astype(np.float32)
    abs_err = np.abs(diff.astype(np.float64))
    denom = np.abs(e.astype(np.float64))
    with np.errstate(divide="ignore", invalid="ignore"):
        rel_err = np.where(finite & (e != 0), abs_err / np.where(denom == 0, 1.0, denom), 0.0)
    if finite.any():
        res.max_abs_error = float(abs_err[finite].max())
        res.max_rel_error = float(rel_err[finite].max())
    failing = ~finite | ((abs_err > DEFAULT_ABS_TOLERANCE) & (rel_err > DEFAULT_REL_TOLERANCE))
    count = int(failing.sum())
    if count:
        idx = int(np.argmax(failing))
        res.passed = False
        res.failing_count = count
        res.first_failing_index = idx
        res.first_expected_value = float(e[idx])
        res.first_actual_value = float(a[idx])
    return res


def detail_code_name(code: int) -> str:
    """runtime.go:434-495, plus this library's HIP path codes."""
    names = {0: "not_applicable", -10: "reactor_load_failed", -11: "reactor_symbol_missing",
             -12: "reactor_abi_mismatch", -13: "reactor_create_failed", -14: "reactor_probe_failed",
             -6001: "injected_upload_failure", -6002: "injected_dispatch_failure",
             -6003: "injected_download_failure", -6004: "size_overflow", -6005: "reuse_in_flight",
             -6006: "capability_mismatch", 6101: "direct", 6102: "staged_upload", 6103: "staged_upload_readback",
             6104: "fallback_to_direct", 6105: "direct_tiled", 6106: "staged_upload_tiled",
             6107: "staged_upload_readback_tiled", -6108: "async_not_ready", -6109: "async_no_task",
             -6110: "async_already_consumed", -6111: "async_invalid_task", -6112: "async_submit_rejected",
             -6113: "async_software_suppressed", -6114: "async_failed", -6115: "async_unconsumed",
             -6116: "injected_async_poll_failure",
             p.DETAIL_PATH_HIP_MFMA_F32: "hip_mfma_f32", p.DETAIL_PATH_HIP_GEMV_F32: "hip_gemv_f32",
             p.DETAIL_HIP_UNAVAILABLE: "hip_unavailable"}
    return names.get(code, f"detail_{code}")


def is_prometheus_unavailable(err: BaseException) -> bool:
    """runtime.go:208-219."""
    return isinstance(err, p.ReactorIssue) and err.code in _UNAVAILABLE_CODES


def bridge_issue_status_code(err: BaseException) -> int:
    """runtime.go:221-240."""
    if not isinstance(err, p.ReactorIssue):
        return -1
    return _BRIDGE_STATUS.get(err.code, -1)


def new_native_runtime() -> p.NativeRuntime:
    """bridge.go:238-340 (newNativeRuntime): load the reactor afresh, check the ABI,
    create a runtime and probe it; a probe without a device is
    ``runtime_probe_unavailable``, as the reference's ``!caps.Available``."""
    lib = p.load_library()
    rt = p.NativeRuntime(lib=lib)
    if not rt.available:
        rt.close()
        raise p.ReactorIssue("runtime_probe_unavailable", "prometheus reactor runtime probe failed")
    if not hasattr(lib, "prometheus_reactor_runtime_sgemm"):
        rt.close()
        raise p.ReactorIssue("symbol_missing", 'prometheus reactor missing symbol "prometheus_reactor_runtime_sgemm"')
    return rt


def _run_sgemm_with_output(req: SGEMMRequest) -> Tuple[Optional[np.ndarray], SGEMMRunResult]:
    """runtime.go:121-206.  Returns (output, result); raises SGEMMError where the Go code returns an error."""
    if req.backend not in (BACKEND_CPU, BACKEND_PROMETHEUS):
        raise ValueError(f'backend must be one of "{BACKEND_CPU}" or "{BACKEND_PROMETHEUS}"')
    m, n, k = req.shape.m, req.shape.n, req.shape.k
    if m <= 0 or n <= 0 or k <= 0:
        raise ValueError("shape dimensions must be positive")
    a = np.ascontiguousarray(req.a, dtype=np.float32).reshape(-1)
    b = np.ascontiguousarray(req.b, dtype=np.float32).reshape(-1)
    if a.size != m * k or b.size != k * n:
        raise ValueError("matrix dimensions do not match shape")

    result = SGEMMRunResult(requested_backend=req.backend, shape=req.shape)
    reference, cpu_ns = _timed_cpu_sgemm(m, n, k, a, b)
    result.cpu_time_ns = cpu_ns

    if req.backend == BACKEND_CPU:
        result.wall_time_ns = cpu_ns
        result.used_backend = BACKEND_CPU
        result.status = p.RunStatus("ok")
        result.detail_name = "cpu"
        result.correctness = compare_against_oracle(reference, reference)
        if not result.correctness.passed:
            raise SGEMMError(f"correctness gate failed for backend={result.used_backend}", result, reference)
        return reference, result

    try:
        rt = new_native_runtime()
    except p.ReactorIssue as exc:
        if is_prometheus_unavailable(exc):
            result.wall_time_ns = cpu_ns
            result.used_backend = BACKEND_CPU
            result.status = p.RunStatus("fallback", fallback_reason="prometheus_unavailable")
            result.notes = f"prometheus reactor unavailable; used cpu fallback: {exc}"
            result.vulkan_env = "unavailable"
            result.detail_name = "fallback_cpu"
            result.correctness = compare_against_oracle(reference, reference)
            if not result.correctness.passed:
                raise SGEMMError(f"correctness gate failed for fallback backend={result.used_backend}", result,
                                 reference) from exc
            return reference, result
        code = bridge_issue_status_code(exc)
        result.used_backend = BACKEND_PROMETHEUS
        result.status = p.RunStatus("error", "init", code)
        result.detail_code = code
        result.detail_name = detail_code_name(code)
        raise SGEMMError(str(exc), result) from exc

    with rt:
        result.vulkan_env = rt.environment()
        t0 = time.perf_counter_ns()
        actual, st, rc = rt.sgemm_with_status(m, n, k, a, b)
        result.vulkan_time_ns = time.perf_counter_ns() - t0
    result.wall_time_ns = result.vulkan_time_ns
    result.used_backend = BACKEND_PROMETHEUS
    result.detail_code = st.detail
    result.detail_name = detail_code_name(st.detail)
    if rc != p.PROM_OK:
        result.status = p.RunStatus("error", p.stage_name(st.stage), st.detail)
        raise SGEMMError(f"prometheus reactor runtime sgemm failed: {result.status}", result)
    result.status = p.RunStatus("ok")
    result.correctness = compare_against_oracle(reference, actual)
    if not result.correctness.passed:
        raise SGEMMError(f"correctness gate failed for backend={result.used_backend}", result, actual)
    return actual, result


def run_sgemm(req: SGEMMRequest) -> SGEMMRunResult:
    """runtime.go:105-108 (RunSGEMM)."""
    return _run_sgemm_with_output(req)[1]


def run_sgemm_with_output(req: SGEMMRequest) -> Tuple[np.ndarray, SGEMMRunResult]:
    """runtime.go:121 (runSGEMMWithOutput): the flat [m*n] float32 output and the run record."""
    out, result = _run_sgemm_with_output(req)
    return out, result


def run_compiled_matmul_mm(left: Sequence[Sequence[float]],
                           right: Sequence[Sequence[float]]) -> Tuple[List[List[float]], SGEMMRunResult]:
    """runtime.go:110-119 (RunCompiledMatMulMM): float64 rows in, float64 rows out,
    through the float32 flattening of compiledMatMulRequest (runtime.go:251-306)."""
    try:
        m, n, k, a, b = p.compiled_matmul_request(left, right)
    except ValueError as exc:
        result = SGEMMRunResult(requested_backend=BACKEND_PROMETHEUS, used_backend=BACKEND_PROMETHEUS,
                                status=p.RunStatus("error", "init", -2))
        raise SGEMMError(str(exc), result) from exc
    out, result = _run_sgemm_with_output(SGEMMRequest(BACKEND_PROMETHEUS, Shape(m, n, k), a, b))
    return out.reshape(m, n).astype(np.float64).tolist(), result


def run_starter_corpus(backend: str) -> List[SGEMMRunResult]:
    """runtime.go:91-103 (RunStarterCorpus): the five starter shapes on deterministic operands."""
    runs: List[SGEMMRunResult] = []
    for shape in STARTER_CORPUS:
        a = deterministic_matrix(shape.m, shape.k)
        b = deterministic_matrix(shape.k, shape.n)
        try:
            runs.append(run_sgemm(SGEMMRequest(backend, shape, a, b)))
        except SGEMMError as exc:
            runs.append(exc.result)
            exc.runs = runs  # type: ignore[attr-defined]  (the report so far, as the Go code returns it)
            raise
    return runs


# ---- Octagon reports (runtime.go:382-432, 497-566) ---------------------------
def _octagon_failing_index(index: int) -> int:
    """runtime.go:427-432: no failing element is written as 0."""
    return 0 if index < 0 else index


def _correctness_fields(c: CorrectnessResult) -> list:
    return [("CorrectnessPass", bool(c.passed)), ("MaxAbsError", float(c.max_abs_error)),
            ("MaxRelError", float(c.max_rel_error)), ("FailingElementCount", int(c.failing_count)),
            ("FirstFailingIndex", _octagon_failing_index(int(c.first_failing_index))),
            ("FirstExpectedValue", float(c.first_expected_value)),
            ("FirstActualValue", float(c.first_actual_value))]


def report_to_octagon(runs: Sequence[SGEMMRunResult]) -> octagon.Record:
    """runtime.go:386-425 (reportToOctagon): a PrometheusSgemmReport of one
    PrometheusSgemmRun record per run, fields in the reference's order."""
    records = []
    for r in runs:
        records.append(octagon.Record("PrometheusSgemmRun", [
            ("BackendRequested", r.requested_backend), ("BackendUsed", r.used_backend),
            ("M", int(r.shape.m)), ("N", int(r.shape.n)), ("K", int(r.shape.k)),
            ("Status", str(r.status)), ("DetailCode", int(r.detail_code)), ("DetailName", r.detail_name),
            *_correctness_fields(r.correctness),
            ("CPUTimeNs", int(r.cpu_time_ns)), ("VulkanTimeNs", int(r.vulkan_time_ns)), ("VulkanEnv", r.vulkan_env),
            ("TimingMode", r.timing_mode), ("WallTimeNs", int(r.wall_time_ns)), ("Notes", r.notes)]))
    return octagon.Record("PrometheusSgemmReport", [("Runs", records)])


def write_octagon_report(path: str, runs: Sequence[SGEMMRunResult], prefix: str = "") -> str:
    """runtime.go:382-384 (WriteOctagonReport)."""
    return octagon.write(path, report_to_octagon(runs), prefix)


_ASYNC_LIFECYCLE = {0: "idle", 1: "submitted", 2: "ready", 3: "failed", 4: "consumed"}


def async_lifecycle_name(state: int) -> str:
    """runtime.go:497-512."""
    return _ASYNC_LIFECYCLE.get(state, f"state_{state}")


@dataclass
class AsyncValidationResult:
    """runtime.go:60-81 (AsyncValidationResult), as ValidateAsyncSGEMMOnHardware
    initialises it (runtime.go:585-596)."""

    shape: Shape
    requested_backend: str = BACKEND_PROMETHEUS
    used_backend: str = BACKEND_PROMETHEUS
    outcome: str = "error(init,-2)"
    environment: str = "not_applicable"
    submit_stage: str = "unknown"
    submit_detail_code: int = 0
    submit_detail_name: str = "not_applicable"
    query_lifecycle: str = "idle"
    query_ready: bool = False
    query_failed: bool = False
    query_consumed: bool = False
    query_outstanding: int = 0
    query_attempts: int = 0
    consume_stage: str = "unknown"
    consume_detail_code: int = 0
    consume_detail_name: str = "not_applicable"
    correctness: CorrectnessResult = field(default_factory=CorrectnessResult)
    wall_time_ns: int = 0
    notes: str = ""


class AsyncValidationError(RuntimeError):
    """An error return of ValidateAsyncSGEMMOnHardware; ``result`` is the record so far."""

    def __init__(self, message: str, result: AsyncValidationResult):
        super().__init__(message)
        self.result = result


def validate_async_sgemm_on_hardware(shape: Shape) -> AsyncValidationResult:
    """runtime.go:585-658 (ValidateAsyncSGEMMOnHardware): one async SGEMM on
    deterministic operands through submit, up to 2000 queries, consume, and
    the correctness gate against the fp32 CPU reference.  Without a reactor
    the result is ``skipped(prometheus_unavailable)`` (no error); a failed
    step raises AsyncValidationError carrying the record."""
    res = AsyncValidationResult(shape=shape)
    a = deterministic_matrix(shape.m, shape.k)
    b = deterministic_matrix(shape.k, shape.n)
    reference, _ = _timed_cpu_sgemm(shape.m, shape.n, shape.k, a.reshape(-1), b.reshape(-1))
    try:
        rt = new_native_runtime()
    except p.ReactorIssue as exc:
        res.used_backend = BACKEND_CPU
        res.environment = "unavailable"
        res.outcome = "skipped(prometheus_unavailable)"
        res.notes = str(exc)
        return res
    with rt:
        res.environment = rt.environment()
        t0 = time.perf_counter_ns()
        rc, task, st = rt.submit_async(shape.m, shape.n, shape.k, a, b)
        res.wall_time_ns = time.perf_counter_ns() - t0
        res.submit_stage = p.stage_name(st.stage)
        res.submit_detail_code = st.detail
        res.submit_detail_name = detail_code_name(st.detail)
        if rc != p.PROM_OK:
            res.outcome = f"error({res.submit_stage},{st.detail})"
            raise AsyncValidationError(f"async submit failed: stage={res.submit_stage} detail={st.detail}", res)
        last = None
        for attempt in range(1, 2001):
            qrc, last = rt.query_async(task)
            res.query_attempts = attempt
            if qrc != p.PROM_OK:
                res.outcome = "error(query,-1)"
                raise AsyncValidationError(f"async query failed with status {qrc}", res)
            res.query_lifecycle = async_lifecycle_name(last.lifecycle_state)
            res.query_ready = bool(last.ready)
            res.query_failed = bool(last.failed)
            res.query_consumed = bool(last.consumed)
            res.query_outstanding = int(last.outstanding_tasks)
            if last.lifecycle_state in (2, 3):
                break
        if last is None or last.lifecycle_state != 2:
            detail = last.detail_code if last is not None else 0
            res.outcome = f"error(query,{detail})"
            res.notes = "async task did not reach ready state"
            raise AsyncValidationError(f"async task did not reach ready state: lifecycle={res.query_lifecycle} "
                                       f"detail={detail}", res)
        out = np.zeros(shape.m * shape.n, dtype=np.float32)
        crc, cst = rt.consume_async(task, out)
        res.consume_stage = p.stage_name(cst.stage)
        res.consume_detail_code = cst.detail
        res.consume_detail_name = detail_code_name(cst.detail)
        if crc != p.PROM_OK:
            res.outcome = f"error({res.consume_stage},{cst.detail})"
            raise AsyncValidationError(f"async consume failed: stage={res.consume_stage} detail={cst.detail}", res)
    res.correctness = compare_against_oracle(reference, out)
    if not res.correctness.passed:
        res.outcome = "error(correctness,-1)"
        raise AsyncValidationError("async correctness gate failed", res)
    res.outcome = "ok"
    return res


def async_validation_to_octagon(r: AsyncValidationResult) -> octagon.Record:
    """runtime.go:525-566 (asyncValidationToOctagon)."""
    return octagon.Record("PrometheusAsyncValidation", [
        ("BackendRequested", r.requested_backend), ("BackendUsed", r.used_backend),
        ("M", int(r.shape.m)), ("N", int(r.shape.n)), ("K", int(r.shape.k)),
        ("Outcome", r.outcome), ("Environment", r.environment),
        ("SubmitStage", r.submit_stage), ("SubmitDetailCode", int(r.submit_detail_code)),
        ("SubmitDetailName", r.submit_detail_name),
        ("QueryLifecycle", r.query_lifecycle), ("QueryReady", r.query_ready), ("QueryFailed", r.query_failed),
        ("QueryConsumed", r.query_consumed), ("QueryOutstanding", int(r.query_outstanding)),
        ("QueryAttempts", int(r.query_attempts)),
        ("ConsumeStage", r.consume_stage), ("ConsumeDetailCode", int(r.consume_detail_code)),
        ("ConsumeDetailName", r.consume_detail_name),
        *_correctness_fields(r.correctness),
        ("WallTimeNs", int(r.wall_time_ns)), ("Notes", r.notes)])


def write_async_validation_octagon(path: str, result: AsyncValidationResult, prefix: str = "") -> str:
    """runtime.go:521-523 (WriteAsyncValidationOctagon)."""
    return octagon.write(path, async_validation_to_octagon(result), prefix)
