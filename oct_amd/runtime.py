"""The non-strict SGEMM path of Oct's Prometheus package.

Mirrors ``internal/prometheus/runtime.go:12-376``: ``RunSGEMM``,
``RunCompiledMatMulMM`` and ``RunStarterCorpus`` over ``runSGEMMWithOutput``.
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
    """runtime.go:30-38."""

    passed: bool = True
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
    res = CorrectnessResult()
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
