"""Where Oct sends a matrix product: the PROMETHEUS strict-dispatch decisions.

Oct decides in two places whether a product runs through the strict GPU path.
This module makes the same decisions with the same error texts; the bridge it
hands over to is ``oct_amd.prometheus.run_compiled_matmul_mm_strict``
(strict.go:11-32) or ``oct_amd.runtime.run_compiled_matmul_mm``
(runtime.go:110-119).

* Interpreter (``internal/interpret``).  Inside a ``PROMETHEUS`` block,
  ``Matrix @ Matrix`` and ``PrometheusMatMul(a, b)`` call the strict hook;
  outside it, ``@`` is the interpreter's ordinary binary evaluation and
  ``PrometheusMatMul`` its CPU ``evalMatrixMultiply`` (interpret.go:1403-1405,
  2113-2117, 4643-4675).  The hook is a process-wide function that the native
  host installs at start-up (interpret/prometheus.go:5-14, strict.go:35-73);
  without it the strict path fails, it never falls back.
* Compiler (``internal/build``).  Lowering picks the MIR callee
  (lower_expr.go:184-200, 544-570) and code generation turns the two
  PROMETHEUS callees into calls of runtime functions that print a status line
  and panic on failure (emit_go.go:1920-1923, emit_go_runtime.go:788-807).

The CPU evaluation outside ``PROMETHEUS`` belongs to the caller's interpreter:
the functions here take it as a callable and never compute a product
themselves.

The ``FFT`` builtin is routed the same way in both lanes: inside
``PROMETHEUS`` the engine must run it on the GPU, outside it selects by
measurement (``oct_amd.fft_engine``).  Unlike a strict product, an FFT
failure is a recoverable Oct error value, not a terminal runtime error
(interpret.go:3464-3486, emit_go_runtime.go:715-721).
"""
from __future__ import annotations

import sys
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence, TextIO, Tuple

import numpy as np

from . import fft_engine as fe
from . import prometheus as p
from . import runtime as rt

# interpret.Value kinds that matter here (interpret.go:187-191).
VALUE_INT = "Int"
VALUE_FLOAT = "Float"
VALUE_MATRIX = "Matrix"
VALUE_COMPLEX = "Complex"
VALUE_ARRAY = "Array"


@dataclass
class Value:
    """A boxed interpreter value: a scalar, a complex number, an array of
    values or a row-major matrix of values."""

    kind: str
    number: float = 0.0
    matrix: Optional["MatrixValue"] = None
    complex_value: complex = 0j
    array: Optional[List["Value"]] = None


@dataclass
class MatrixValue:
    rows: int
    cols: int
    elements: List[Value] = field(default_factory=list)


class StrictDispatchError(RuntimeError):
    """An error the reference returns from the dispatch (not from the bridge)."""


def float_matrix(rows: Sequence[Sequence[float]]) -> Value:
    """A Matrix<Float> value from rows (the hook's result, strict.go:66-72)."""
    n_rows = len(rows)
    n_cols = len(rows[0]) if n_rows else 0
    elements = [Value(VALUE_FLOAT, float(x)) for row in rows for x in row]
    return Value(VALUE_MATRIX, matrix=MatrixValue(n_rows, n_cols, elements))


def _float_rows(value: Value) -> List[List[float]]:
    """strict.go:37-53: a Matrix whose every element is a Float, as rows."""
    if value.kind != VALUE_MATRIX or value.matrix is None:
        raise StrictDispatchError("PROMETHEUS matrix execution requires Matrix<Float>")
    mat = value.matrix
    rows = []
    for r in range(mat.rows):
        row = []
        for c in range(mat.cols):
            entry = mat.elements[r * mat.cols + c]
            if entry.kind != VALUE_FLOAT:
                raise StrictDispatchError("PROMETHEUS matrix execution requires Matrix<Float>")
            row.append(entry.number)
        rows.append(row)
    return rows


# ---- the hook (interpret/prometheus.go:5-14, strict.go:35-73) ---------------
StrictMatMul = Callable[[Value, Value], Value]
_strict_hook: Optional[StrictMatMul] = None


def set_strict_prometheus_matmul(hook: Optional[StrictMatMul]) -> None:
    """Install (or, with None, remove) the process-wide strict hook."""
    global _strict_hook
    _strict_hook = hook


def strict_prometheus_matmul(left: Value, right: Value) -> Value:
    """interpret/prometheus.go:9-14: the hook, or an error when none is installed."""
    if _strict_hook is None:
        raise StrictDispatchError("PROMETHEUS requires GPU matrix execution: backend unavailable")
    return _strict_hook(left, right)


def gpu_strict_matmul(left: Value, right: Value) -> Value:
    """The hook the native host installs (strict.go:35-73): Matrix<Float>
    operands to rows, the strict GPU product, rows back to a Matrix<Float>.
    Bridge failures propagate unchanged."""
    a = _float_rows(left)
    b = _float_rows(right)
    out, _env = p.run_compiled_matmul_mm_strict(a, b)
    return float_matrix(out)


def install_strict_hook() -> None:
    """strict.go:35's init(): make the reactor the strict backend."""
    set_strict_prometheus_matmul(gpu_strict_matmul)


# ---- interpreter decisions (interpret.go) -----------------------------------
BinaryEval = Callable[[str, Value, Value], Value]
MatMulEval = Callable[[Value, Value], Value]


def eval_binary(in_prometheus: bool, operator: str, left: Value, right: Value, evaluate: BinaryEval) -> Value:
    """interpret.go:2113-2117: a PROMETHEUS block's ``Matrix @ Matrix`` goes to
    the strict hook; everything else to the interpreter's own ``evaluate``."""
    if in_prometheus and operator == "@" and left.kind == VALUE_MATRIX and right.kind == VALUE_MATRIX:
        return strict_prometheus_matmul(left, right)
    return evaluate(operator, left, right)


def eval_prometheus_matmul_call(in_prometheus: bool, type_arguments: Sequence[str], arguments: Sequence[Value],
                                multiply: MatMulEval) -> Value:
    """interpret.go:4643-4675, with the arguments already evaluated in order.

    Inside PROMETHEUS the call is strict; outside it is ``multiply``
    (the interpreter's evalMatrixMultiply)."""
    if type_arguments:
        raise StrictDispatchError("runtime invariant violation: PrometheusMatMul does not accept type arguments")
    if len(arguments) != 2:
        raise StrictDispatchError("runtime invariant violation: PrometheusMatMul expects 2 arguments")
    left, right = arguments
    if left.kind != VALUE_MATRIX or right.kind != VALUE_MATRIX:
        raise StrictDispatchError("runtime invariant violation: PrometheusMatMul expects matrix arguments")
    if in_prometheus:
        return strict_prometheus_matmul(left, right)
    return multiply(left, right)


@dataclass
class EvalResult:
    """An evaluation's outcome: a value, or a recoverable Oct error value
    (the interpreter's ``evalResult{hasError, errorVal}``)."""

    value: Optional[Value] = None
    error: Optional[str] = None


def complex_array(values) -> Value:
    """A Complex[] value."""
    return Value(VALUE_ARRAY, array=[Value(VALUE_COMPLEX, complex_value=complex(z)) for z in values])


def eval_fft_call(engine: "fe.FFTEngine", in_prometheus: bool, type_arguments: Sequence[str],
                  arguments: Sequence[Value]) -> EvalResult:
    """interpret.go:3464-3486 with the argument evaluated, and
    interpret/fft.go:10-29: the Complex[] argument goes to the engine in
    binary64, GPU-required inside PROMETHEUS; an engine error (validation,
    GPU unavailable or failed) becomes a recoverable error value."""
    if type_arguments:
        raise StrictDispatchError("runtime invariant violation: FFT does not accept type arguments")
    if len(arguments) != 1:
        raise StrictDispatchError("runtime invariant violation: FFT expects 1 argument")
    argument = arguments[0]
    if argument.kind != VALUE_ARRAY or argument.array is None:
        raise StrictDispatchError("runtime invariant violation: FFT expects Complex[] argument")
    values = np.empty(len(argument.array), dtype=np.complex128)
    for index, entry in enumerate(argument.array):
        if entry.kind != VALUE_COMPLEX:
            raise StrictDispatchError("runtime invariant violation: FFT expects Complex[] input")
        values[index] = entry.complex_value
    try:
        out = engine.transform(values, required_gpu=in_prometheus)
    except fe.FFTError as exc:
        return EvalResult(error=str(exc))
    return EvalResult(value=complex_array(out))


# ---- compiler decisions (internal/build) ------------------------------------
def parse_matrix_elem_type(type_name: str) -> Optional[str]:
    """lower_expr.go:3154-3156: ``Matrix<E>`` -> ``E``, else None."""
    prefix = "Matrix<"
    if type_name.startswith(prefix) and type_name.endswith(">") and len(type_name) > len(prefix) + 1:
        return type_name[len(prefix):-1]
    return None


def unify_linear_elem_type(left_elem: str, right_elem: str) -> str:
    """lower_expr.go:3230-3241: a unit-carrying Float wins, then Float, else the left type."""
    if left_elem.startswith("Float<") or right_elem.startswith("Float<"):
        return left_elem if left_elem.startswith("Float<") else right_elem
    if left_elem == "Float" or right_elem == "Float":
        return "Float"
    return left_elem


def lower_matmul_operator(in_prometheus: bool, left_type: str, right_type: str) -> Tuple[str, str]:
    """lower_expr.go:184-200 for ``Matrix<L> @ Matrix<R>``: (callee, result type).

    Inside PROMETHEUS both operands must be exactly Matrix<Float> (a unit
    type such as Float<m> is refused) and the callee is the strict one."""
    left_elem = parse_matrix_elem_type(left_type)
    right_elem = parse_matrix_elem_type(right_type)
    if left_elem is None or right_elem is None:
        raise StrictDispatchError(f"matrix product needs Matrix operands, got {left_type} @ {right_type}")
    ret = f"Matrix<{unify_linear_elem_type(left_elem, right_elem)}>"
    callee = "MatMulMM"
    if in_prometheus:
        if left_elem != "Float" or right_elem != "Float":
            raise StrictDispatchError("PROMETHEUS matrix execution requires Matrix<Float>")
        callee = "PrometheusMatMulMMStrict"
    return callee, ret


def lower_prometheus_matmul_call(in_prometheus: bool, argument_types: Sequence[str]) -> Tuple[str, str]:
    """lower_expr.go:544-570 for ``PrometheusMatMul(a, b)``: (callee, result type)."""
    if len(argument_types) != 2:
        raise StrictDispatchError("PrometheusMatMul expects 2 arguments")
    if argument_types[0] != "Matrix<Float>" or argument_types[1] != "Matrix<Float>":
        raise StrictDispatchError("PrometheusMatMul expects Matrix<Float> arguments")
    return ("PrometheusMatMulMMStrict" if in_prometheus else "PrometheusMatMulMM"), "Matrix<Float>"


def oct_prometheus_matmul_mm_strict(left: Sequence[Sequence[float]], right: Sequence[Sequence[float]],
                                    log: Optional[TextIO] = None) -> List[List[float]]:
    """emit_go_runtime.go:788-794 (``__octPrometheusMatMulMMStrict``): the
    strict product, one status line, and any failure raised (Go panics)."""
    out, env = p.run_compiled_matmul_mm_strict(left, right)
    print("backend_requested=prometheus backend_used=prometheus status=ok detail_code=0 detail_name=gpu "
          f"vulkan_env={env}", file=log or sys.stdout, flush=True)
    return out


def oct_prometheus_matmul_mm(left: Sequence[Sequence[float]], right: Sequence[Sequence[float]],
                             log: Optional[TextIO] = None) -> List[List[float]]:
    """emit_go_runtime.go:795-807 (``__octPrometheusMatMulMM``): the non-strict
    product (CPU reference, reactor or truthful fallback, correctness gate),
    its status line, and a failure raised after the line is printed."""
    err: Optional[Exception] = None
    out: List[List[float]] = []
    try:
        out, run = rt.run_compiled_matmul_mm(left, right)
    except rt.SGEMMError as exc:
        err, run = exc, exc.result
    print(f"backend_requested={run.requested_backend} backend_used={run.used_backend} status={run.status} "
          f"correctness={'true' if run.correctness.passed else 'false'} detail_code={run.detail_code} "
          f"detail_name={run.detail_name} vulkan_env={run.vulkan_env} wall={run.wall_time_ns}ns",
          file=log or sys.stdout, flush=True)
    if err is not None:
        raise RuntimeError(f"PrometheusMatMulMM failed: {err}") from err
    return out


def lower_fft_call(in_prometheus: bool, argument_types: Sequence[str]) -> Tuple[str, str]:
    """lower_expr.go:2598-2603 and 3320-3327 for ``FFT(x)``: (callee, result
    type); the GPU-required callee inside PROMETHEUS."""
    if len(argument_types) != 1:
        raise StrictDispatchError(f"function 'FFT' expects 1 arguments, got {len(argument_types)}")
    if argument_types[0] != "Complex[]":
        raise StrictDispatchError(f"compiled mode does not yet support builtin FFT for type {argument_types[0]}")
    return ("FFTGPU" if in_prometheus else "FFT"), "Complex[]"


@dataclass
class ComplexSliceResult:
    """The compiled program's ``octResult_ComplexSlice``."""

    value: Optional[np.ndarray] = None
    err: str = ""
    is_err: bool = False


def new_fft_engine() -> "fe.FFTEngine":
    """internal/prometheus/fft.go:19 (``NewFFTEngine``): the compiled
    program's one engine, closed when its main returns (emit_go.go:793-794)."""
    return fe.FFTEngine()


def oct_fft(engine: "fe.FFTEngine", values, required_gpu: bool) -> ComplexSliceResult:
    """emit_go_runtime.go:715-721 (``__octFFT``): the engine's result or its
    error as a recoverable result value."""
    try:
        return ComplexSliceResult(value=engine.transform(values, required_gpu))
    except fe.FFTError as exc:
        return ComplexSliceResult(err=str(exc), is_err=True)
