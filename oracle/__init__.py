"""ctypes wrapper of the CPU oracle ``oracle/liboct_oracle.so``.

TEST INFRASTRUCTURE ONLY: the parity checker.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this package; the reactor never does.  The C sources cite the reference
file:line each function restates (``oracle/oct_oracle.c``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, Structure, c_double, c_float, c_int32, c_int64, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboct_oracle.so"


class OctCorrectness(Structure):
    _fields_ = [
        ("pass_", c_int32),
        ("failing_count", c_int32),
        ("first_failing_index", c_int64),
        ("max_abs_error", c_double),
        ("max_rel_error", c_double),
        ("first_expected", c_float),
        ("first_actual", c_float),
    ]


class OctReductionMismatch(Structure):
    _fields_ = [
        ("row", c_uint32),
        ("column", c_uint32),
        ("expected", c_float),
        ("actual", c_float),
        ("absolute_error", c_float),
        ("relative_error", c_float),
    ]


_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        L = ctypes.CDLL(str(LIB_PATH))
        P = c_void_p
        sig = {
            "oct_gen_uniform_f32": (None, [c_uint64, P, c_uint64, c_float, c_float]),
            "oct_gen_normal_f32": (None, [c_uint64, P, c_uint64, c_float, c_float]),
            "oct_deterministic_matrix": (None, [P, c_uint64]),
            "oct_concept_sgemm_matrix": (None, [P, c_uint32, c_uint32]),
            "oct_reduction_deterministic_input": (None, [P, c_uint32, c_uint32, c_float]),
            "oct_f32_to_bf16": (c_uint16, [c_float]),
            "oct_bf16_to_f32": (c_float, [c_uint16]),
            "oct_f32_to_bf16_array": (None, [P, P, c_uint64]),
            "oct_bf16_to_f32_array": (None, [P, P, c_uint64]),
            "oct_matmul_f64": (None, [P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32]),
            "oct_matmul_f32in_f64": (None, [P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32]),
            "oct_matmul_bf16in_f64": (None, [P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32]),
            "oct_matmul_compiled_f64": (None, [P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32]),
            "oct_cpu_sgemm_f32": (None, [P, P, P, c_uint32, c_uint32, c_uint32]),
            "oct_compare_against_oracle": (None, [P, P, c_uint64, POINTER(OctCorrectness)]),
            "oct_normwise_rel_err": (c_double, [P, P, c_uint64]),
            "oct_normwise_rel_err_f32": (c_double, [P, P, c_uint64]),
            "oct_reduction_cpu_reference": (c_int32, [P, P, c_uint32, c_uint32, c_uint32]),
            "oct_reduction_compare": (c_int32, [c_uint32, c_uint32, c_uint32, P, P, POINTER(OctReductionMismatch)]),
            "oct_rmsnorm_cpu_reference": (c_int32, [P, P, P, P, c_uint32, c_uint32, c_uint32, c_float]),
            "oct_fft64_roots": (None, [P, c_uint32]),
            "oct_fft64_with_roots": (None, [P, P, P, c_uint32]),
            "oct_fft64": (c_int32, [P, P, P, c_uint32]),
            "oct_fft64_agrees": (c_int32, [P, P, c_uint32]),
            "oct_dft_c32": (None, [P, P, c_uint32, c_uint32, c_uint32, c_int32]),
            "oct_m1_rmsnorm": (None, [P, c_uint32, P, P, P, c_uint32, c_uint32, c_float, c_int32, c_int32]),
            "oct_m1_head_rmsnorm_go": (None, [P, P, P, c_uint32, c_uint32, c_float]),
            "oct_m1_rope": (None, [P, P, P, P, c_uint32, c_uint32, c_uint32]),
            "oct_m1_raw_scores": (None, [P, P, P, c_uint32, c_uint32, c_uint32, c_float]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _p(a):
    return None if a is None else a.ctypes.data


def default_threads() -> int:
    # The GPU box shares 16 cores per GPU; this container has 8.
    return max(1, min(16, os.cpu_count() or 1))


# ---- generators ---------------------------------------------------------------
def uniform(seed: int, shape, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().oct_gen_uniform_f32(seed, _p(out), out.size, lo, hi)
    return out


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().oct_gen_normal_f32(seed, _p(out), out.size, mean, std)
    return out


def deterministic_matrix(rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    lib().oct_deterministic_matrix(_p(out), out.size)
    return out


def concept_sgemm_matrix(count: int, seed: int) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib().oct_concept_sgemm_matrix(_p(out), count, seed)
    return out


def reduction_input(rows: int, width: int, bias: float = 0.0) -> np.ndarray:
    out = np.empty((rows, width), dtype=np.float32)
    lib().oct_reduction_deterministic_input(_p(out), rows, width, bias)
    return out


def to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oct_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def from_bf16(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().oct_bf16_to_f32_array(_p(bits), _p(out), bits.size)
    return out


# ---- `@` ---------------------------------------------------------------------
def matmul_f64(a: np.ndarray, b: np.ndarray, rows=None, threads=None) -> np.ndarray:
    """Oct's `@` (interpret.go:6278-6305) on float64 or fp32 operands; rows=(begin,end)."""
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    out = np.zeros((m, n), dtype=np.float64)
    rb, re = rows if rows else (0, m)
    t = threads or default_threads()
    if a.dtype == np.float64:
        a = np.ascontiguousarray(a)
        b = np.ascontiguousarray(b, dtype=np.float64)
        lib().oct_matmul_f64(_p(a), _p(b), _p(out), m, n, k, rb, re, t)
    elif a.dtype == np.uint16:
        a = np.ascontiguousarray(a)
        b = np.ascontiguousarray(b, dtype=np.uint16)
        lib().oct_matmul_bf16in_f64(_p(a), _p(b), _p(out), m, n, k, rb, re, t)
    else:
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        lib().oct_matmul_f32in_f64(_p(a), _p(b), _p(out), m, n, k, rb, re, t)
    return out


def matmul_compiled_f64(a: np.ndarray, b: np.ndarray, rows=None) -> np.ndarray:
    """__octMatMulMM (emit_go_runtime.go:168-205), single thread."""
    a = np.ascontiguousarray(a, dtype=np.float64)
    b = np.ascontiguousarray(b, dtype=np.float64)
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), dtype=np.float64)
    rb, re = rows if rows else (0, m)
    lib().oct_matmul_compiled_f64(_p(a), _p(b), _p(out), m, n, k, rb, re)
    return out


def cpu_sgemm_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), dtype=np.float32)
    lib().oct_cpu_sgemm_f32(_p(a), _p(b), _p(out), m, n, k)
    return out


def compare_against_oracle(expected: np.ndarray, actual: np.ndarray) -> OctCorrectness:
    e = np.ascontiguousarray(expected, dtype=np.float32).reshape(-1)
    a = np.ascontiguousarray(actual, dtype=np.float32).reshape(-1)
    res = OctCorrectness()
    lib().oct_compare_against_oracle(_p(e), _p(a), e.size, ctypes.byref(res))
    return res


def normwise_rel_err(actual: np.ndarray, expected: np.ndarray) -> float:
    a = np.ascontiguousarray(actual, dtype=np.float32).reshape(-1)
    if expected.dtype == np.float64:
        e = np.ascontiguousarray(expected).reshape(-1)
        return lib().oct_normwise_rel_err(_p(a), _p(e), a.size)
    e = np.ascontiguousarray(expected, dtype=np.float32).reshape(-1)
    return lib().oct_normwise_rel_err_f32(_p(a), _p(e), a.size)


# ---- reductions -------------------------------------------------------------
def reduction_reference(x: np.ndarray, operation: int):
    """Returns (detail, output) of prom_reduction_cpu_reference (fused_reduction.c:996-1036)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, width = x.shape
    out = np.zeros((rows, width) if operation == 3 else (rows,), dtype=np.float32)
    d = lib().oct_reduction_cpu_reference(_p(x), _p(out), rows, width, operation)
    return d, out


def reduction_compare(x_shape, operation: int, expected: np.ndarray, actual: np.ndarray):
    rows, width = x_shape
    e = np.ascontiguousarray(expected, dtype=np.float32)
    a = np.ascontiguousarray(actual, dtype=np.float32)
    mm = OctReductionMismatch()
    rc = lib().oct_reduction_compare(rows, width, operation, _p(e), _p(a), ctypes.byref(mm))
    return rc, mm


def rmsnorm_reference(z: np.ndarray, w: np.ndarray, eps: float, width=None):
    z = np.ascontiguousarray(z, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    tokens, stride = z.shape
    width = width or w.size
    y = np.zeros((tokens, width), dtype=np.float32)
    inv = np.zeros(tokens, dtype=np.float32)
    rc = lib().oct_rmsnorm_cpu_reference(_p(z), _p(w), _p(y), _p(inv), tokens, width, stride, eps)
    return rc, y, inv


# ---- FFT (internal/fft/fft.go) --------------------------------------------------
def fft64_roots(n: int) -> np.ndarray:
    """fft.go:218-226: the n/2 twiddles cos(a) + i sin(a), a = -2*pi/n * j."""
    tw = np.zeros(max(1, n // 2), dtype=np.complex128)
    lib().oct_fft64_roots(_p(tw), n)
    return tw[: n // 2]


def fft64(x) -> np.ndarray:
    """fft.go:206-258 restated in C: forward, unnormalised, binary64."""
    x = np.ascontiguousarray(x, dtype=np.complex128)
    n = x.size
    out = np.zeros(n, dtype=np.complex128)
    scratch = np.zeros(max(1, n), dtype=np.float64)
    if lib().oct_fft64(_p(x), _p(out), _p(scratch), n) != 0:
        raise ValueError("FFT requires a non-empty power-of-two length")
    return out


def dft_c32(x, n: int, batch: int = 1, stride: int = 0, inverse: bool = False) -> np.ndarray:
    """reactor_fft_api_tests.cpp:525-553 restated in C: direct binary64 DFT of
    ``batch`` complex64 sequences of ``n`` points ``stride`` apart (0:
    contiguous), divided by n for the inverse, rounded to complex64; the
    padding between batches is the input's."""
    x = np.ascontiguousarray(x, dtype=np.complex64)
    stride = stride or n
    if n < 1 or batch < 1 or stride < n or x.size < (batch - 1) * stride + n:
        raise ValueError("invalid batched DFT shape")
    out = np.zeros_like(x)
    lib().oct_dft_c32(_p(x), _p(out), n, batch, stride, 1 if inverse else 0)
    return out


def fft64_agrees(reference, actual) -> bool:
    """fft.go:176-192: |actual - reference| <= 1e-12 * max|reference| per component."""
    r = np.ascontiguousarray(reference, dtype=np.complex128)
    a = np.ascontiguousarray(actual, dtype=np.complex128)
    if r.size != a.size:
        return False
    return bool(lib().oct_fft64_agrees(_p(r), _p(a), r.size))


# ---- Gemma-4-E2B M1 stages (oct_oracle_m1.c) -----------------------------------------
def m1_rmsnorm(x, w, eps: float = 1e-6, round_in: bool = False, round_out: bool = False, width=None):
    """Double-sum RMSNorm of rows of x (row pitch = x.shape[1]); returns (y, inv_rms)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, stride = x.shape
    width = width or w.size
    y = np.zeros((rows, width), np.float32)
    inv = np.zeros(rows, np.float32)
    lib().oct_m1_rmsnorm(_p(x), stride, _p(w), _p(y), _p(inv), rows, width, eps, int(round_in), int(round_out))
    return y, inv


def m1_head_rmsnorm_go(x, w, eps: float = 1e-6):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, width = x.shape
    y = np.zeros_like(x)
    lib().oct_m1_head_rmsnorm_go(_p(x), _p(w), _p(y), rows, width, eps)
    return y


def m1_rope(source, cosine, sine, tokens: int = 15, heads: int = 8, width: int = 256):
    s = np.ascontiguousarray(source, dtype=np.float32).reshape(-1)
    c = np.ascontiguousarray(cosine, dtype=np.float32).reshape(-1)
    n = np.ascontiguousarray(sine, dtype=np.float32).reshape(-1)
    out = np.zeros_like(s)
    lib().oct_m1_rope(_p(s), _p(c), _p(n), _p(out), tokens, heads, width)
    return out


def m1_raw_scores(query, key, tokens: int = 15, query_heads: int = 8, width: int = 256, scale: float = 0.0625):
    q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
    k = np.ascontiguousarray(key, dtype=np.float32).reshape(-1)
    out = np.zeros(query_heads * tokens * tokens, np.float32)
    lib().oct_m1_raw_scores(_p(q), _p(k), _p(out), tokens, query_heads, width, scale)
    return out


def m1_positional(x, w, cosine, sine, heads: int):
    """Head RMSNorm (BF16 in and out) then RoPE: the head_rmsnorm_rope chain."""
    y, _ = m1_rmsnorm(np.asarray(x, np.float32).reshape(15 * heads, 256), w, 1e-6, True, True)
    return m1_rope(y, cosine, sine, 15, heads, 256)
