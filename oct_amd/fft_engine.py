"""Oct's binary64 FFT engine with the reactor as its GPU backend.

Mirrors ``internal/fft/fft.go:13-258`` (the engine: validation, strict and
automatic execution, measured backend selection, the CPU transform) and
``internal/prometheus/fft.go:1-55`` (the backend: a runtime that must be on
a hardware GPU, calling ``prometheus_reactor_runtime_fft64``).

* ``transform(values, required_gpu=True)`` (a ``PROMETHEUS`` block) runs on
  the reactor or raises ``"PROMETHEUS FFT requires GPU execution: ..."``; it
  never computes a CPU substitute.
* ``transform(values, required_gpu=False)`` selects per length: the first
  call of a length times the CPU transform (three windows of >= 10 ms),
  calls the GPU once cold and three times warm, checks every GPU result
  against the CPU one (1e-12 of the largest component, fft.go:177-194), and
  keeps the GPU only if its warm call beats 4/5 of the CPU's; later calls of
  that length use the choice (a failed GPU call falls back to the CPU and
  says why in ``measurement()``).

The CPU transform is fft.go's radix-2 decimation in time with its twiddles
cos(a) + i sin(a), a = -2*pi/n*j, in binary64 with each product and sum
rounded separately (no fused multiply-add), as the reference's CPU path
computes it.  It is part of this contract (automatic mode's result when the
CPU is selected, and the calibration reference), not a fallback of the
reactor: the reactor's FFT has none.
"""
from __future__ import annotations

import math
import threading
import time
from dataclasses import dataclass
from typing import Callable, Optional, Tuple

import numpy as np

from . import prometheus as p
from . import runtime as rt

MAX_GPU_ELEMENTS = 1 << 20


class FFTError(RuntimeError):
    """An error the engine returns (the reference's error text)."""


@dataclass
class Measurement:
    """fft.go:22-29."""

    elements: int = 0
    selected: str = ""
    reason: str = ""
    cpu_warm_ns: int = 0
    gpu_cold_ns: int = 0
    gpu_warm_ns: int = 0


def validate(n: int) -> None:
    """fft.go:196-204."""
    if n == 0:
        raise FFTError("runtime error: FFT requires non-empty input")
    if n & (n - 1):
        raise FFTError("runtime error: FFT requires power-of-two input length")


def roots(n: int) -> np.ndarray:
    """fft.go:219-226: the n/2 twiddles cos(a) + i sin(a), a = -2*pi/n * j
    (the angle rounded as Go rounds it: (-2*pi/n) first, then times j).  The
    cosine and sine are the C library's cos and sin, two calls (math.cos and
    math.sin call them), as the reactor's host code evaluates its twiddle
    table, so this engine's CPU transform and the reactor's agree bit for bit
    where the reactor's is exact (n <= 4096).  glibc's sincos differs from
    them in the last bit for some angles."""
    step = -2.0 * math.pi / float(n)
    return np.array([complex(math.cos(step * j), math.sin(step * j)) for j in range(n // 2)], dtype=np.complex128)


def cpu_with_roots(values: np.ndarray, twiddles: np.ndarray) -> np.ndarray:
    """fft.go:228-258: bit-reversal permutation, then radix-2 stages of
    growing span; t = w * x[odd], x[even] + t, x[even] - t, with the complex
    product as (ac - bd) + (ad + bc)i, every operation rounded on its own."""
    x = np.array(values, dtype=np.complex128)
    n = x.size
    if n > 1:
        bits = n.bit_length() - 1
        idx = np.arange(n)
        rev = np.zeros(n, dtype=np.int64)
        for b in range(bits):
            rev |= ((idx >> b) & 1) << (bits - 1 - b)
        x = x[rev]
    re, im = x.real.copy(), x.imag.copy()
    wr_all, wi_all = twiddles.real, twiddles.imag
    span = 2
    while span <= n:
        half = span // 2
        w = np.arange(half) * (n // span)
        wr, wi = wr_all[w], wi_all[w]
        r = re.reshape(n // span, span)
        i = im.reshape(n // span, span)
        br, bi = r[:, half:].copy(), i[:, half:].copy()
        tr = wr * br - wi * bi
        ti = wr * bi + wi * br
        ar, ai = r[:, :half].copy(), i[:, :half].copy()
        r[:, :half] = ar + tr
        i[:, :half] = ai + ti
        r[:, half:] = ar - tr
        i[:, half:] = ai - ti
        span *= 2
    return re + 1j * im


def cpu(values) -> np.ndarray:
    """fft.go:207-209 (CPU): requires a validated length."""
    x = np.asarray(values, dtype=np.complex128)
    return cpu_with_roots(x, roots(x.size))


def agrees(reference: np.ndarray, actual: np.ndarray) -> bool:
    """fft.go:177-194: every component within 1e-12 of the reference's largest
    component (plus n smallest subnormals), nothing non-finite."""
    if reference.shape != actual.shape:
        return False
    scale = float(np.max(np.maximum(np.abs(reference.real), np.abs(reference.imag)))) if reference.size else 0.0
    tol = 1e-12 * scale + 5e-324 * reference.size
    parts = (reference.real, reference.imag, actual.real, actual.imag)
    if not all(np.all(np.isfinite(v)) for v in parts):
        return False
    return bool(np.all(np.abs(actual.real - reference.real) <= tol) and
                np.all(np.abs(actual.imag - reference.imag) <= tol))


class ReactorFFTBackend:
    """internal/prometheus/fft.go:21-48: a runtime on a hardware GPU and its
    binary64 FFT entry."""

    def __init__(self):
        self.runtime = rt.new_native_runtime()
        try:
            self.runtime.require_hardware_gpu()
            if not hasattr(self.runtime.lib, "prometheus_reactor_runtime_fft64"):
                # bridge_dlopen_linux.go:234: dlsym's error (glibc's dlerror wording)
                path = getattr(self.runtime.lib, "_oct_path", "")
                raise FFTError(f"dlsym prometheus_reactor_runtime_fft64: {path}: undefined symbol: "
                               "prometheus_reactor_runtime_fft64")
        except Exception:
            self.runtime.close()
            raise

    def transform(self, values: np.ndarray) -> np.ndarray:
        if values.size > MAX_GPU_ELEMENTS:
            raise FFTError("Vulkan FFT supports at most 1048576 complex values")
        rc, st, out = self.runtime.fft64(values)
        if rc != p.PROM_OK:
            # bridge_dlopen_linux.go:296-298
            raise FFTError(f"Vulkan FFT64 failed: status={rc} stage={st.stage} detail={st.detail}")
        return out

    def close(self) -> None:
        self.runtime.close()


def _measure(call: Callable[[], np.ndarray]) -> Tuple[np.ndarray, int]:
    """fft.go:156-170: repeat full calls until 10 ms have passed; the mean."""
    start = time.perf_counter_ns()
    count = 0
    while True:
        count += 1
        out = call()
        elapsed = time.perf_counter_ns() - start
        if elapsed >= 10_000_000:
            return out, elapsed // count


class FFTEngine:
    """internal/fft/fft.go:35-154 (Engine), scoped to a program run."""

    def __init__(self, new_backend: Optional[Callable[[], ReactorFFTBackend]] = ReactorFFTBackend):
        self._lock = threading.Lock()
        self._new_backend = new_backend
        self._backend: Optional[ReactorFFTBackend] = None
        self._attempted = False
        self._backend_err: Optional[BaseException] = None
        self._last = Measurement()
        self._roots: Optional[np.ndarray] = None

    def close(self) -> None:
        with self._lock:
            if self._backend is not None:
                self._backend.close()
                self._backend = None
            self._attempted = False
            self._last = Measurement()
            self._roots = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def measurement(self) -> Measurement:
        with self._lock:
            return Measurement(**vars(self._last))

    def _gpu(self, values: np.ndarray) -> np.ndarray:
        if not self._attempted:
            self._attempted = True
            self._backend_err = FFTError("Vulkan FFT backend unavailable")
            if self._new_backend is not None:
                try:
                    self._backend = self._new_backend()
                    self._backend_err = None
                except Exception as exc:  # the reference keeps the error and reports it on every GPU request
                    self._backend_err = exc
        if self._backend_err is not None:
            raise self._backend_err
        return self._backend.transform(values)

    def _cpu(self, values: np.ndarray) -> np.ndarray:
        if self._roots is None or self._roots.size * 2 != values.size:
            self._roots = roots(values.size)
        return cpu_with_roots(values, self._roots)

    def transform(self, values, required_gpu: bool) -> np.ndarray:
        """fft.go:80-154."""
        x = np.ascontiguousarray(values, dtype=np.complex128).reshape(-1)
        validate(x.size)
        with self._lock:
            if required_gpu:
                if self._last.elements != x.size:
                    self._last = Measurement()
                try:
                    return self._gpu(x)
                except Exception as exc:
                    raise FFTError(f"PROMETHEUS FFT requires GPU execution: {exc}") from exc
            if self._last.elements == x.size:
                if self._last.selected == "vulkan-fp64":
                    try:
                        return self._gpu(x)
                    except Exception as exc:
                        self._last.selected = "cpu"
                        self._last.reason = f"GPU execution failed: {exc}"
                return self._cpu(x)
            self._last = Measurement(elements=x.size, selected="cpu")
            cpu_times = []
            reference = None
            for _ in range(3):
                reference, ns = _measure(lambda: self._cpu(x))
                cpu_times.append(ns)
            self._last.cpu_warm_ns = sorted(cpu_times)[1]
            t0 = time.perf_counter_ns()
            try:
                candidate = self._gpu(x)
            except Exception as exc:
                self._last.gpu_cold_ns = time.perf_counter_ns() - t0
                self._last.reason = str(exc)
                return reference
            self._last.gpu_cold_ns = time.perf_counter_ns() - t0
            if not agrees(reference, candidate):
                self._last.reason = "GPU calibration did not preserve binary64 accuracy"
                return reference
            gpu_times = []
            for _ in range(3):
                try:
                    candidate, ns = _measure(lambda: self._gpu(x))
                except Exception as exc:
                    self._last.reason = str(exc)
                    return reference
                gpu_times.append(ns)
                if not agrees(reference, candidate):
                    self._last.reason = "GPU calibration did not preserve binary64 accuracy"
                    return reference
            self._last.gpu_warm_ns = sorted(gpu_times)[1]
            if self._last.gpu_warm_ns < self._last.cpu_warm_ns * 4 // 5:
                self._last.selected = "vulkan-fp64"
                self._last.reason = "warm GPU call exceeds 20 percent speedup margin"
                return candidate
            self._last.reason = "CPU wins measured full-call comparison with 20 percent stability margin"
            return reference
