"""The FFT engine (internal/fft/fft.go:80-154) with the reactor as its GPU
backend (internal/prometheus/fft.go:21-48).

Strict execution returns the reactor's transform, bit-identical to the
engine's CPU transform where the reactor's is one LDS-resident workgroup
(n <= 4096), and reports the reference's error beyond 2^20 elements.
Automatic execution at 2^20 times both sides, accepts the reactor only after
its results pass fft.go's agreement rule, and the next call of that length
uses the selected backend.
"""
from __future__ import annotations

import numpy as np
import pytest

from oct_amd import fft_engine as fe

pytestmark = pytest.mark.gpu


def _values(n, seed):
    rng = np.random.default_rng(seed)
    return rng.standard_normal(n) + 1j * rng.standard_normal(n)


def test_strict_runs_on_the_reactor():
    with fe.FFTEngine() as eng:
        for n in (1, 2, 64, 4096):
            x = _values(n, n)
            out = eng.transform(x, required_gpu=True)
            assert np.array_equal(out.view(np.uint64), fe.cpu(x).view(np.uint64)), n
        x = _values(1 << 16, 5)
        assert fe.agrees(fe.cpu(x), eng.transform(x, required_gpu=True))
        assert eng.measurement().elements == 0
        with pytest.raises(fe.FFTError, match="^PROMETHEUS FFT requires GPU execution: Vulkan FFT supports at most "
                                              "1048576 complex values$"):
            eng.transform(np.zeros(1 << 21, np.complex128), required_gpu=True)
        with pytest.raises(fe.FFTError, match="power-of-two"):
            eng.transform(np.zeros(12, np.complex128), required_gpu=True)


def test_automatic_selection_at_full_size():
    n = 1 << 20
    x = _values(n, 11)
    ref = fe.cpu(x)
    with fe.FFTEngine() as eng:
        out = eng.transform(x, required_gpu=False)
        m = eng.measurement()
        print(f"n=2^20: selected={m.selected} cpu_warm={m.cpu_warm_ns / 1e6:.2f} ms "
              f"gpu_cold={m.gpu_cold_ns / 1e6:.2f} ms gpu_warm={m.gpu_warm_ns / 1e6:.2f} ms ({m.reason})")
        assert m.elements == n and m.cpu_warm_ns > 0 and m.gpu_cold_ns > 0 and m.gpu_warm_ns > 0
        assert m.reason in ("warm GPU call exceeds 20 percent speedup margin",
                            "CPU wins measured full-call comparison with 20 percent stability margin")
        assert fe.agrees(ref, out)
        if m.selected == "vulkan-fp64":
            assert m.gpu_warm_ns < m.cpu_warm_ns * 4 // 5
        again = eng.transform(x, required_gpu=False)
        assert np.array_equal(again.view(np.uint64), out.view(np.uint64))
        assert eng.measurement() == m


@pytest.mark.parametrize("seed", [4096, 1, 2, 3, 4])
def test_4096_points_bit_identical_for_several_inputs(seed):
    """A one-ulp difference in one twiddle shows in the output for some
    inputs only (seed 4096 shows the sincos/cos-sin difference at n = 4096)."""
    x = _values(4096, seed)
    with fe.FFTEngine() as eng:
        out = eng.transform(x, required_gpu=True)
    assert np.array_equal(out.view(np.uint64), fe.cpu(x).view(np.uint64))
