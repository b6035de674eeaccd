"""Oct's PROMETHEUS GPU-lane contracts (Language/Prometheus/gpu/*.octest,
bench/strict_matrix.octest) through this package's dispatch on the reactor,
in the interpreter's lane and the compiled program's lane."""
from __future__ import annotations

import io

import numpy as np
import pytest

from oct_amd import dispatch as d
from oct_amd import fft_engine as fe

pytestmark = pytest.mark.gpu


@pytest.fixture
def hook():
    d.install_strict_hook()
    yield
    d.set_strict_prometheus_matmul(None)


def _no_cpu(*_):
    raise AssertionError("a PROMETHEUS block must not evaluate on the CPU")


def test_strict_matrix_execution_uses_the_gpu(hook):
    # gpu/matrix.octest:3-10
    a = d.float_matrix([[1.0, 2.0], [3.0, 4.0]])
    result = d.eval_binary(True, "@", a, a, _no_cpu)
    assert result.matrix.elements[0].number == 7.0
    log = io.StringIO()
    assert d.oct_prometheus_matmul_mm_strict([[1.0, 2.0], [3.0, 4.0]], [[1.0, 2.0], [3.0, 4.0]], log=log)[0][0] == 7.0
    assert "backend_used=prometheus status=ok" in log.getvalue()


def test_strict_matrix_benchmark(hook):
    # bench/strict_matrix.octest:12-19
    a = d.float_matrix([[3.0, 3.0], [3.0, 3.0]])
    b = d.float_matrix([[5.0, 5.0], [5.0, 5.0]])
    assert d._float_rows(d.eval_binary(True, "@", a, b, _no_cpu)) == [[30.0, 30.0], [30.0, 30.0]]


def _forced_facts(transform):
    # gpu/fft.octest:7-16
    source = [1.0000000000291038 + 0j, 1.0 + 0j]
    spectrum = transform(source)
    assert spectrum[0].real > 2.0
    assert abs(0.0000000000291038 - spectrum[1].real) <= 0.000000000000001
    assert source[0].real == 1.0000000000291038
    # gpu/fft.octest:19-28
    spectrum = transform([0j, 1 + 0j, 0j, 0j])
    assert abs(1.0 - spectrum[0].real) <= 1e-12
    assert abs(-1.0 - spectrum[1].imag) <= 1e-12
    assert abs(-1.0 - spectrum[2].real) <= 1e-12
    assert abs(1.0 - spectrum[3].imag) <= 1e-12


def test_forced_fft_interpreted():
    with fe.FFTEngine() as engine:
        def transform(values):
            res = d.eval_fft_call(engine, True, [], [d.complex_array(values)])
            assert res.error is None, res.error
            return [v.complex_value for v in res.value.array]

        _forced_facts(transform)


def test_forced_fft_compiled():
    assert d.lower_fft_call(True, ["Complex[]"])[0] == "FFTGPU"
    with d.new_fft_engine() as engine:
        def transform(values):
            res = d.oct_fft(engine, np.array(values, np.complex128), required_gpu=True)
            assert not res.is_err, res.err
            return list(res.value)

        _forced_facts(transform)
