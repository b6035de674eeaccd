"""PROMETHEUS dispatch on the GPU: a block's ``@`` and ``PrometheusMatMul``
through the installed strict hook (interpret.go:2113-2117, 4643-4675;
strict.go:35-73), and the compiled runtime functions' status lines
(emit_go_runtime.go:788-807).  Operands are small integers over 8, so every
product and partial sum is exact in fp32 and the expected matrix is the
integer product computed in Python."""
from __future__ import annotations

import io

import pytest

from oct_amd import dispatch as d

pytestmark = pytest.mark.gpu


def _ints(rows, cols, seed):
    return [[((seed * 31 + r * 7 + c * 13) % 17 - 8) / 8.0 for c in range(cols)] for r in range(rows)]


def _exact_product(a, b):
    ai = [[int(x * 8) for x in row] for row in a]
    bi = [[int(x * 8) for x in row] for row in b]
    return [[sum(ai[r][k] * bi[k][c] for k in range(len(bi))) / 64.0 for c in range(len(bi[0]))]
            for r in range(len(ai))]


@pytest.fixture
def hook():
    d.install_strict_hook()
    yield
    d.set_strict_prometheus_matmul(None)


def test_block_at_and_builtin_run_on_the_gpu(hook):
    def no_cpu(*_):
        raise AssertionError("a PROMETHEUS block must not evaluate on the CPU")

    for m, k, n in ((2, 3, 2), (64, 80, 48), (130, 257, 65)):
        a, b = _ints(m, k, 1), _ints(k, n, 2)
        want = _exact_product(a, b)
        got = d.eval_binary(True, "@", d.float_matrix(a), d.float_matrix(b), no_cpu)
        assert (got.matrix.rows, got.matrix.cols) == (m, n)
        assert d._float_rows(got) == want, (m, k, n)
        got2 = d.eval_prometheus_matmul_call(True, [], [d.float_matrix(a), d.float_matrix(b)], no_cpu)
        assert d._float_rows(got2) == want


def test_compiled_runtime_status_lines():
    a, b = _ints(33, 40, 3), _ints(40, 21, 4)
    want = _exact_product(a, b)
    log = io.StringIO()
    assert d.oct_prometheus_matmul_mm_strict(a, b, log=log) == want
    assert log.getvalue().strip() == ("backend_requested=prometheus backend_used=prometheus status=ok detail_code=0 "
                                      "detail_name=gpu vulkan_env=hardware_gpu_hip")
    log = io.StringIO()
    assert d.oct_prometheus_matmul_mm(a, b, log=log) == want
    line = log.getvalue().strip()
    assert line.startswith("backend_requested=prometheus backend_used=prometheus status=ok correctness=true ")
    assert " vulkan_env=hardware_gpu_hip wall=" in line
