"""The non-strict runtime's async hardware validation and its Octagon
reports on the GPU (runtime.go:382-425, 521-658): the reference's 64x64x32
validation reaches `ok` through submit, query and consume, and the starter
corpus on the reactor passes its gate in every run."""
from __future__ import annotations

import pytest

from oct_amd import runtime as rt

pytestmark = pytest.mark.gpu


def test_async_validation_on_hardware(tmp_path):
    res = rt.validate_async_sgemm_on_hardware(rt.Shape(64, 64, 32))
    assert res.outcome == "ok", (res.outcome, res.notes)
    assert (res.used_backend, res.environment, res.query_lifecycle) == ("prometheus", "hardware_gpu_hip", "ready")
    assert res.query_ready and not res.query_failed and res.query_attempts >= 1
    assert res.correctness.passed and res.correctness.failing_count == 0
    text = open(rt.write_async_validation_octagon(str(tmp_path / "async.octagon"), res)).read()
    assert '    Outcome: "ok"\n' in text and "    CorrectnessPass: true\n" in text
    assert '    QueryLifecycle: "ready"\n' in text


def test_prometheus_corpus_report(tmp_path):
    runs = rt.run_starter_corpus(rt.BACKEND_PROMETHEUS)
    assert [r.used_backend for r in runs] == ["prometheus"] * 5
    assert all(r.correctness.passed and str(r.status) == "ok" for r in runs)
    text = open(rt.write_octagon_report(str(tmp_path / "corpus.octagon"), runs)).read()
    assert text.count('        BackendUsed: "prometheus"\n') == 5 and text.count("        CorrectnessPass: true\n") == 5
    assert '        VulkanEnv: "hardware_gpu_hip"\n' in text
