"""Octagon reports of the non-strict runtime (runtime.go:382-432, 497-658;
octagon_emit.go:11-130) on the CPU.

The float format is Go's strconv.FormatFloat(v, 'g', -1, 64): shortest
round-trip digits, %e form for decimal exponents below -4 or from 6 up, the
exponent with a sign and at least two digits.  The expected strings below are
those rules applied by hand, and each value is checked to parse back to
itself.  The reactor is forced unavailable with the SKIP_VULKAN_INIT test flag
for the async validation, whose result is then a skip, not an error.
"""
from __future__ import annotations

import pytest

from oct_amd import octagon
from oct_amd import prometheus as p
from oct_amd import runtime as rt

GO_G = [
    (1e6, "1e+06"), (123456.0, "123456"), (999999.0, "999999"), (1234567.0, "1.234567e+06"),
    (0.0001, "0.0001"), (0.00001, "1e-05"), (0.000123, "0.000123"), (1.5, "1.5"), (3.0, "3"),
    (-2.5e-7, "-2.5e-07"), (0.1, "0.1"), (1e21, "1e+21"), (1e100, "1e+100"), (5e-324, "5e-324"),
    (1.7976931348623157e308, "1.7976931348623157e+308"), (100000.0, "100000"), (0.0, "0"), (-0.0, "-0"),
    (float("nan"), "NaN"), (float("inf"), "+Inf"), (float("-inf"), "-Inf"), (2.0 ** -20, "9.5367431640625e-07"),
    (1 / 3, "0.3333333333333333"), (-123.456, "-123.456"), (1e-4 * 3, "0.00030000000000000003"),
]


@pytest.mark.parametrize("v,want", GO_G)
def test_float_format_is_go_shortest_g(v, want):
    got = octagon.format_float_g(v)
    assert got == want
    if want not in ("NaN", "+Inf", "-Inf"):
        assert float(got) == v


def test_serialized_floats_keep_a_decimal_mark():
    assert octagon.serialize(3.0) == "3.0" and octagon.serialize(1e6) == "1e+06" and octagon.serialize(-0.0) == "-0.0"
    assert octagon.serialize(2) == "2" and octagon.serialize(True) == "true"


def test_quote_matches_go():
    assert octagon.quote('a "b" \\ c') == '"a \\"b\\" \\\\ c"'
    assert octagon.quote("tab\tnl\nbell\a") == '"tab\\tnl\\nbell\\a"'
    assert octagon.quote("\x01\x7f") == '"\\x01\\x7f"'
    assert octagon.quote("µs é") == '"µs é"'
    assert octagon.quote("\u200b") == '"\\u200b"'


def test_record_layout_nesting_and_parentheses():
    inner = octagon.Record("pkg.Inner", [("X", 1), ("Y", 0.5), ("S", "s")])
    outer = octagon.Record("Outer", [("Items", [inner, inner]), ("Flag", False), ("N", -3)])
    want = ("Outer {\n"
            "    Items: [Inner {\n"
            "        X: (1)\n"
            "        Y: (0.5)\n"
            "        S: \"s\"\n"
            "    }, Inner {\n"
            "        X: (1)\n"
            "        Y: (0.5)\n"
            "        S: \"s\"\n"
            "    }]\n"
            "    Flag: false\n"
            "    N: (-3)\n"
            "}")
    assert octagon.serialize(outer) == want


def test_write_checks_the_suffix_and_applies_the_prefix(tmp_path):
    with pytest.raises(ValueError, match="must end with .octagon"):
        octagon.write(str(tmp_path / "r.txt"), 1)
    path = octagon.write(str(tmp_path / "r.octagon"), octagon.Record("R", [("A", 1)]), prefix="run7")
    assert path.endswith("run7.r.octagon")
    assert open(path).read() == "R {\n    A: (1)\n}\n"


def test_cpu_corpus_report():
    runs = rt.run_starter_corpus(rt.BACKEND_CPU)
    text = octagon.serialize(rt.report_to_octagon(runs))
    assert text.startswith("PrometheusSgemmReport {\n    Runs: [PrometheusSgemmRun {\n")
    assert text.count("PrometheusSgemmRun {") == 5
    fields = ["BackendRequested", "BackendUsed", "M", "N", "K", "Status", "DetailCode", "DetailName",
              "CorrectnessPass", "MaxAbsError", "MaxRelError", "FailingElementCount", "FirstFailingIndex",
              "FirstExpectedValue", "FirstActualValue", "CPUTimeNs", "VulkanTimeNs", "VulkanEnv", "TimingMode",
              "WallTimeNs", "Notes"]
    first = text.split("PrometheusSgemmRun {\n")[1].split("\n    }")[0]
    assert [line.strip().split(":")[0] for line in first.splitlines()] == fields
    assert '        BackendUsed: "cpu"\n        M: (1)\n        N: (1)\n        K: (1)\n        Status: "ok"\n' in text
    assert "        CorrectnessPass: true\n" in text and "        FirstFailingIndex: (0)\n" in text


def test_async_validation_without_a_device_is_a_skip(monkeypatch, tmp_path):
    monkeypatch.setenv(p.REACTOR_TEST_FLAGS_ENV_VAR, str(p.TESTCFG_SKIP_VULKAN_INIT))
    res = rt.validate_async_sgemm_on_hardware(rt.Shape(64, 64, 32))
    assert (res.outcome, res.used_backend, res.environment) == ("skipped(prometheus_unavailable)", "cpu",
                                                               "unavailable")
    path = rt.write_async_validation_octagon(str(tmp_path / "async.octagon"), res)
    text = open(path).read()
    want_head = ("PrometheusAsyncValidation {\n    BackendRequested: \"prometheus\"\n    BackendUsed: \"cpu\"\n"
                 "    M: (64)\n    N: (64)\n    K: (32)\n    Outcome: \"skipped(prometheus_unavailable)\"\n"
                 "    Environment: \"unavailable\"\n    SubmitStage: \"unknown\"\n    SubmitDetailCode: (0)\n"
                 "    SubmitDetailName: \"not_applicable\"\n    QueryLifecycle: \"idle\"\n    QueryReady: false\n"
                 "    QueryFailed: false\n    QueryConsumed: false\n    QueryOutstanding: (0)\n"
                 "    QueryAttempts: (0)\n    ConsumeStage: \"unknown\"\n    ConsumeDetailCode: (0)\n"
                 "    ConsumeDetailName: \"not_applicable\"\n    CorrectnessPass: false\n    MaxAbsError: (0.0)\n"
                 "    MaxRelError: (0.0)\n    FailingElementCount: (0)\n    FirstFailingIndex: (0)\n"
                 "    FirstExpectedValue: (0.0)\n    FirstActualValue: (0.0)\n    WallTimeNs: (0)\n    Notes: \"")
    assert text.startswith(want_head), text
    assert text.endswith("\"\n}\n")


def test_lifecycle_names():
    assert [rt.async_lifecycle_name(s) for s in range(6)] == ["idle", "submitted", "ready", "failed", "consumed",
                                                               "state_5"]
