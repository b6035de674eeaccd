"""The reference's real-model linear witnesses, against the binary64 `@` oracle.

Fixtures (tests/golden/m6_* .. m9_*, copied verbatim from
Experiments/ZImageTurboNoiseRefiner0/M6..M9): one Z-Image NoiseRefiner
projection output (token 0, channel 0) each, with the captured fp32 input
row, the weight column (FP16 as cached, and BF16 as in the source
checkpoint) and the captured projection.  Inputs span ~1e-15 to 2e2; the M9
"cancel" rows were chosen to cancel.

The reference's facts, restated here against `oracle.matmul_f64` (Oct's `@`,
interpret.go:6278-6305; a 1 x K by K x 1 product is the fixed-order binary64
dot the .octest files write out):
  M6/W2.octest:7-13            |Expected - dot(Input, Weight)| <= 1e-3, K = 10240
  M7/W2Policy.octest:9-16      |dot(Input, BF16) - dot(Input, FP16)| <= 1e-3
  M8/LinearPolicy.octest:1-16  the same, and |Expected - dot(Input, FP16)| <= 1e-3, K = 3840
  M9/AdverseLinear.octest:1-21 the same on the nine high / error / cancel rows
"""
import numpy as np
import pytest

import oracle
from tests.golden import octagon

TOL = 1e-3  # Assert.Near's absolute tolerance (interpret.go:2912-2944)
M8 = [f"m8_{n}_token0_channel0_policy.octagon" for n in ("qkv", "w1", "w3")]
M9 = [f"m9_{n}_{c}.octagon" for c in ("high", "error", "cancel") for n in ("qkv", "w1", "w3")]
POLICY = M8 + M9


def oct_dot(x, w) -> float:
    return float(oracle.matmul_f64(np.asarray(x, np.float32)[None, :], np.asarray(w, np.float32)[:, None])[0, 0])


def test_fixture_values_are_the_stored_precisions():
    """Inputs are fp32 values, FP16Weight FP16 values and BF16Weight BF16 values,
    printed to 9 significant digits: each reads back to its own format within
    a printing error, so widening to fp32 is exact for every operand."""
    for name in POLICY + ["m7_w2_token0_channel0_policy.octagon"]:
        f = octagon.load(name)
        for field, fmt in (("Input", np.float32), ("FP16Weight", np.float16)):
            v = f[field]
            np.testing.assert_allclose(v.astype(fmt).astype(np.float64), v, rtol=1e-8, atol=0)
        b = f["BF16Weight"]
        np.testing.assert_allclose(oracle.from_bf16(oracle.to_bf16(b.astype(np.float32))), b, rtol=1e-8, atol=0)


def test_oct_at_is_the_fixed_order_dot():
    """The witnesses' dot (sum = 0.0; sum += x*w in order) and Oct's `@` round
    identically: a1 = x0*w0 then a += x_k*w_k."""
    f = octagon.load("m9_qkv_cancel.octagon")
    x, w = f["Input"].astype(np.float32), f["FP16Weight"].astype(np.float32)
    s = 0.0
    for a, b in zip(x.astype(np.float64), w.astype(np.float64)):
        s = s + a * b
    assert oct_dot(x, w) == s


def test_m6_w2_dot():
    f = octagon.load("m6_w2_token0_channel0.octagon")
    assert len(f["Input"]) == 10240 == len(f["Weight"])
    got = oct_dot(f["Input"], f["Weight"])
    assert abs(got) < 1e6
    assert abs(f["Expected"] - got) <= TOL


def test_m7_w2_policy_dot():
    f = octagon.load("m7_w2_token0_channel0_policy.octagon")
    assert len(f["Input"]) == 10240
    assert abs(oct_dot(f["Input"], f["BF16Weight"]) - oct_dot(f["Input"], f["FP16Weight"])) <= TOL


@pytest.mark.parametrize("name", POLICY)
def test_policy_and_adverse_dots(name):
    f = octagon.load(name)
    assert len(f["Input"]) == 3840
    fp16 = oct_dot(f["Input"], f["FP16Weight"])
    assert abs(oct_dot(f["Input"], f["BF16Weight"]) - fp16) <= TOL
    assert abs(f["Expected"] - fp16) <= TOL


def test_witnesses_are_sensitive():
    """A dropped last term or a sign error would break the facts above."""
    f = octagon.load("m9_qkv_high.octagon")
    x, w = f["Input"], f["FP16Weight"]
    assert abs(oct_dot(x[:-1], w[:-1]) - f["Expected"]) > TOL or abs(x[-1] * w[-1]) <= TOL
    assert abs(oct_dot(x, -w) - f["Expected"]) > TOL
    # at least one term is large enough that dropping it fails the check
    big = int(np.argmax(np.abs(x * w)))
    keep = np.arange(len(x)) != big
    assert abs(oct_dot(x[keep], w[keep]) - f["Expected"]) > TOL
