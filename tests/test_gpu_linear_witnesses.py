"""The reference's real-model linear witnesses through the HIP fp32 SGEMM.

Each witness (tests/golden/m6_* .. m9_*, from
Experiments/ZImageTurboNoiseRefiner0/M6..M9) is one Z-Image NoiseRefiner
projection output: a captured fp32 input row times one weight column, FP16
as cached and BF16 as in the source checkpoint (both widen to fp32
exactly), with the captured projection.  The rows are stacked into A and
the columns into B, so one product computes every witness dot (and the
cross terms, which are checked against the binary64 `@` at the fp32 bar).
Each witness dot must meet the reference's facts (absolute 1e-3,
M6/W2.octest:7-13, M8/LinearPolicy.octest:1-16, M9/AdverseLinear.octest:1-21)
on the GPU's fp32 result.
"""
import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p
from tests.golden import octagon
from tests.test_oracle_linear_witnesses import POLICY, TOL

pytestmark = pytest.mark.gpu


def _product(rt, a, b):
    m, k = a.shape
    n = b.shape[1]
    out, status = rt.sgemm(m, n, k, a, b)
    assert str(status) == "ok"
    return out.reshape(m, n)


def _check_product(out, a, b):
    ref = oracle.matmul_f64(a, b)
    assert oracle.normwise_rel_err(out, ref) <= 1e-5
    return ref


def test_policy_and_adverse_witnesses(gpu_runtime):
    """K = 3840: the three M8 rows and nine M9 rows, FP16 and BF16 columns."""
    wit = [octagon.load(n) for n in POLICY]
    a = np.stack([f["Input"] for f in wit]).astype(np.float32)
    b = np.stack([f[c] for f in wit for c in ("FP16Weight", "BF16Weight")], axis=1).astype(np.float32)
    out = _product(gpu_runtime, a, b)
    ref = _check_product(out, a, b)
    for i, (name, f) in enumerate(zip(POLICY, wit)):
        fp16, bf16 = float(out[i, 2 * i]), float(out[i, 2 * i + 1])
        print(f"{name}: gpu fp16 {fp16:.7g} bf16 {bf16:.7g} expected {f['Expected']:.9g} "
              f"|gpu - binary64| {abs(fp16 - ref[i, 2 * i]):.2e}", flush=True)
        assert abs(f["Expected"] - fp16) <= TOL, name
        assert abs(bf16 - fp16) <= TOL, name
        assert abs(fp16 - ref[i, 2 * i]) <= TOL, name


def test_w2_witnesses(gpu_runtime):
    """K = 10240: the M6 row with its weight column and the M7 row with its
    FP16 and BF16 columns."""
    m6 = octagon.load("m6_w2_token0_channel0.octagon")
    m7 = octagon.load("m7_w2_token0_channel0_policy.octagon")
    a = np.stack([m6["Input"], m7["Input"]]).astype(np.float32)
    b = np.stack([m6["Weight"], m7["FP16Weight"], m7["BF16Weight"]], axis=1).astype(np.float32)
    out = _product(gpu_runtime, a, b)
    ref = _check_product(out, a, b)
    print(f"M6: gpu {out[0, 0]:.7g} expected {m6['Expected']:.9g} binary64 {ref[0, 0]:.9g}; "
          f"M7: fp16 {out[1, 1]:.7g} bf16 {out[1, 2]:.7g}", flush=True)
    assert abs(m6["Expected"] - out[0, 0]) <= TOL
    assert abs(out[0, 0] - ref[0, 0]) <= TOL
    assert abs(out[1, 2] - out[1, 1]) <= TOL


@pytest.mark.parametrize("tile,slices", [(0, 1), (3, 1), (5, 1), (6, 1), (0, 4), (4, 2)])
def test_witnesses_on_each_kernel_family(gpu_runtime, tile, slices):
    """The K = 3840 witnesses through the register-staged, direct-to-LDS and
    64x64 kernels, with and without split-K (fixed variants instead of the
    plan): every witness dot stays within the reference's 1e-3."""
    wit = [octagon.load(n) for n in POLICY]
    a = np.stack([f["Input"] for f in wit]).astype(np.float32)
    b = np.stack([f["FP16Weight"] for f in wit], axis=1).astype(np.float32)
    m, k = a.shape
    n = b.shape[1]
    rt = gpu_runtime
    da, db, dc = rt.upload_new(a), rt.upload_new(b), rt.alloc(m * n * 4)
    try:
        rc, st = rt.sgemm_device_variant(da, db, dc, m, n, k, tile, slices)
        assert rc == p.PROM_OK, (st.stage, st.detail)
        rt.synchronize()
        out = rt.download(np.empty((m, n), np.float32), dc)
    finally:
        for d in (da, db, dc):
            rt.free(d)
    ref = _check_product(out, a, b)
    worst = max(abs(float(out[i, i]) - f["Expected"]) for i, f in enumerate(wit))
    print(f"tile {tile} slices {slices}: worst |gpu - expected| {worst:.2e}", flush=True)
    for i, f in enumerate(wit):
        assert abs(float(out[i, i]) - f["Expected"]) <= TOL
        assert abs(float(out[i, i]) - ref[i, i]) <= TOL
