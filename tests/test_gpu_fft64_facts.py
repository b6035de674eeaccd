"""The reference's native FFT64 facts (internal/prometheus/native/Marionette/
reactor_fft64_tests.cpp:16-94) against the reactor's host-pointer FFT64.

* Independent DFT precision: lengths 1, 2, 8, 32, 128 with inputs whose low
  bits an fp32 conversion would lose, against an O(n^2) DFT in extended
  precision (numpy longdouble, x87 80-bit here) within 2e-12 * n; the input is
  left unchanged; the same runtime then runs the legacy 2x2x2 SGEMM.  The
  reference also checks that a warm call allocates no Vulkan buffers (Concept
  owner statistics) and that the Vulkan validation layer saw no errors; this
  library has neither (its device staging is reused by construction).
* Every injected fault (SKIP_VULKAN_INIT, FAIL_BUFFER_ALLOC, FAIL_UPLOAD,
  FAIL_DISPATCH, FAIL_DOWNLOAD, FAIL_COMMAND_END, FAIL_QUEUE_SUBMIT) fails
  the call with a reason and leaves the destination untouched.
* Binary64 dynamic range: inputs scaled by 1e-200 and 1e200 keep 1e-12
  relative accuracy.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu


def _dft_longdouble(x: np.ndarray) -> np.ndarray:
    n = x.size
    k = np.arange(n, dtype=np.longdouble)
    angle = -2 * np.longdouble(math.pi) * np.outer(k, k) / np.longdouble(n)
    c, s = np.cos(angle), np.sin(angle)
    re = x.real.astype(np.longdouble)
    im = x.imag.astype(np.longdouble)
    return (c @ re - s @ im), (s @ re + c @ im)


@pytest.mark.parametrize("count", [1, 2, 8, 32, 128])
def test_independent_dft_precision_and_coexistence(gpu_runtime, count):
    i = np.arange(count)
    x = (1.0 + np.ldexp(i + 1.0, -35)) + 1j * (np.sin(i.astype(np.float64)) + np.ldexp(1.0, -40))
    original = x.copy()
    out = np.full(count, -999.0 - 999.0j)
    rc, st, out = gpu_runtime.fft64(x, output=out)
    assert rc == p.PROM_OK and st.detail == 0
    assert np.array_equal(x.view(np.uint64), original.view(np.uint64))
    want_re, want_im = _dft_longdouble(x)
    tol = 2e-12 * count
    assert np.all(np.abs(want_re - out.real.astype(np.longdouble)) <= tol)
    assert np.all(np.abs(want_im - out.imag.astype(np.longdouble)) <= tol)
    # the legacy SGEMM on the same runtime (reactor_fft64_tests.cpp:53-56)
    c, status = gpu_runtime.sgemm(2, 2, 2, np.array([1, 2, 3, 4], np.float32), np.array([5, 6, 7, 8], np.float32))
    assert abs(float(c.reshape(-1)[0]) - 19.0) <= 1e-5


FLAGS = [p.TESTCFG_SKIP_VULKAN_INIT, p.TESTCFG_FAIL_BUFFER_ALLOC, p.TESTCFG_FAIL_UPLOAD, p.TESTCFG_FAIL_DISPATCH,
         p.TESTCFG_FAIL_DOWNLOAD, p.TESTCFG_FAIL_COMMAND_END, p.TESTCFG_FAIL_QUEUE_SUBMIT]


@pytest.mark.parametrize("flag", FLAGS, ids=["skip_init", "alloc", "upload", "dispatch", "download", "command_end",
                                              "queue_submit"])
def test_unavailable_and_failure_do_not_write_output(flag):
    rt = p.NativeRuntime(test_flags=flag)
    try:
        out = np.array([91 + 92j, 93 + 94j])
        rc, st, out = rt.fft64(np.array([1 + 0j, 2 + 0j]), output=out)
        assert rc == p.PROM_ERROR and st.detail != 0
        assert out[0].real == 91.0 and out[1].imag == 94.0  # no CPU fallback or partial output
    finally:
        rt.close()


@pytest.mark.parametrize("scale", [1e-200, 1e200])
def test_preserves_binary64_dynamic_range(gpu_runtime, scale):
    x = np.array([scale - scale * 1j, 2 * scale + scale * 1j, -scale + 0j, 0 + 2 * scale * 1j])
    rc, _, out = gpu_runtime.fft64(x)
    assert rc == p.PROM_OK
    for k in range(4):
        expected = sum((x[i] / scale) * complex(math.cos(-2.0 * math.pi * k * i / 4), math.sin(-2.0 * math.pi * k * i / 4))
                       for i in range(4))
        assert abs(expected.real - out[k].real / scale) <= 1e-12
        assert abs(expected.imag - out[k].imag / scale) <= 1e-12


def test_sgemm_command_end_and_queue_submit_fail_at_submit():
    """reactor_sgemm.cpp:5071-5078: stage SUBMIT, VK_ERROR_DEVICE_LOST (-4), no output."""
    for flag in (p.TESTCFG_FAIL_COMMAND_END, p.TESTCFG_FAIL_QUEUE_SUBMIT):
        rt = p.NativeRuntime(test_flags=flag)
        try:
            out, st, rc = rt.sgemm_with_status(2, 2, 2, np.ones(4, np.float32), np.ones(4, np.float32))
            assert rc == p.PROM_ERROR and (st.stage, st.detail) == (p.STAGE_SUBMIT, -4)
        finally:
            rt.close()
