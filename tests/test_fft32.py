"""The batched complex-fp32 FFT: its oracle pinned, and the C ABI's
validation and diagnostics (no device needed).

The oracle (oracle.dft_c32) restates the reference's acceptance authority,
a direct binary64 DFT (internal/prometheus/native/Marionette/
reactor_fft_api_tests.cpp:525-553).  It is pinned by the reference's own
known answers (:198-233, :591-620), closed forms, numpy.fft (an independent
implementation) and the round trip.  The ABI cases follow
reactor_fft_api_tests.cpp:127-142, 687-733, 760-865: validation order and
details, diagnostics defaults, sized snapshots, per-call freshness and the
deterministic radix-2 plan; on a device-less runtime a valid request records
its plan and reports VULKAN_UNAVAILABLE (there is no CPU fallback).
"""
import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p

FD = p.PROM_FFT_DETAIL


# ------------------------------------------------------------ oracle
def test_reference_known_answers():
    # reactor_fft_api_tests.cpp:198-233: N=2 and N=4, forward negative sign
    np.testing.assert_allclose(oracle.dft_c32(np.array([1, 2], np.complex64), 2), [3, -1], atol=1e-6)
    got = oracle.dft_c32(np.array([1, 2, 3, 4], np.complex64), 4)
    np.testing.assert_allclose(got, [10, -2 + 2j, -2, -2 - 2j], atol=1e-6)
    # :591-620: two N=2 batches four apart; padding is the input's; the inverse restores
    x = np.array([1, 2, 91 - 91j, 92 - 92j, 3, 5], np.complex64)
    y = oracle.dft_c32(x, 2, batch=2, stride=4)
    np.testing.assert_allclose(y[[0, 1, 4, 5]], [3, -1, 8, -2], atol=1e-6)
    assert y[2] == x[2] and y[3] == x[3]
    back = oracle.dft_c32(y, 2, batch=2, stride=4, inverse=True)
    np.testing.assert_allclose(back[[0, 1, 4, 5]], [1, 2, 3, 5], atol=1e-6)


@pytest.mark.parametrize("n", [1, 2, 8, 64, 256])
def test_closed_forms(n):
    impulse = np.zeros(n, np.complex64)
    impulse[0] = 1
    np.testing.assert_allclose(oracle.dft_c32(impulse, n), np.ones(n), atol=1e-6)
    np.testing.assert_allclose(oracle.dft_c32(np.full(n, 2 - 0.5j, np.complex64), n)[0], n * (2 - 0.5j), rtol=1e-6)
    f = n // 4 if n >= 4 else 0
    tone = np.exp(2j * np.pi * f * np.arange(n) / n).astype(np.complex64)
    ref = np.zeros(n, np.complex128)
    ref[f] = n
    np.testing.assert_allclose(oracle.dft_c32(tone, n), ref, atol=2e-4 * n)


@pytest.mark.parametrize("n", [8, 64, 512])
def test_matches_numpy_fft_and_round_trip(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(3 * n) + 1j * rng.standard_normal(3 * n)).astype(np.complex64)
    got = oracle.dft_c32(x, n, batch=3)
    ref = np.fft.fft(x.astype(np.complex128).reshape(3, n), axis=1).ravel()
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    inv = oracle.dft_c32(got, n, batch=3, inverse=True)
    np.testing.assert_allclose(inv, np.fft.ifft(got.astype(np.complex128).reshape(3, n), axis=1).ravel(),
                               atol=1e-6 * np.abs(x).max())
    assert np.abs(inv - x).max() <= 1e-5 * np.abs(x).max()


def test_planted_sign_error_is_caught():
    # a forward transform with the inverse's sign disagrees with numpy.fft
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(16) + 1j * rng.standard_normal(16)).astype(np.complex64)
    wrong = oracle.dft_c32(x, 16, inverse=True) * 16
    assert np.abs(wrong - np.fft.fft(x.astype(np.complex128))).max() > 1e-2


# ------------------------------------------------------------ C ABI, no device
@pytest.fixture
def rt():
    r = p.NativeRuntime(test_flags=0)
    yield r
    r.close()


def test_diagnostics_default_state(rt):
    d = rt.fft_diagnostics()
    assert d.struct_size == p.ctypes.sizeof(p.PrometheusFftDiagnostics) == 216 and d.api_declared == 1
    assert d.capability_reported == 0 and d.production_enabled == 0 and d.benchmark_enabled == 0
    assert d.executed_path_id == p.PROM_FFT_PATH_UNAVAILABLE and d.last_failure_detail == FD["UNAVAILABLE"]


def test_validation_failures(rt):
    x = np.zeros(4, np.complex64)
    cases = [
        (dict(request_patch=lambda r: setattr(r, "struct_size", 0)), "INVALID_REQUEST"),
        (dict(request_patch=lambda r: setattr(r, "input", None)), "NULL_INPUT"),
        (dict(request_patch=lambda r: setattr(r, "output", None)), "NULL_OUTPUT"),
        (dict(count=0), "ZERO_ELEMENT_COUNT"),
        (dict(count=3), "NON_POWER_OF_TWO"),
        (dict(count=1 << 21), "UNSUPPORTED_SIZE"),
        (dict(batch=0), "ZERO_BATCH_COUNT"),
        (dict(flags=p.PROM_FFT_FLAG_FORWARD | p.PROM_FFT_FLAG_INVERSE), "INVALID_DIRECTION_FLAGS"),
        (dict(flags=p.PROM_FFT_FLAG_INVERSE_NORMALIZE), "INVERSE_NORMALIZE_REQUIRES_INVERSE"),
        (dict(stride=1), "INVALID_STRIDE"),
        (dict(stride=1 << 16, batch=1 << 16), "SIZE_OVERFLOW"),
        (dict(stride=1 << 26, batch=64), "SIZE_OVERFLOW"),   # 8 bytes * physical > UINT32_MAX
        (dict(count=256, batch=65536), "UNSUPPORTED_SIZE"),  # 256 * 65536 > 65535 * 256
    ]
    for kw, name in cases:
        args = dict(count=2, batch=1, stride=0, flags=0)
        args.update(kw)
        patch = args.pop("request_patch", None)
        rc, cs, _ = rt.fft(x, request_patch=patch, **args)
        assert rc == p.PROM_ERROR and cs.stage == p.STAGE_INIT and cs.detail == FD[name], (kw, cs.detail)
        d = rt.fft_diagnostics()
        assert d.last_failure_detail == FD[name] and d.plan_valid == 0
        assert d.requested_path_id == p.PROM_FFT_PATH_NONE and d.executed_path_id == p.PROM_FFT_PATH_UNAVAILABLE
    # a null request
    stage, detail = p.c_uint32(0), p.c_int(0)
    assert rt.lib.prometheus_reactor_runtime_fft(rt.handle, None, p.byref(stage), p.byref(detail)) == p.PROM_ERROR
    assert detail.value == FD["INVALID_REQUEST"]


def test_invalid_handle_and_variant(rt):
    x = np.zeros(2, np.complex64)
    r = p.PrometheusFftRequest(p.ctypes.sizeof(p.PrometheusFftRequest), x.ctypes.data, x.ctypes.data, 2, 1, 0, 0)
    stage, detail = p.c_uint32(0), p.c_int(0)
    assert rt.lib.prometheus_reactor_runtime_fft(None, p.byref(r), p.byref(stage), p.byref(detail)) == \
        p.PROM_INVALID_HANDLE
    d = p.PrometheusFftDiagnostics()
    assert rt.lib.prometheus_reactor_runtime_fft_diagnostics(None, p.byref(d)) == p.PROM_INVALID_HANDLE
    assert rt.lib.prometheus_reactor_runtime_fft_diagnostics(rt.handle, None) == p.PROM_ERROR
    assert rt.lib.prometheus_reactor_runtime_fft_diagnostics_sized(rt.handle, p.byref(d), 0) == p.PROM_ERROR
    rc, cs, _ = rt.fft(x, 2, variant=7)
    assert rc == p.PROM_ERROR and cs.detail == FD["PLAN_DISPATCH_DISAGREEMENT"]


def test_sized_diagnostics_snapshot(rt):
    d = p.PrometheusFftDiagnostics()
    d.plan_valid = 9
    assert rt.lib.prometheus_reactor_runtime_fft_diagnostics_sized(rt.handle, p.byref(d), 4) == p.PROM_OK
    assert d.struct_size == 216 and d.plan_valid == 9  # only the first four bytes were written
    full = rt.fft_diagnostics(size=10_000)
    assert full.api_declared == 1


def test_plan_recorded_before_the_device_check(rt):
    # reactor_fft_api_tests.cpp:824-865 on a device-less runtime: the plan is
    # deterministic and recorded; execution reports VULKAN_UNAVAILABLE
    if rt.available:
        pytest.skip("a device is present: the plan is checked after execution by the GPU tests")
    x = np.zeros(16, np.complex64)
    for n, flags, passes, last, direction, role in ((1, 0, 0, 0, 1, 2), (8, 0, 3, 8, 1, 3),
                                                     (16, p.PROM_FFT_FLAG_INVERSE, 4, 16, 2, 2)):
        rc, cs, _ = rt.fft(x, n, flags=flags)
        assert rc == p.PROM_ERROR and cs.detail == FD["VULKAN_UNAVAILABLE"]
        d = rt.fft_diagnostics()
        assert d.plan_valid == 1 and d.plan_pass_count == passes and d.ping_pong_swap_count == passes
        assert d.plan_log2_element_count == passes and d.plan_last_span == last
        assert d.plan_first_span == (2 if n > 1 else 0) and d.plan_bit_reversal_required == (1 if n > 1 else 0)
        assert d.plan_direction == direction and d.last_direction == direction and d.final_output_role == role
        assert d.requested_path_id == p.PROM_FFT_PATH_VULKAN_RADIX2_RESERVED and d.requested_radix == 2
        assert d.executed_path_id == p.PROM_FFT_PATH_UNAVAILABLE and d.last_effective_stride_elements == n
