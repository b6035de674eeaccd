"""GPU parity of the binary64 FFT against the CPU contract (internal/fft/fft.go).

Bar: the reference's own agreement rule (fft.go:176-192), every component within
1e-12 * max|X|; for n <= 4096 (one LDS-resident workgroup performing the
reference's butterflies with its twiddles) the result must be bit-identical to
the oracle.  Cases: the Oct FFT facts (Language/Prometheus/gpu/fft.octest),
every power of two 1..2^20, closed forms at full size, in-place use, and the
device-pointer entry.
"""
import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu


def _rand(n, seed):
    rng = np.random.default_rng(seed)
    return rng.standard_normal(n) + 1j * rng.standard_normal(n)


def test_octest_facts(gpu_runtime):
    # gpu/fft.octest:7-28
    delta = 0.0000000000291038304567337
    x = np.array([1.0 + delta, 1.0], np.complex128)
    rc, cs, X = gpu_runtime.fft64(x)
    assert rc == p.PROM_OK and (cs.stage, cs.detail) == (p.STAGE_TRANSFER_OUT, 0)
    assert X[0].real > 2.0 and abs(X[1].real - delta) <= 1e-15
    assert x[0].real == 1.0 + delta
    rc, cs, X = gpu_runtime.fft64(np.array([0, 1, 0, 0], np.complex128))
    assert abs(X[0].real - 1) <= 1e-12 and abs(X[1].imag + 1) <= 1e-12
    assert abs(X[2].real + 1) <= 1e-12 and abs(X[3].imag - 1) <= 1e-12


@pytest.mark.parametrize("log2n", list(range(0, 13)))
def test_lds_sizes_bit_identical(gpu_runtime, log2n):
    n = 1 << log2n
    x = _rand(n, log2n)
    rc, _, X = gpu_runtime.fft64(x)
    assert rc == p.PROM_OK
    np.testing.assert_array_equal(X, oracle.fft64(x))


@pytest.mark.parametrize("log2n", list(range(13, 21)))
def test_four_step_sizes_agree(gpu_runtime, log2n):
    n = 1 << log2n
    x = _rand(n, 100 + log2n)
    rc, _, X = gpu_runtime.fft64(x)
    assert rc == p.PROM_OK
    ref = oracle.fft64(x)
    assert oracle.fft64_agrees(ref, X)
    scale = np.abs(ref).max()
    print(f"n=2^{log2n}: max |GPU - CPU| / max|X| = {np.abs(X - ref).max() / scale:.2e}")


def test_full_size_closed_forms(gpu_runtime):
    n = 1 << 20
    impulse = np.zeros(n, np.complex128)
    impulse[5] = 1
    rc, _, X = gpu_runtime.fft64(impulse)
    assert rc == p.PROM_OK
    np.testing.assert_allclose(X, np.exp(-2j * np.pi * ((np.arange(n) * 5) % n) / n), rtol=0, atol=1e-12)
    k0 = 12345
    # phase reduced exactly (k0*j mod n) so that the input itself is accurate to 1 ulp
    tone = np.exp(2j * np.pi * ((k0 * np.arange(n)) % n) / n)
    rc, _, X = gpu_runtime.fft64(tone)
    assert oracle.fft64_agrees(oracle.fft64(tone), X)
    expect = np.zeros(n, np.complex128)
    expect[k0] = n
    np.testing.assert_allclose(X, expect, rtol=0, atol=1e-12 * n)
    # linearity and Parseval on random data
    x, y = _rand(n, 1), _rand(n, 2)
    X = gpu_runtime.fft64(x)[2]
    Y = gpu_runtime.fft64(y)[2]
    Z = gpu_runtime.fft64(2 * x - 3 * y)[2]
    assert oracle.fft64_agrees(Z, 2 * X - 3 * Y)
    assert abs(np.vdot(X, X).real - n * np.vdot(x, x).real) <= 1e-10 * n * np.vdot(x, x).real


def test_in_place_and_repeat_sizes(gpu_runtime):
    for n in (1 << 14, 64, 1 << 14, 1 << 20, 8):
        x = _rand(n, n)
        ref = oracle.fft64(x)
        buf = x.copy()
        rc, _, out = gpu_runtime.fft64(buf, output=buf)
        assert rc == p.PROM_OK and out is buf
        assert oracle.fft64_agrees(ref, buf)


def test_device_entry(gpu_runtime):
    rt = gpu_runtime
    for n in (4096, 1 << 20):
        x = _rand(n, 7 * n)
        din, dout = rt.upload_new(x.view(np.float64)), rt.alloc(x.nbytes)
        try:
            assert rt.fft64_device(din, dout, n) == 0
            rt.synchronize()
            X = rt.download(np.empty(n, np.complex128), dout)
        finally:
            rt.free(din)
            rt.free(dout)
        ref = oracle.fft64(x)
        if n <= 4096:
            np.testing.assert_array_equal(X, ref)
        else:
            assert oracle.fft64_agrees(ref, X)


# ------------------------------------------------------------ batched complex-fp32 FFT
# Bars of the reference's acceptance (reactor_fft_api_tests.cpp:525-620):
# maximum absolute error <= 3e-3 against the direct binary64 DFT for its
# corpus, output padding untouched; at large lengths (beyond an O(n^2) DFT)
# numpy's binary64 FFT is the authority, relative L2 <= 1e-6 per batch.
def _lcg_c32(n):
    # reactor_fft_api_tests.cpp:626-633
    state = (0x9E3779B9 ^ n) & 0xFFFFFFFF
    out = np.empty(n, np.complex64)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        re = (((state >> 8) & 0xFFFF) - 32768) / 32768.0
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        im = (((state >> 8) & 0xFFFF) - 32768) / 32768.0
        out[i] = complex(re, im)
    return out


def _valid_index(n, batch, stride):
    return (np.arange(batch)[:, None] * stride + np.arange(n)[None, :]).ravel()


def _fft32_vs_dft(rt, x, n, batch=1, stride=None, inverse=False, atol=3e-3):
    stride = stride or n
    out = np.full(x.shape, 77 - 77j, np.complex64)
    rc, cs, out = rt.fft(x, n, batch, 0 if stride == n else stride, p.PROM_FFT_FLAG_INVERSE if inverse else 0,
                         output=out)
    assert rc == p.PROM_OK and (cs.stage, cs.detail) == (p.STAGE_TRANSFER_OUT, 0), cs.detail
    ref = oracle.dft_c32(x, n, batch, stride, inverse)
    valid = _valid_index(n, batch, stride)
    err = np.abs(out[valid] - ref[valid]).max()
    assert err <= atol, (n, batch, stride, inverse, err)
    pad = np.setdiff1d(np.arange(x.size), valid)
    assert (out[pad] == np.complex64(77 - 77j)).all()
    return out


def test_fft32_reference_facts(gpu_runtime):
    # reactor_fft_api_tests.cpp:198-233, 591-620
    rc, cs, out = gpu_runtime.fft(np.array([1, 2], np.complex64), 2)
    assert rc == p.PROM_OK and abs(out[0] - 3) <= 1e-5 and abs(out[1] + 1) <= 1e-5
    rc, cs, out = gpu_runtime.fft(np.array([1, 2, 3, 4], np.complex64), 4)
    np.testing.assert_allclose(out, [10, -2 + 2j, -2, -2 - 2j], atol=2e-5)
    x = np.array([1, 2, 91 - 91j, 92 - 92j, 3, 5], np.complex64)
    out = np.array([-1 - 1j, -1 - 1j, 77 - 77j, 78 - 78j, -1 - 1j, -1 - 1j], np.complex64)
    rc, cs, out = gpu_runtime.fft(x, 2, batch=2, stride=4, output=out)
    assert rc == p.PROM_OK
    np.testing.assert_allclose(out[[0, 1, 4, 5]], [3, -1, 8, -2], atol=1e-5)
    assert out[2] == np.complex64(77 - 77j) and out[3] == np.complex64(78 - 78j)
    back = x.copy()
    rc, cs, back = gpu_runtime.fft(out, 2, batch=2, stride=4, flags=p.PROM_FFT_FLAG_INVERSE, output=back)
    assert rc == p.PROM_OK
    np.testing.assert_allclose(back[[0, 1, 4, 5]], [1, 2, 3, 5], atol=1e-5)
    # INVERSE_NORMALIZE with INVERSE is the same normalised inverse
    rc, cs, again = gpu_runtime.fft(out, 2, batch=2, stride=4,
                                    flags=p.PROM_FFT_FLAG_INVERSE | p.PROM_FFT_FLAG_INVERSE_NORMALIZE)
    np.testing.assert_array_equal(again[[0, 1, 4, 5]], back[[0, 1, 4, 5]])


def test_fft32_numerical_corpus(gpu_runtime):
    # reactor_fft_api_tests.cpp:622-685
    for n in (1, 2, 8, 16, 64, 256, 1024):
        x = _lcg_c32(n)
        _fft32_vs_dft(gpu_runtime, x, n)
        _fft32_vs_dft(gpu_runtime, x, n, inverse=True)
    i = np.arange(32, dtype=np.float32)
    angle = np.float32(2.0 * np.pi * 5.0) * i / np.float32(32.0)
    _fft32_vs_dft(gpu_runtime, (np.cos(angle) + 1j * np.sin(angle)).astype(np.complex64), 32)
    i = np.arange(16)
    _fft32_vs_dft(gpu_runtime, (((i * i + 3 * i + 1) % 11) - 5.0).astype(np.complex64), 16)
    _fft32_vs_dft(gpu_runtime, np.full(8, 2 - 0.5j, np.complex64), 8)
    _fft32_vs_dft(gpu_runtime, np.where(np.arange(8) % 2 == 0, 1.0, -1.0).astype(np.complex64), 8)
    batched = np.full(57, 31 - 31j, np.complex64)
    for b in range(3):
        for k in range(16):
            batched[b * 19 + k] = complex((b * 7 + k) / 9.0, (b * 5 - k) / 11.0)
    _fft32_vs_dft(gpu_runtime, batched, 16, batch=3, stride=19)
    r = np.array([complex(k % 9 - 4, (3 * k) % 13 - 6) for k in range(64)], np.complex64)
    rc, cs, f = gpu_runtime.fft(r, 64)
    rc, cs, back = gpu_runtime.fft(f, 64, flags=p.PROM_FFT_FLAG_INVERSE)
    assert rc == p.PROM_OK and np.abs(back - r).max() <= 3e-3


def test_fft32_element_envelope(gpu_runtime):
    # reactor_vulkan_fft.c:77: element_count * batch_count <= 65535 * 256
    x = np.zeros(4096 * 4096, np.complex64)
    rc, cs, _ = gpu_runtime.fft(x, 4096, 4096)
    assert rc == p.PROM_ERROR and (cs.stage, cs.detail) == (p.STAGE_INIT, p.PROM_FFT_DETAIL["UNSUPPORTED_SIZE"])


@pytest.mark.parametrize("n,batch,pad", [(4096, 4095, 0), (2048, 3, 5), (8192, 5, 3), (1 << 16, 4, 1),
                                         (1 << 20, 2, 7), (1 << 20, 15, 0)])
def test_fft32_large_batches(gpu_runtime, n, batch, pad):
    """One launch (n <= 4096, up to the 65535*256-element envelope) and the
    two-launch four-step (n > 4096) against numpy's binary64 FFT, forward
    and normalised inverse, padded strides."""
    stride = n + pad
    rng = np.random.default_rng(n + batch)
    x = np.full((batch - 1) * stride + n, 5 + 5j, np.complex64)
    valid = _valid_index(n, batch, stride)
    x[valid] = (rng.standard_normal(valid.size) + 1j * rng.standard_normal(valid.size)).astype(np.complex64)
    xs = x[valid].astype(np.complex128).reshape(batch, n)
    check = slice(None) if batch <= 16 else np.arange(0, batch, 97)
    for inverse in (False, True):
        out = np.full_like(x, 9 - 9j)
        rc, cs, out = gpu_runtime.fft(x, n, batch, 0 if pad == 0 else stride,
                                      p.PROM_FFT_FLAG_INVERSE if inverse else 0, output=out)
        assert rc == p.PROM_OK and cs.detail == 0
        got = out[valid].reshape(batch, n)[check].astype(np.complex128)
        ref = (np.fft.ifft if inverse else np.fft.fft)(xs[check], axis=1)
        rel = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
        print(f"fft32 n={n} batch={batch} inverse={inverse}: max rel L2 {rel.max():.2e}", flush=True)
        assert rel.max() <= 1e-6
        if pad:
            assert (np.delete(out, valid) == np.complex64(9 - 9j)).all()


def test_fft32_diagnostics_and_variant(gpu_runtime):
    x = np.zeros(32, np.complex64)
    rc, cs, _ = gpu_runtime.fft(x, 32, variant=p.PROM_FFT_BENCHMARK_VARIANT_RADIX2)
    assert rc == p.PROM_OK and cs.detail == 0
    rc, cs, _ = gpu_runtime.fft(x, 8)
    d = gpu_runtime.fft_diagnostics()
    assert d.production_enabled == 1 and d.capability_reported == 1 and d.benchmark_enabled == 1
    assert d.executed_path_id == p.PROM_FFT_PATH_VULKAN_RADIX2_RESERVED and d.executed_radix == 2
    assert d.last_failure_detail == 0 and d.plan_pass_count == 3 and d.last_effective_stride_elements == 8
    rc, cs, _ = gpu_runtime.fft(x, 8, request_patch=lambda r: setattr(r, "input", None))
    assert rc == p.PROM_ERROR and cs.detail == p.PROM_FFT_DETAIL["NULL_INPUT"]
    d = gpu_runtime.fft_diagnostics()
    assert d.last_failure_detail == p.PROM_FFT_DETAIL["NULL_INPUT"] and d.plan_valid == 0
    assert d.requested_path_id == p.PROM_FFT_PATH_NONE and d.executed_path_id == p.PROM_FFT_PATH_UNAVAILABLE


@pytest.mark.parametrize("flag,stage,name", [(p.TESTCFG_FAIL_BUFFER_ALLOC, p.STAGE_INIT, "ALLOCATION_FAILED"),
                                             (p.TESTCFG_FAIL_UPLOAD, p.STAGE_TRANSFER_IN, "UPLOAD_FAILED"),
                                             (p.TESTCFG_FAIL_DISPATCH, p.STAGE_SUBMIT, "DISPATCH_FAILED"),
                                             (p.TESTCFG_FAIL_DOWNLOAD, p.STAGE_TRANSFER_OUT, "READBACK_FAILED")])
def test_fft32_injected_faults(flag, stage, name):
    rt = p.NativeRuntime(test_flags=flag)
    try:
        assert rt.available
        out = np.full(8, 3 + 3j, np.complex64)
        rc, cs, out = rt.fft(np.ones(8, np.complex64), 8, output=out)
        assert rc == p.PROM_ERROR and (cs.stage, cs.detail) == (stage, p.PROM_FFT_DETAIL[name])
        assert rt.fft_diagnostics().executed_path_id == p.PROM_FFT_PATH_UNAVAILABLE
        if name != "READBACK_FAILED":
            assert (out == np.complex64(3 + 3j)).all()  # nothing written on failure
    finally:
        rt.close()
