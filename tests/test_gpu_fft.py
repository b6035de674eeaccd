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
