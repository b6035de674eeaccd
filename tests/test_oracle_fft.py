"""Pins the binary64 FFT oracle (oracle/oct_oracle_fft.c) before it judges the GPU.

Sources: Language/Prometheus/gpu/fft.octest:7-28 and
Language/Prometheus/valid/fft_contract.octest:3-11 (sign, normalisation and
binary64 facts), Libraries/Mathematics/Mathematics.Transforms.octest:16-46
(length one, impulse and constant cases), closed forms, an O(n^2) DFT in
extended precision, numpy.fft (an independent implementation) and the
transform's invariants.  The agreement rule itself (internal/fft/fft.go:176-192)
is checked with planted perturbations.
"""
import numpy as np
import pytest

import oracle

TOL = 1e-12


def test_forward_sign_and_no_normalisation():
    # gpu/fft.octest:19-28
    x = np.array([0, 1, 0, 0], np.complex128)
    X = oracle.fft64(x)
    assert abs(X[0].real - 1.0) <= TOL
    assert abs(X[1].imag + 1.0) <= TOL
    assert abs(X[2].real + 1.0) <= TOL
    assert abs(X[3].imag - 1.0) <= TOL
    np.testing.assert_array_equal(x, [0, 1, 0, 0])


def test_binary64_low_bits_survive():
    # gpu/fft.octest:7-16, valid/fft_contract.octest:3-11
    delta = 0.0000000000291038304567337
    x = np.array([1.0 + delta, 1.0], np.complex128)
    X = oracle.fft64(x)
    assert X[0].real > 2.0
    assert abs(X[1].real - delta) <= 1e-15
    assert X.size == 2 and x[0].real == 1.0 + delta


def test_length_one_is_identity():
    x = np.array([3.5 - 2.25j])
    np.testing.assert_array_equal(oracle.fft64(x), x)


def test_invalid_lengths_rejected():
    for n in (0, 3, 6, 12):
        with pytest.raises(ValueError):
            oracle.fft64(np.zeros(n, np.complex128))


@pytest.mark.parametrize("n", [2, 8, 64, 1024, 4096])
def test_closed_forms(n):
    impulse = np.zeros(n, np.complex128)
    impulse[0] = 1
    np.testing.assert_allclose(oracle.fft64(impulse), np.ones(n), rtol=0, atol=TOL)
    const = np.full(n, 0.75 - 0.5j)
    expect = np.zeros(n, np.complex128)
    expect[0] = n * (0.75 - 0.5j)
    np.testing.assert_allclose(oracle.fft64(const), expect, rtol=0, atol=TOL * n)
    k0 = n // 2 - 1 if n > 2 else 1
    tone = np.exp(2j * np.pi * k0 * np.arange(n) / n)
    expect = np.zeros(n, np.complex128)
    expect[k0] = n
    np.testing.assert_allclose(oracle.fft64(tone), expect, rtol=0, atol=1e-9 * n)
    # delayed impulse: X[k] = exp(-2 pi i k d / n)
    d = 3 % n
    shifted = np.zeros(n, np.complex128)
    shifted[d] = 1
    np.testing.assert_allclose(oracle.fft64(shifted), np.exp(-2j * np.pi * np.arange(n) * d / n), rtol=0, atol=1e-12)


@pytest.mark.parametrize("n", [2, 4, 16, 32, 64])
def test_against_quadratic_dft_in_extended_precision(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    k = np.arange(n, dtype=np.longdouble)
    ang = -2 * np.pi * np.longdouble(1) * np.outer(k, k) / n
    xr, xi = x.real.astype(np.longdouble), x.imag.astype(np.longdouble)
    re = (np.cos(ang) * xr - np.sin(ang) * xi).sum(axis=1)
    im = (np.cos(ang) * xi + np.sin(ang) * xr).sum(axis=1)
    ref = (re.astype(np.float64) + 1j * im.astype(np.float64))
    assert oracle.fft64_agrees(ref, oracle.fft64(x))


@pytest.mark.parametrize("n", [2, 128, 4096, 1 << 16, 1 << 20])
def test_matches_numpy_fft(n):
    rng = np.random.default_rng(100 + n.bit_length())
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    X = oracle.fft64(x)
    assert oracle.fft64_agrees(np.fft.fft(x), X)
    # invariants: Parseval and linearity
    assert abs(np.vdot(X, X).real - n * np.vdot(x, x).real) <= 1e-10 * n * np.vdot(x, x).real
    y = rng.standard_normal(n) + 0j
    assert oracle.fft64_agrees(oracle.fft64(2 * x + 3 * y), 2 * X + 3 * oracle.fft64(y))


def test_roots_table():
    n = 1024
    tw = oracle.fft64_roots(n)
    assert tw.size == n // 2
    assert tw[0] == 1 + 0j
    assert tw[n // 4].imag == -1.0 and abs(tw[n // 4].real) < 1e-16
    np.testing.assert_allclose(tw, np.exp(-2j * np.pi * np.arange(n // 2) / n), rtol=0, atol=2e-16)


@pytest.mark.parametrize("n", [4096, 1 << 14])
def test_roots_are_two_libm_calls(n):
    """The table is cos(a) and sin(a) from two libm calls, as the reactor's
    host code computes it; at these sizes glibc's sincos differs from them in
    the last bit for at least one angle, so a build that merges the pair fails."""
    import math

    step = -2.0 * math.pi / n
    want = np.array([complex(math.cos(step * j), math.sin(step * j)) for j in range(n // 2)])
    assert np.array_equal(oracle.fft64_roots(n).view(np.uint64), want.view(np.uint64))


def test_agreement_rule_catches_planted_errors():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(256) + 1j * rng.standard_normal(256)
    ref = oracle.fft64(x)
    scale = max(np.abs(ref.real).max(), np.abs(ref.imag).max())
    ok = ref.copy()
    ok[17] += 0.5e-12 * scale
    assert oracle.fft64_agrees(ref, ok)
    bad = ref.copy()
    bad[17] += 2e-12 * scale
    assert not oracle.fft64_agrees(ref, bad)
    nan = ref.copy()
    nan[3] = complex(np.nan, 0)
    assert not oracle.fft64_agrees(ref, nan)
    # a plausible kernel mistake -- the inverse sign -- is far outside the rule
    assert not oracle.fft64_agrees(ref, np.fft.ifft(x) * 256)
