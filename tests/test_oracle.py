"""Pins the CPU oracle against the reference's known answers and mathematics.

The oracle (oracle/oct_oracle.c) is the parity checker for the HIP reactor, so
it is itself checked against: the reference's KATs and golden fixtures,
exact rational arithmetic, closed forms, and invariants chosen so that a
dropped term, a transposed operand or a wrong index fails.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle
from tests.golden import octagon


# --------------------------------------------------------------------- `@`
def test_kat_runtime_test_2x2():
    # internal/prometheus/runtime_test.go:180-203
    a = np.array([[1, 2], [3, 4]], dtype=np.float64)
    b = np.array([[5, 6], [7, 8]], dtype=np.float64)
    np.testing.assert_array_equal(oracle.matmul_f64(a, b), [[19, 22], [43, 50]])
    np.testing.assert_array_equal(oracle.matmul_f64(a.astype(np.float32), b.astype(np.float32)), [[19, 22], [43, 50]])
    np.testing.assert_array_equal(oracle.matmul_compiled_f64(a, b), [[19, 22], [43, 50]])
    np.testing.assert_array_equal(oracle.cpu_sgemm_f32(a, b), [[19, 22], [43, 50]])


def test_kat_strict_matrix_octest():
    # Language/Prometheus/gpu/matrix.octest:3-9: (a @ a)[0,0] == 7
    a = np.array([[1.0, 2.0], [3.0, 4.0]])
    assert oracle.matmul_f64(a, a)[0, 0] == 7.0


def _exact_product(a, b):
    m, k = a.shape
    n = b.shape[1]
    fa = [[Fraction(float(x)) for x in row] for row in a]
    fb = [[Fraction(float(x)) for x in row] for row in b]
    return [[sum(fa[i][t] * fb[t][j] for t in range(k)) for j in range(n)] for i in range(m)]


def _sequential_f64(a, b):
    # Independent restatement of the evaluation order with Python floats
    # (IEEE binary64, no fused multiply-add).
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            acc = float(a[i, 0]) * float(b[0, j])
            for t in range(1, k):
                acc = acc + float(a[i, t]) * float(b[t, j])
            out[i, j] = acc
    return out


STARTER_CORPUS = [(1, 1, 1), (4, 4, 4), (16, 16, 16), (32, 32, 32), (3, 5, 7)]  # runtime.go:83-89
STUB_CORPUS = [(1, 1, 1), (4, 4, 4), (3, 7, 5), (1, 9, 4), (11, 1, 3), (2, 13, 3)]  # reactor_stub_tests.cpp:224-231


@pytest.mark.parametrize("m,n,k", sorted(set(STARTER_CORPUS + STUB_CORPUS)))
def test_deterministic_corpus_exact(m, n, k):
    a = oracle.deterministic_matrix(m, k)
    b = oracle.deterministic_matrix(k, n)
    # generator: ((i % 23) - 11) / 7 rounded to fp32 (runtime.go:242-249)
    flat = np.array([np.float32(((i % 23) - 11) / np.float32(7)) for i in range(m * k)], dtype=np.float32)
    np.testing.assert_array_equal(a.reshape(-1), flat)
    got = oracle.matmul_f64(a, b)
    # bit-exact against the independent sequential restatement
    np.testing.assert_array_equal(got, _sequential_f64(a.astype(np.float64), b.astype(np.float64)))
    # and within a few ulps of the exact rational product
    exact = _exact_product(a, b)
    for i in range(m):
        for j in range(n):
            assert abs(got[i, j] - float(exact[i][j])) <= 1e-14 * max(1.0, abs(float(exact[i][j]))) * k


def test_closed_forms_identity_diagonal_rank1():
    rng = np.random.default_rng(7)
    a = rng.standard_normal((9, 6)).astype(np.float32)
    eye = np.eye(6, dtype=np.float32)
    np.testing.assert_array_equal(oracle.matmul_f64(a, eye), a.astype(np.float64))
    d = np.diag(np.arange(1, 7, dtype=np.float32))
    np.testing.assert_array_equal(oracle.matmul_f64(a, d), a.astype(np.float64) * np.arange(1, 7))
    u = rng.integers(-5, 5, (7, 1)).astype(np.float32)
    v = rng.integers(-5, 5, (1, 5)).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_f64(u, v), u.astype(np.float64) * v.astype(np.float64))


def test_transpose_identity_catches_swapped_operands():
    a = oracle.uniform(11, (5, 7))
    b = oracle.uniform(12, (7, 3))
    ab = oracle.matmul_f64(a, b)
    btat = oracle.matmul_f64(np.ascontiguousarray(b.T), np.ascontiguousarray(a.T))
    np.testing.assert_allclose(ab, btat.T, rtol=1e-13, atol=1e-13)
    assert ab.shape == (5, 3)


def test_thread_count_and_row_subset_are_bit_identical():
    a = oracle.uniform(1, (37, 61))
    b = oracle.uniform(2, (61, 29))
    ref = oracle.matmul_f64(a, b, threads=1)
    np.testing.assert_array_equal(ref, oracle.matmul_f64(a, b, threads=7))
    sub = oracle.matmul_f64(a, b, rows=(5, 9), threads=3)
    np.testing.assert_array_equal(sub[5:9], ref[5:9])
    assert not sub[:5].any() and not sub[9:].any()


def test_compiled_and_interpreted_orders_agree():
    # acc starts at 0 (compiled) vs first term (interpreted): identical except -0.
    a = oracle.uniform(3, (8, 33)).astype(np.float64)
    b = oracle.uniform(4, (33, 6)).astype(np.float64)
    np.testing.assert_array_equal(oracle.matmul_compiled_f64(a, b), oracle.matmul_f64(a, b))


def test_concept_sgemm_corpus_binary64_tolerance():
    # reactor_concept_sgemm_tests.cpp:17-29: ((i*7+seed)%23-11)/8, 37x29x13, binary64 within 1e-4
    m, n, k = 37, 29, 13
    a = oracle.concept_sgemm_matrix(m * k, 3).reshape(m, k)
    b = oracle.concept_sgemm_matrix(k * n, 5).reshape(k, n)
    assert a[0, 0] == ((3 % 23) - 11) / 8
    f32 = oracle.cpu_sgemm_f32(a, b)
    f64 = oracle.matmul_f64(a, b)
    assert np.max(np.abs(f32 - f64)) <= 1e-4


def test_cpu_sgemm_f32_is_sequential_float32():
    a = oracle.uniform(5, (3, 17))
    b = oracle.uniform(6, (17, 4))
    out = np.zeros((3, 4), dtype=np.float32)
    for i in range(3):
        for j in range(4):
            s = np.float32(0)
            for t in range(17):
                s = np.float32(s + np.float32(a[i, t] * b[t, j]))
            out[i, j] = s
    np.testing.assert_array_equal(oracle.cpu_sgemm_f32(a, b), out)


def test_compare_against_oracle_thresholds():
    # runtime.go:339-376: fail only when abs > 1e-4 AND rel > 1e-4, or non-finite
    e = np.array([1.0, 100.0, 0.0, 1.0], dtype=np.float32)
    ok = oracle.compare_against_oracle(e, e + np.array([5e-5, 5e-3, 0, 0], dtype=np.float32))
    assert ok.pass_ == 1
    bad = oracle.compare_against_oracle(e, e + np.array([0, 0.02, 0, 0], dtype=np.float32))
    assert bad.pass_ == 0 and bad.first_failing_index == 1
    nan = oracle.compare_against_oracle(e, np.array([1, 100, np.nan, 1], dtype=np.float32))
    assert nan.pass_ == 0 and nan.first_failing_index == 2


def test_normwise_error_metric():
    e = np.array([3.0, 4.0])
    a = np.array([3.0, 4.5], dtype=np.float32)
    assert abs(oracle.normwise_rel_err(a, e) - 0.1) < 1e-12


def test_generators_are_seeded_and_in_range():
    u = oracle.uniform(42, (1000,))
    assert np.array_equal(u, oracle.uniform(42, (1000,)))
    assert not np.array_equal(u, oracle.uniform(43, (1000,)))
    assert u.min() >= -1 and u.max() < 1 and abs(u.mean()) < 0.1
    z = oracle.normal(9, (200000,))
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_bf16_rounding_rne():
    # gemma4e2b_m1_rtx.go:1009-1014: bits + 0x7FFF + lsb, truncate
    vals = np.array([1.0, 1.00390625, 1.01171875, -3.140625, 65504.0], dtype=np.float32)
    bits = oracle.to_bf16(vals)
    expect = []
    for v in vals:
        u = int(np.float32(v).view(np.uint32))
        expect.append(((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF)
    np.testing.assert_array_equal(bits, np.array(expect, dtype=np.uint16))
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: round to even -> 1
    assert oracle.from_bf16(oracle.to_bf16(np.array([1.00390625], np.float32)))[0] == 1.0


def test_bf16_matmul_equals_widened_f64():
    a = oracle.to_bf16(oracle.uniform(1, (6, 9)))
    b = oracle.to_bf16(oracle.uniform(2, (9, 4)))
    np.testing.assert_array_equal(oracle.matmul_f64(a, b),
                                  oracle.matmul_f64(oracle.from_bf16(a), oracle.from_bf16(b)))


# --------------------------------------------------------------- reductions
def test_reduction_kats_fused_reduction_semantics():
    # Language/SDSL-V/M39b/FusedReductionSemantics.sdslvtest:6-95
    d, s = oracle.reduction_reference(np.array([[1.5, -2.0, 4.25]]), 1)
    assert d == 0 and abs(s[0] - 3.75) <= 1e-5
    d, s = oracle.reduction_reference(np.array([[-7.5]]), 1)
    assert s[0] == -7.5
    d, mx = oracle.reduction_reference(np.array([[-9.0, -4.0, -12.0, -4.5, -20.0]]), 2)
    assert mx[0] == -4.0
    for vals in ([10000.0, 10001.0, 9999.0, 10000.0], [-10000.0, -9999.0, -10001.0, -10000.0]):
        d, y = oracle.reduction_reference(np.array([vals]), 3)
        assert abs(y.sum() - 1.0) <= 1e-4 and y[0, 1] > y[0, 0] and y[0, 2] >= 0
    d, y = oracle.reduction_reference(np.array([[7.0] * 4]), 3)
    assert np.all(np.abs(y - 0.25) <= 1e-5)
    d, y = oracle.reduction_reference(np.array([[80.0, -80.0, -80.0, -80.0]]), 3)
    assert abs(y[0, 0] - 1.0) <= 1e-5


def test_reduction_rejects_nonfinite_and_bad_ops():
    x = np.ones((2, 3), np.float32)
    x[1, 2] = np.inf
    assert oracle.reduction_reference(x, 1)[0] == -6814
    assert oracle.reduction_reference(np.ones((2, 3), np.float32), 4)[0] == -6806


def test_softmax_matches_captured_attention_row():
    # Experiments/ZImageTurboNoiseRefiner0/M5/Attention.octest: 1024 logits, expected
    # probabilities computed by Oct in binary64 (tolerance 2e-8).  The oracle rounds
    # to fp32, so each value may also differ by half an fp32 ulp.
    w = octagon.load("attention_token0_head0.octagon")
    logits = w["Logits"].astype(np.float32)[None, :]
    d, y = oracle.reduction_reference(logits, 3)
    assert d == 0
    tol = 2e-8 + np.abs(w["Expected"]) * 2.0 ** -24
    assert np.all(np.abs(y[0].astype(np.float64) - w["Expected"]) <= tol)


def test_sum_matches_binary64_accumulation_and_max_is_exact():
    x = oracle.reduction_input(5, 77, bias=0.25)
    # generator: ((row*29 + col*17) % 101 - 50)/16 + bias (reactor_reduction_tests.cpp:78-87)
    assert x[1, 2] == np.float32(0.25 + ((29 + 34) % 101 - 50) / 16)
    d, s = oracle.reduction_reference(x, 1)
    np.testing.assert_array_equal(s, x.astype(np.float64).sum(axis=1).astype(np.float32))
    d, m = oracle.reduction_reference(x, 2)
    np.testing.assert_array_equal(m, x.max(axis=1))


def test_softmax_invariants_shift_and_order():
    x = oracle.normal(3, (4, 300))
    d, y = oracle.reduction_reference(x, 3)
    d2, y2 = oracle.reduction_reference(x + np.float32(5.0), 3)
    np.testing.assert_allclose(y, y2, rtol=2e-5, atol=1e-9)
    np.testing.assert_allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)
    order = np.argsort(x[0])
    assert np.all(np.diff(y[0][order]) >= -1e-9)


def test_reduction_compare_thresholds():
    shape = (1, 4)
    e = np.array([0.25, 0.25, 0.25, 0.25], np.float32)
    assert oracle.reduction_compare(shape, 3, e, e)[0] == 0
    rc, mm = oracle.reduction_compare(shape, 3, e, np.array([0.26, 0.24, 0.25, 0.25], np.float32))
    assert rc == 1 and mm.column == 0
    # row sum check: each element within abs 2e-5 but the row sum off by >3e-4 cannot
    # happen at width 4; use a wide row.
    e = np.full((1, 40), 1 / 40, np.float32)
    a = e + np.float32(1.9e-5)
    rc, mm = oracle.reduction_compare((1, 40), 3, e.reshape(-1), a.reshape(-1))
    assert rc == 1 and mm.column == 0xFFFFFFFF
    # max is exact
    assert oracle.reduction_compare((2, 8), 2, np.array([1, 2], np.float32), np.array([1, np.nextafter(np.float32(2), np.float32(3))], np.float32))[0] == 1
    # sum tolerance abs 2e-5*width
    assert oracle.reduction_compare((1, 1000), 1, np.array([1.0], np.float32), np.array([1.019], np.float32))[0] == 0


# ------------------------------------------------------------------ RMSNorm
def test_rmsnorm_matches_captured_qnorm_row():
    # Experiments/ZImageTurboNoiseRefiner0/M4/RmsNorm.octest: eps 1e-5, 2e-6
    w = octagon.load("qnorm_row0_head0.octagon")
    z = w["Input"].astype(np.float32)[None, :]
    rc, y, inv = oracle.rmsnorm_reference(z, w["Scale"].astype(np.float32), 1e-5)
    assert rc == 0
    assert np.max(np.abs(y[0].astype(np.float64) - w["Expected"])) <= 2e-6


def test_rmsnorm_constant_row_closed_form():
    c, eps = np.float32(3.0), 1e-6
    z = np.full((2, 64), c, np.float32)
    wt = np.linspace(0.5, 1.5, 64, dtype=np.float32)
    rc, y, inv = oracle.rmsnorm_reference(z, wt, eps)
    expect = wt.astype(np.float64) * 3.0 / np.sqrt(9.0 + eps)
    np.testing.assert_allclose(y[0], expect, rtol=3e-7)
    # no mean subtraction: a shifted row is not normalised to zero mean
    z2 = z + np.arange(64, dtype=np.float32)
    rc, y2, _ = oracle.rmsnorm_reference(z2, np.ones(64, np.float32), eps)
    assert y2[0].mean() > 0.5


def test_rmsnorm_stride_and_rejections():
    z = oracle.normal(1, (3, 10))
    rc, y, _ = oracle.rmsnorm_reference(z, np.ones(8, np.float32), 1e-6, width=8)
    rc2, y2, _ = oracle.rmsnorm_reference(np.ascontiguousarray(z[:, :8]), np.ones(8, np.float32), 1e-6)
    assert rc == 0 and rc2 == 0
    np.testing.assert_array_equal(y, y2)
    bad = z.copy()
    bad[0, 0] = np.nan
    assert oracle.rmsnorm_reference(bad, np.ones(10, np.float32), 1e-6)[0] == 1
    assert oracle.rmsnorm_reference(z, np.ones(10, np.float32), 0.0)[0] == 1
