"""A seeded sweep of random SGEMM shapes through the host-pointer entry
(prometheus_reactor_runtime_sgemm, reactor_sgemm.cpp:4152-4191), so that every
plan the planner can reach (tile shapes, K slices, the tail-row split, padded
copies for k or n not a multiple of 4, the GEMV) meets the parity bar on
shapes nobody picked by hand.

Bar: normwise relative error <= 1e-5 against Oct's `@` in binary64 (the
oracle's matmul_f64) on four sampled rows (first, last, two random), and the
whole product through Freivalds' check, |C x - A (B x)| <= 1e-5 |A| |B| |x|
row-wise in binary64.  Log-uniform sizes in 1..2100 per dimension, 48 shapes,
the seed fixed.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu


def _shapes(count=48, seed=20261202):
    rng = np.random.default_rng(seed)
    dims = np.exp(rng.uniform(0.0, np.log(2100.0), size=(count, 3))).astype(int) + 1
    out = [tuple(int(v) for v in row) for row in dims]
    out += [(1, 1, 1), (2049, 1, 777), (1, 1500, 3), (130, 131, 1), (257, 1023, 2099)]  # fixed corners
    return out


SHAPES = _shapes()


@pytest.mark.parametrize("m,n,k", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
def test_random_shape_parity(gpu_runtime, m, n, k):
    rng = np.random.default_rng(m * 1_000_003 + n * 1009 + k)
    a = rng.uniform(-1.0, 1.0, (m, k)).astype(np.float32)
    b = rng.uniform(-1.0, 1.0, (k, n)).astype(np.float32)
    out, status, rc = gpu_runtime.sgemm_with_status(m, n, k, a, b)
    assert rc == p.PROM_OK, status
    c = np.asarray(out, dtype=np.float32).reshape(m, n)
    assert np.all(np.isfinite(c))
    rows = sorted({0, m - 1, int(rng.integers(m)), int(rng.integers(m))})
    for r in rows:
        want = oracle.matmul_f64(a, b, rows=(r, r + 1))[r]
        assert oracle.normwise_rel_err(c[r], want) <= 1e-5, (m, n, k, r)
    x = rng.standard_normal(n)
    lhs = c.astype(np.float64) @ x
    rhs = a.astype(np.float64) @ (b.astype(np.float64) @ x)
    bound = 1e-5 * (np.abs(a).astype(np.float64) @ (np.abs(b).astype(np.float64) @ np.abs(x)))
    assert np.all(np.abs(lhs - rhs) <= bound + 1e-30), (m, n, k)
