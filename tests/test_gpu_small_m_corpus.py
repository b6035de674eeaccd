"""The reference's small-M production SGEMM corpus on the reactor
(internal/prometheus/gemma4e2b_sgemm_corpus_test.go:29-96, generators
:98-113): Gemma-4-E2B-shaped products with 1-33 rows, fp32 A and
bf16-valued B, through the host-pointer SGEMM with status.  Gate as in the
reference: compareAgainstOracle (runtime.go:319-376) against the fp32
sequential-k product (cpuMatmulRowMajor, gemma4e2b_m1_rtx.go:795-809, the
same loop as the oracle's oct_cpu_sgemm_f32), and every output finite.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p

CASES = [  # gemma4e2b_sgemm_corpus_test.go:44-59
    ("m1_n256_k1536", 1, 256, 1536),
    ("m2_n256_k1536", 2, 256, 1536),
    ("m7_n256_k1536", 7, 256, 1536),
    ("m15_n256_k1536", 15, 256, 1536),
    ("m16_n256_k1536", 16, 256, 1536),
    ("m17_n256_k1536", 17, 256, 1536),
    ("m31_n256_k1536", 31, 256, 1536),
    ("m32_n256_k1536", 32, 256, 1536),
    ("m33_n256_k1536", 33, 256, 1536),
    ("canonical_q_m15_n2048_k1536", 15, 2048, 1536),
    ("compact_exhaustive_m17_n19_k17", 17, 19, 17),
    ("alternate_m15_n256_k1536", 15, 256, 1536),
    ("alternate_m32_n256_k1536", 32, 256, 1536),
    ("alternate_m15_repeat_n256_k1536", 15, 256, 1536),
]


def deterministic_corpus_fp32(count: int) -> np.ndarray:
    """:98-104: float32((i*17)%101 - 50) / 31 in float32."""
    i = np.arange(count, dtype=np.int64)
    return (((i * 17) % 101 - 50).astype(np.float32) / np.float32(31.0)).astype(np.float32)


def deterministic_corpus_bf16(count: int) -> np.ndarray:
    """:106-113: float32((i*29)%127 - 63) / 37, rounded to bf16 (RNE) and back."""
    i = np.arange(count, dtype=np.int64)
    v = (((i * 29) % 127 - 63).astype(np.float32) / np.float32(37.0)).astype(np.float32)
    return oracle.from_bf16(oracle.to_bf16(v))


def test_generators_first_values():
    a = deterministic_corpus_fp32(4)
    assert a.tolist() == [np.float32(-50) / np.float32(31), np.float32(-33) / np.float32(31),
                          np.float32(-16) / np.float32(31), np.float32(1) / np.float32(31)]
    b = deterministic_corpus_bf16(3)
    bits = b.view(np.uint32)
    assert np.all(bits & 0xFFFF == 0)  # bf16-representable
    assert np.all(np.abs(b - (np.array([-63, -34, -5], np.float32) / np.float32(37))) <= 2.0 ** -8)


@pytest.mark.gpu
@pytest.mark.parametrize("name,m,n,k", CASES, ids=[c[0] for c in CASES])
def test_small_m_production_corpus(gpu_runtime, name, m, n, k):
    a = deterministic_corpus_fp32(m * k).reshape(m, k)
    b = deterministic_corpus_bf16(k * n).reshape(k, n)
    reference = oracle.cpu_sgemm_f32(a, b)
    out, status, rc = gpu_runtime.sgemm_with_status(m, n, k, a, b)
    assert rc == p.PROM_OK, (name, status)
    actual = np.asarray(out, dtype=np.float32).reshape(m, n)
    policy = oracle.compare_against_oracle(reference, actual)
    assert np.all(np.isfinite(actual)), name
    assert policy.pass_ == 1, (name, policy.failing_count, policy.first_failing_index, policy.max_abs_error,
                               policy.max_rel_error)
