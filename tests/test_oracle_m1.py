"""Pins the Gemma-4-E2B M1 oracle (oracle/oct_oracle_m1.c).

Each stage is checked against an independent formulation: the pinned C
RMSNorm oracle and the Go witness cpuHeadRMSNorm (gemma4e2b_m1_rtx.go:811-832),
the reference's loop statement of the BF16 RoPE graph written here in Python
(gemma4e2b_m1_rtx.go:834-861), the Marionette positional formulation with
constant tables (reactor_concept_rmsnorm_tests.cpp:52-63), a binary64 dot
product for the scores, and the closed forms the reference tests use
(constant vectors give 16: reactor_concept_rmsnorm_tests.cpp:224-269).
"""
import numpy as np

import oracle


def _bf16(x):
    return oracle.from_bf16(oracle.to_bf16(np.asarray(x, np.float32)))


def test_rmsnorm_agrees_with_pinned_oracle_and_go_witness():
    x = oracle.normal(11, (40, 256))
    w = oracle.normal(12, (256,), 1.0, 0.1)
    y, inv = oracle.m1_rmsnorm(x, w, 1e-6)
    rc, y_c, inv_c = oracle.rmsnorm_reference(x, w, 1e-6)
    np.testing.assert_allclose(y, y_c, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(inv, inv_c, rtol=2e-6)
    np.testing.assert_allclose(y, oracle.m1_head_rmsnorm_go(x, w, 1e-6), rtol=2e-6, atol=1e-7)


def test_rmsnorm_rounding_flags():
    x = oracle.normal(13, (6, 64))
    w = oracle.normal(14, (64,), 1.0, 0.1)
    y_in, _ = oracle.m1_rmsnorm(x, w, 1e-6, round_in=True)
    y_pre, _ = oracle.m1_rmsnorm(_bf16(x), w, 1e-6)
    np.testing.assert_array_equal(y_in, y_pre)
    y_out, _ = oracle.m1_rmsnorm(x, w, 1e-6, round_out=True)
    np.testing.assert_array_equal(y_out, _bf16(oracle.m1_rmsnorm(x, w, 1e-6)[0]))
    assert np.all((y_out.view(np.uint32) & 0xFFFF) == 0)
    # constant row c: y = w * c / sqrt(c^2 + eps)
    c = 0.375
    y, inv = oracle.m1_rmsnorm(np.full((1, 64), c, np.float32), w, 1e-6)
    np.testing.assert_allclose(y[0], w * c / np.sqrt(c * c + 1e-6), rtol=1e-6)


def _rope_loop(source, cos, sin, tokens, heads, width=256):
    out = np.zeros_like(source)
    half = width // 2
    for t in range(tokens):
        for h in range(heads):
            base = (t * heads + h) * width
            for comp in range(width):
                f = comp % half
                mate = base + f + half if comp < half else base + f
                first = _bf16(np.float32(source[base + comp]) * np.float32(cos[t * width + f])).item()
                second = _bf16(np.float32(source[mate]) * np.float32(sin[t * width + f])).item()
                value = np.float32(first) - np.float32(second) if comp < half else np.float32(first) + np.float32(second)
                out[base + comp] = _bf16(value).item()
    return out


def test_rope_matches_reference_loop():
    src = _bf16(oracle.normal(15, (15 * 8 * 256,)))
    ang = np.outer(np.arange(15), 1.0 / 10000 ** (np.arange(256) % 128 * 2 / 256))
    cos, sin = _bf16(np.cos(ang).reshape(-1)), _bf16(np.sin(ang).reshape(-1))
    np.testing.assert_array_equal(oracle.m1_rope(src, cos, sin, 15, 8), _rope_loop(src, cos, sin, 15, 8))
    k = src[: 15 * 256]
    np.testing.assert_array_equal(oracle.m1_rope(k, cos, sin, 15, 1), _rope_loop(k, cos, sin, 15, 1))


def test_rope_closed_forms():
    src = _bf16(oracle.normal(16, (15 * 256,)))
    ones, zeros = np.ones(3840, np.float32), np.zeros(3840, np.float32)
    # identity rotation keeps BF16 values
    np.testing.assert_array_equal(oracle.m1_rope(src, ones, zeros, 15, 1), src)
    # quarter turn: first half -> -mate, second half -> +mate
    out = oracle.m1_rope(src, zeros, ones, 15, 1).reshape(15, 256)
    s = src.reshape(15, 256)
    np.testing.assert_array_equal(out[:, :128], -s[:, 128:])
    np.testing.assert_array_equal(out[:, 128:], s[:, :128])


def test_positional_matches_marionette_formulation():
    # reactor_concept_rmsnorm_tests.cpp:52-63 with cosine 0.75, sine 0.5
    i = np.arange(15 * 8 * 256)
    q = ((i * 13 % 61) - 30).astype(np.float32) / np.float32(71.0)
    w = (0.75 + (np.arange(256) % 5) / 32).astype(np.float32)
    norm, _ = oracle.m1_rmsnorm(q.reshape(120, 256), w, 1e-6, True, True)
    n = norm.reshape(-1)
    comp = i % 256
    pair = np.where(comp < 128, i + 128, i - 128)
    a = _bf16(n * np.float32(0.75))
    b = _bf16(n[pair] * np.float32(0.5))
    expect = _bf16(np.where(comp < 128, a - b, a + b))
    got = oracle.m1_positional(q, w, np.full(3840, 0.75, np.float32), np.full(3840, 0.5, np.float32), 8)
    np.testing.assert_array_equal(got, expect)


def test_scores_against_binary64_and_constant_fact():
    q = oracle.normal(17, (15 * 8 * 256,))
    k = oracle.normal(18, (15 * 256,))
    s = oracle.m1_raw_scores(q, k).reshape(8, 15, 15)
    Q = q.reshape(15, 8, 256).astype(np.float64)
    K = k.reshape(15, 256).astype(np.float64)
    ref = np.einsum("ihc,jc->hij", Q, K) * 0.0625
    np.testing.assert_allclose(s, ref, rtol=1e-5, atol=1e-5)
    ones_q, ones_k = np.ones(15 * 8 * 256, np.float32), np.ones(15 * 256, np.float32)
    w, c, z = np.ones(256, np.float32), np.ones(3840, np.float32), np.zeros(3840, np.float32)
    scores = oracle.m1_raw_scores(oracle.m1_positional(ones_q, w, c, z, 8), oracle.m1_positional(ones_k, w, c, z, 1))
    assert np.all(scores == 16.0)
