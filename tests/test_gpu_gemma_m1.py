"""GPU parity of the Gemma-4-E2B M1 entry points against the CPU oracle.

Restates the reference's facts for these entries
(native/Marionette/reactor_concept_rmsnorm_tests.cpp:70-140 weight publication,
rounding flags and stale generations; :146-216 the resident head chain feeding
the scores; :224-269 constant vectors; :331-380 standalone RoPE), with the
reference's bars: outputs within 1e-4 absolute, inverse RMS within 1e-5,
scores within 1e-3.  Each test uses its own runtime because the committed
weight generation is per runtime and must increase.
"""
import ctypes

import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu


@pytest.fixture
def rt():
    with p.NativeRuntime() as r:
        r.require_hardware_gpu()
        yield r


def _rms_request(x, w, y, inv, rows, width, stride, gen):
    r = p.PrometheusGemma4E2BM1InputRmsNormRequest()
    r.struct_size = ctypes.sizeof(r)
    r.input, r.weight, r.output, r.inv_rms_output = x.ctypes.data, w.ctypes.data, y.ctypes.data, inv.ctypes.data
    r.input_element_count, r.weight_element_count = rows * stride, width
    r.output_element_count, r.inv_rms_output_element_count = rows * width, rows
    r.tokens, r.model_width, r.input_row_stride, r.epsilon = rows, width, stride, 1e-6
    r.input_generation, r.weight_generation, r.exact_source_hash = 1, gen, 0x52A1
    return r


@pytest.mark.parametrize("width", [31, 1536, 4096])
def test_rmsnorm_family_widths_generations(rt, width):
    # reactor_concept_rmsnorm_tests.cpp:82-124: rows 3, stride width + 7, the test's generators
    rows, stride = 3, width + 7
    i = np.arange(rows * stride)
    x = (((i * 7) % 31) - 15).astype(np.float32) / np.float32(63.0)
    w = (0.75 + (np.arange(width) % 7) / 64).astype(np.float32)
    gen = 0
    for name, round_out in (("input_rmsnorm", False), ("projection_activation_rmsnorm", True)):
        fn = getattr(rt.lib, f"prometheus_reactor_runtime_gemma4e2b_m1_{name}")
        y, inv = np.zeros((rows, width), np.float32), np.zeros(rows, np.float32)
        gen += 1
        req = _rms_request(x, w, y, inv, rows, width, stride, gen)
        res = p.PrometheusGemma4E2BM1InputRmsNormResult()
        assert fn(rt.handle, ctypes.byref(req), ctypes.byref(res)) == p.PROM_OK
        assert (res.stage, res.detail_code, res.output_written) == (0, 0, 1)
        y_ref, inv_ref = oracle.m1_rmsnorm(x.reshape(rows, stride), w, 1e-6, False, round_out, width=width)
        assert np.max(np.abs(y - y_ref)) < 1e-4
        assert np.max(np.abs(inv - inv_ref)) < 1e-5
        if round_out:
            assert np.all((y.view(np.uint32) & 0xFFFF) == 0)
        first_hash = res.output_hash
        # the same generation again is stale and changes nothing
        y2 = np.full_like(y, -7.0)
        req2 = _rms_request(x, w, y2, inv, rows, width, stride, gen)
        res2 = p.PrometheusGemma4E2BM1InputRmsNormResult()
        assert fn(rt.handle, ctypes.byref(req2), ctypes.byref(res2)) == p.PROM_ERROR
        assert (res2.stage, res2.detail_code) == (p.STAGE_TRANSFER_IN, p.DETAIL_M46_STALE_WEIGHT_GENERATION)
        assert np.all(y2 == -7.0)
        # a newer generation repeats bit-identically (warm output is bitwise stable)
        gen += 1
        req3 = _rms_request(x, w, y2, inv, rows, width, stride, gen)
        assert fn(rt.handle, ctypes.byref(req3), ctypes.byref(res2)) == p.PROM_OK
        assert res2.output_hash == first_hash
        np.testing.assert_array_equal(y2, y)
    # a non-finite candidate weight is rejected and the committed generation is kept
    w_bad = w.copy()
    w_bad[0] = np.nan
    req = _rms_request(x, w_bad, y, inv, rows, width, stride, gen + 1)
    res = p.PrometheusGemma4E2BM1InputRmsNormResult()
    assert rt.lib.prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm(rt.handle, ctypes.byref(req),
                                                                         ctypes.byref(res)) == p.PROM_ERROR
    assert res.detail_code == p.DETAIL_M46_NONFINITE_INPUT
    req = _rms_request(x, w, y, inv, rows, width, stride, gen + 1)
    assert rt.lib.prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm(rt.handle, ctypes.byref(req),
                                                                         ctypes.byref(res)) == p.PROM_OK


def test_head_rmsnorm_rounds_in_and_out(rt):
    rows = 120
    x = oracle.normal(21, (rows, 256))
    w = oracle.normal(22, (256,), 1.0, 0.05)
    y, inv = np.zeros_like(x), np.zeros(rows, np.float32)
    req = _rms_request(x, w, y, inv, rows, 256, 256, 1)
    res = p.PrometheusGemma4E2BM1InputRmsNormResult()
    assert rt.lib.prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm(rt.handle, ctypes.byref(req),
                                                                        ctypes.byref(res)) == p.PROM_OK
    y_ref, inv_ref = oracle.m1_rmsnorm(x, w, 1e-6, True, True)
    assert np.max(np.abs(y - y_ref)) < 1e-4 and np.max(np.abs(inv - inv_ref)) < 1e-5
    assert np.mean(y == y_ref) > 0.999


def _tables(kind):
    if kind == "marionette":
        return np.full(3840, 0.75, np.float32), np.full(3840, 0.5, np.float32)
    ang = np.outer(np.arange(15), 1.0 / 10000.0 ** ((np.arange(256) % 128) * 2.0 / 256))
    bf = lambda v: oracle.from_bf16(oracle.to_bf16(v.astype(np.float32)))
    return bf(np.cos(ang).reshape(-1)), bf(np.sin(ang).reshape(-1))


@pytest.mark.parametrize("heads", [1, 8])
@pytest.mark.parametrize("tables", ["marionette", "rope"])
def test_standalone_rope_bit_identical(rt, heads, tables):
    cos, sin = _tables(tables)
    src = oracle.from_bf16(oracle.to_bf16(oracle.normal(23 + heads, (15 * heads * 256,))))
    out = np.zeros_like(src)
    r = p.PrometheusGemma4E2BM1RopeRequest()
    r.struct_size = ctypes.sizeof(r)
    r.source, r.cosine, r.sine, r.output = src.ctypes.data, cos.ctypes.data, sin.ctypes.data, out.ctypes.data
    r.source_element_count = r.output_element_count = src.size
    r.cosine_element_count = r.sine_element_count = 3840
    r.tokens, r.heads, r.head_width = 15, heads, 256
    r.source_generation = r.table_generation = 1
    res = p.PrometheusGemma4E2BM1RopeResult()
    assert rt.lib.prometheus_reactor_runtime_gemma4e2b_m1_rope(rt.handle, ctypes.byref(r), ctypes.byref(res)) == 0
    assert (res.stage, res.detail_code, res.output_written, res.dispatch_count) == (0, 0, 1, 1)
    np.testing.assert_array_equal(out, oracle.m1_rope(src, cos, sin, 15, heads))


def _marionette_qk():
    # reactor_concept_rmsnorm_tests.cpp:152-156
    i = np.arange(15 * 8 * 256)
    q = ((i * 13 % 61) - 30).astype(np.float32) / np.float32(71.0)
    j = np.arange(15 * 256)
    k = ((j * 7 % 41) - 20).astype(np.float32) / np.float32(53.0)
    w = (0.75 + (np.arange(256) % 5) / 32).astype(np.float32)
    return q, k, w


def _head_rope_request(x, w, cos, sin, out, heads, gen):
    h = p.PrometheusGemma4E2BM1HeadRmsNormRopeRequest()
    h.struct_size = ctypes.sizeof(h)
    h.input, h.weight, h.cosine, h.sine = x.ctypes.data, w.ctypes.data, cos.ctypes.data, sin.ctypes.data
    h.output = out.ctypes.data if out is not None else None
    h.input_element_count, h.weight_element_count = x.size, 256
    h.cosine_element_count = h.sine_element_count = 3840
    h.output_element_count = out.size if out is not None else 0
    h.tokens, h.heads, h.head_width, h.epsilon = 15, heads, 256, 1e-6
    h.input_generation, h.weight_generation, h.table_generation, h.exact_source_hash = 1, gen, 1, 11
    return h


def test_head_rmsnorm_rope_matches_positional_oracle(rt):
    q, k, w = _marionette_qk()
    cos, sin = _tables("marionette")
    out = np.zeros_like(q)
    res = p.PrometheusGemma4E2BM1HeadRmsNormRopeResult()
    req = _head_rope_request(q, w, cos, sin, out, 8, 1)
    assert rt.lib.prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm_rope(rt.handle, ctypes.byref(req),
                                                                             ctypes.byref(res)) == 0
    expect = oracle.m1_positional(q, w, cos, sin, 8)
    assert np.max(np.abs(out - expect)) < 1e-4
    assert res.normalized_readback_count == 0 and res.output_written == 1
    # resident-only form: no output array
    req = _head_rope_request(k, w, cos, sin, None, 1, 2)
    assert rt.lib.prometheus_reactor_runtime_gemma4e2b_m1_head_rmsnorm_rope(rt.handle, ctypes.byref(req),
                                                                             ctypes.byref(res)) == 0
    assert res.output_written == 0 and res.output_hash == 1


def _scores_request(q, k, wq, wk, cos, sin, scores, order, gq, gk):
    a = p.PrometheusGemma4E2BM1AttentionScoresRequest()
    a.struct_size = ctypes.sizeof(a)
    a.query_input, a.key_input, a.query_weight, a.key_weight = q.ctypes.data, k.ctypes.data, wq.ctypes.data, wk.ctypes.data
    a.cosine, a.sine, a.scores = cos.ctypes.data, sin.ctypes.data, scores.ctypes.data
    a.query_input_element_count, a.key_input_element_count = q.size, k.size
    a.query_weight_element_count = a.key_weight_element_count = 256
    a.cosine_element_count = a.sine_element_count = 3840
    a.score_element_count = scores.size
    a.tokens, a.query_heads, a.key_heads, a.head_width, a.epsilon, a.scale = 15, 8, 1, 256, 1e-6, 0.0625
    a.preparation_order = order
    a.query_input_generation, a.key_input_generation, a.table_generation = 1, 2, 1
    a.query_weight_generation, a.key_weight_generation = gq, gk
    a.query_exact_source_hash, a.key_exact_source_hash = 11, 12
    return a


def test_attention_scores_both_preparation_orders(rt):
    # reactor_concept_rmsnorm_tests.cpp:146-216
    q, k, w = _marionette_qk()
    cos, sin = _tables("marionette")
    eq, ek = oracle.m1_positional(q, w, cos, sin, 8), oracle.m1_positional(k, w, cos, sin, 1)
    expected = (np.einsum("ihc,jc->hij", eq.reshape(15, 8, 256).astype(np.float64),
                          ek.reshape(15, 256).astype(np.float64)) * 0.0625).reshape(-1)
    for order, gq, gk in ((0, 2, 3), (1, 5, 4)):
        scores = np.full(1800, -99, np.float32)
        req = _scores_request(q, k, w, w, cos, sin, scores, order, gq, gk)
        res = p.PrometheusGemma4E2BM1AttentionScoresResult()
        assert rt.lib.prometheus_reactor_runtime_gemma4e2b_m1_attention_scores(rt.handle, ctypes.byref(req),
                                                                                ctypes.byref(res)) == 0
        assert np.max(np.abs(scores - expected)) < 1e-3
        np.testing.assert_allclose(scores, oracle.m1_raw_scores(eq, ek), rtol=0, atol=1e-5)
        assert res.host_detour_count == 0 and res.score_readback_count == 1 and res.positional_dispatch_count == 2
        assert len({res.query_slot_id, res.key_slot_id, res.score_slot_id}) == 3
    # reusing a committed generation is stale (the query weight is prepared first in order 0)
    scores = np.full(1800, -99, np.float32)
    req = _scores_request(q, k, w, w, cos, sin, scores, 0, 5, 6)
    res = p.PrometheusGemma4E2BM1AttentionScoresResult()
    assert rt.lib.prometheus_reactor_runtime_gemma4e2b_m1_attention_scores(rt.handle, ctypes.byref(req),
                                                                            ctypes.byref(res)) == 1
    assert res.detail_code == p.DETAIL_M46_STALE_WEIGHT_GENERATION and np.all(scores == -99)


def test_attention_scores_constant_vectors_give_sixteen(rt):
    # reactor_concept_rmsnorm_tests.cpp:224, 268-269
    q, k = np.ones(15 * 8 * 256, np.float32), np.ones(15 * 256, np.float32)
    w, cos, sin = np.ones(256, np.float32), np.ones(3840, np.float32), np.zeros(3840, np.float32)
    scores = np.full(1800, -99, np.float32)
    req = _scores_request(q, k, w, w, cos, sin, scores, 0, 1, 2)
    res = p.PrometheusGemma4E2BM1AttentionScoresResult()
    assert rt.lib.prometheus_reactor_runtime_gemma4e2b_m1_attention_scores(rt.handle, ctypes.byref(req),
                                                                            ctypes.byref(res)) == 0
    assert np.all(scores == 16.0)
