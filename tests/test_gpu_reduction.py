"""GPU parity of the fused row reductions and RMSNorm against the CPU oracle.

Bar: normwise relative error <= 1e-5 (north_star) and the reference's own
comparator (prom_reduction_compare: softmax abs 2e-5/rel 2e-4 plus row sums;
sum abs 2e-5*width/rel 2e-5; max exact), on the reference's generators,
KATs, the captured witness rows, and the C3 shape [8192, 4096].
"""
import ctypes

import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p
from tests.golden import octagon

pytestmark = pytest.mark.gpu

NORMWISE = 1e-5


def _check(x, op, got):
    d, ref = oracle.reduction_reference(x, op)
    assert d == 0
    rc, mm = oracle.reduction_compare(x.shape, op, ref.reshape(-1), np.asarray(got).reshape(-1))
    assert rc == 0, (mm.row, mm.column, mm.expected, mm.actual)
    if op == p.OP_MAX:
        np.testing.assert_array_equal(np.asarray(got).reshape(-1), ref.reshape(-1))
    else:
        assert oracle.normwise_rel_err(np.asarray(got), ref) <= NORMWISE
    return ref


@pytest.mark.parametrize("op", [p.OP_SUM, p.OP_MAX, p.OP_SOFTMAX])
def test_c3_8192x4096(gpu_runtime, op):
    x = oracle.normal(77, (8192, 4096))
    rc, res, out = gpu_runtime.reduction(x, op)
    assert rc == 0 and res.stage == p.STAGE_TRANSFER_OUT and res.detail_code == 0
    assert res.gpu_timestamp_valid == 1
    _check(x, op, out)


@pytest.mark.parametrize("rows,width", [(1, 1), (1, 3), (3, 77), (5, 128), (16, 256), (7, 1000), (128, 1024),
                                        (4, 1056), (9, 1057), (2, 4095), (3, 4097), (2, 5000), (1, 65536)])
@pytest.mark.parametrize("op", [p.OP_SUM, p.OP_MAX, p.OP_SOFTMAX])
def test_ragged_widths(gpu_runtime, rows, width, op):
    x = oracle.reduction_input(rows, width, bias=0.5)
    rc, res, out = gpu_runtime.reduction(x, op)
    assert rc == 0
    _check(x, op, out)


@pytest.mark.parametrize("rows,width", [(1024, 512), (128, 4096), (16, 4096), (1024, 64), (512, 96)])
@pytest.mark.parametrize("op", [p.OP_SUM, p.OP_MAX, p.OP_SOFTMAX])
def test_reference_entry_reference_shapes(gpu_runtime, rows, width, op):
    # reactor_reduction_tests.cpp:574-645 shapes and generator, through the reference envelope entry
    x = oracle.reduction_input(rows, width, bias=-0.25)
    rc, res, out = gpu_runtime.reduction(x, op, lifted=False)
    assert rc == 0 and res.detail_code == 0
    _check(x, op, out)
    # the result carries the reference's plan for this request
    plan = p.PrometheusReductionPlan()
    req = p.PrometheusReductionRequest()
    req.struct_size = ctypes.sizeof(req)
    req.row_count, req.elements_per_row, req.operation = rows, width, op
    req.finalization = 1 if op == p.OP_SOFTMAX else 0
    req.input_element_count = rows * width
    req.output_element_count = rows * width if op == p.OP_SOFTMAX else rows
    assert gpu_runtime.lib.prometheus_reactor_reduction_plan(ctypes.byref(req), ctypes.byref(plan)) == 0
    assert plan.replay_id == res.plan.replay_id


@pytest.mark.parametrize("dist", ["constant", "positive-extreme", "negative-extreme", "heterogeneous"])
def test_softmax_distributions(gpu_runtime, dist):
    # reactor_reduction_tests.cpp:89-115 (fr_m0_input)
    rows, width = 64, 1056
    x = oracle.reduction_input(rows, width)
    col = np.arange(width)
    if dist == "constant":
        x[:] = 3.25
    elif dist == "positive-extreme":
        x[:] = 10000.0 + ((col % 17) - 8)
    elif dist == "negative-extreme":
        x[:] = -10000.0 + ((col % 17) - 8)
    else:
        for r in range(rows):
            mode = r % 4
            x[r] = [2.0 * np.ones(width), ((col % 101) - 50) / 8.0, 10000.0 + ((col % 17) - 8),
                    -10000.0 + ((col % 17) - 8)][mode]
    rc, res, out = gpu_runtime.reduction(x.astype(np.float32), p.OP_SOFTMAX, flags=p.FLAG_FORCE_FUSED, lifted=False)
    assert rc == 0
    _check(x.astype(np.float32), p.OP_SOFTMAX, out)


def test_softmax_kats(gpu_runtime):
    # FusedReductionSemantics.sdslvtest:6-95
    rc, _, s = gpu_runtime.reduction(np.array([[1.5, -2.0, 4.25]], np.float32), p.OP_SUM)
    assert abs(s[0] - 3.75) <= 1e-5
    rc, _, m = gpu_runtime.reduction(np.array([[-9.0, -4.0, -12.0, -4.5, -20.0]], np.float32), p.OP_MAX)
    assert m[0] == -4.0
    rc, _, y = gpu_runtime.reduction(np.array([[10000.0, 10001.0, 9999.0, 10000.0]], np.float32), p.OP_SOFTMAX)
    assert abs(y.sum() - 1) <= 1e-4 and y[0, 1] > y[0, 0] > y[0, 2]
    rc, _, y = gpu_runtime.reduction(np.array([[7.0] * 4], np.float32), p.OP_SOFTMAX)
    assert np.all(np.abs(y - 0.25) <= 1e-5)
    rc, _, y = gpu_runtime.reduction(np.array([[80.0, -80.0, -80.0, -80.0]], np.float32), p.OP_SOFTMAX)
    assert abs(y[0, 0] - 1) <= 1e-5


def test_softmax_captured_attention_row(gpu_runtime):
    w = octagon.load("attention_token0_head0.octagon")
    x = w["Logits"].astype(np.float32)[None, :]
    rc, _, y = gpu_runtime.reduction(x, p.OP_SOFTMAX)
    assert rc == 0
    # the Oct witness is binary64; an fp32 result is within a few fp32 ulps of it
    assert np.all(np.abs(y[0] - w["Expected"]) <= 2e-8 + 4 * 2.0 ** -24 * np.abs(w["Expected"]))


def test_row_wise_softmax_in_place(gpu_runtime):
    x = oracle.reduction_input(100, 1000)
    ref = oracle.reduction_reference(x, 3)[1]
    buf = x.copy()
    req = p.PrometheusRowWiseSoftmaxRequest()
    req.struct_size = ctypes.sizeof(req)
    req.input = req.output = buf.ctypes.data
    req.row_count, req.elements_per_row = 100, 1000
    req.input_element_count = req.output_element_count = 100000
    res = p.PrometheusRowWiseSoftmaxResult()
    rc = gpu_runtime.lib.prometheus_reactor_runtime_row_wise_softmax(gpu_runtime.handle, ctypes.byref(req),
                                                                     ctypes.byref(res))
    assert rc == 0 and res.output_written == 1 and res.physical_dispatch_count == 1
    assert oracle.normwise_rel_err(buf, ref) <= NORMWISE


def test_reduction_device_entry_matches_host_entry(gpu_runtime):
    rt = gpu_runtime
    x = oracle.normal(5, (1000, 4096))
    for op in (p.OP_SUM, p.OP_MAX, p.OP_SOFTMAX):
        out_host = rt.reduction(x, op)[2]
        din = rt.alloc(x.nbytes)
        dout = rt.alloc(x.nbytes)
        try:
            rt.upload(din, x)
            rt.reduction_device(din, dout, 1000, 4096, op)
            rt.synchronize()
            got = rt.download(np.empty(out_host.shape, np.float32), dout)
        finally:
            rt.free(din)
            rt.free(dout)
        np.testing.assert_array_equal(got, out_host)


# ------------------------------------------------------------------ RMSNorm
def test_rmsnorm_c3_8192x4096(gpu_runtime):
    x = oracle.normal(88, (8192, 4096))
    w = (1.0 + oracle.normal(89, (4096,), 0.0, 0.02)).astype(np.float32)
    rc, res, y, inv = gpu_runtime.rmsnorm(x, w, 1e-6)
    assert rc == 0 and res.output_written == 1
    rc2, y_ref, inv_ref = oracle.rmsnorm_reference(x, w, 1e-6)
    assert rc2 == 0
    assert oracle.normwise_rel_err(y, y_ref) <= NORMWISE
    assert oracle.normwise_rel_err(inv, inv_ref) <= NORMWISE


@pytest.mark.parametrize("tokens,width,stride", [(1, 1, 1), (3, 7, 7), (15, 1536, 1536), (4, 256, 260),
                                                 (9, 4097, 4097), (33, 100, 128), (2, 8192, 8192)])
def test_rmsnorm_shapes(gpu_runtime, tokens, width, stride):
    z = oracle.normal(tokens * 7 + width, (tokens, stride))
    w = oracle.normal(width, (width,), 1.0, 0.02)
    rc, res, y, inv = gpu_runtime.rmsnorm(z, w, 1e-6, stride=stride)
    assert rc == 0
    rc2, y_ref, inv_ref = oracle.rmsnorm_reference(z, w, 1e-6, width=width)
    assert oracle.normwise_rel_err(y, y_ref) <= NORMWISE
    np.testing.assert_allclose(inv, inv_ref, rtol=1e-6)


def test_rmsnorm_captured_qnorm_row(gpu_runtime):
    w = octagon.load("qnorm_row0_head0.octagon")
    rc, res, y, inv = gpu_runtime.rmsnorm(w["Input"].astype(np.float32)[None, :], w["Scale"].astype(np.float32),
                                          1e-5)
    assert rc == 0
    assert np.max(np.abs(y[0] - w["Expected"])) <= 2e-6


def test_gemma_input_rmsnorm_entry(gpu_runtime):
    # reactor_api.c:250-359: Gemma-4-E2B layer-0 input RMSNorm (15 tokens x 1536)
    tokens, width = 15, 1536
    z = oracle.normal(3, (tokens, width))
    wt = oracle.normal(4, (width,), 1.0, 0.1)
    y = np.zeros((tokens, width), np.float32)
    inv = np.zeros(tokens, np.float32)
    req = p.PrometheusGemma4E2BM1InputRmsNormRequest()
    req.struct_size = ctypes.sizeof(req)
    req.input, req.weight, req.output, req.inv_rms_output = (z.ctypes.data, wt.ctypes.data, y.ctypes.data,
                                                             inv.ctypes.data)
    req.input_element_count = req.output_element_count = tokens * width
    req.weight_element_count, req.inv_rms_output_element_count = width, tokens
    req.tokens, req.model_width, req.input_row_stride, req.epsilon = tokens, width, width, 1e-6
    req.input_generation = req.weight_generation = req.exact_source_hash = 7
    res = p.PrometheusGemma4E2BM1InputRmsNormResult()
    rc = gpu_runtime.lib.prometheus_reactor_runtime_gemma4e2b_m1_input_rmsnorm(gpu_runtime.handle, ctypes.byref(req),
                                                                               ctypes.byref(res))
    # success leaves stage 0 (reactor_concept_rmsnorm.cpp:110-146 never sets it)
    assert rc == 0 and res.output_written == 1 and res.stage == 0 and res.detail_code == 0
    rc2, y_ref, inv_ref = oracle.rmsnorm_reference(z, wt, 1e-6)
    assert oracle.normwise_rel_err(y, y_ref) <= NORMWISE


@pytest.mark.parametrize("op", [p.OP_SUM, p.OP_MAX, p.OP_SOFTMAX])
def test_reduction_benchmark_entry(op):
    """reactor_vulkan_fused_reduction.c:1122-1201 on the reference envelope
    (1024 rows of 4096): every measured iteration completes, the device's
    binary64 check accepts the output, the timings are ordered, and the
    output also passes the CPU oracle's comparator; the diagnostics count
    every execution."""
    rt = p.NativeRuntime()
    try:
        assert rt.available
        rng = np.random.default_rng(op)
        x = rng.standard_normal((1024, 4096)).astype(np.float32)
        rc, res, out = rt.reduction_benchmark(x, op, warmup=3, measured=9)
        assert rc == p.PROM_OK and res.detail_code == 0, (res.detail_code, res.first_mismatch_row)
        assert res.completed_iterations == 9 and res.correctness_passed == 1 and res.validation_passed == 1
        assert 0 < res.gpu_min_ns <= res.gpu_median_ns <= res.gpu_max_ns
        assert res.gpu_min_ns <= res.end_to_end_min_ns <= res.end_to_end_median_ns <= res.end_to_end_max_ns
        assert res.first_mismatch_row == 0xFFFFFFFF and res.stage_count >= 1 and res.replay_id != 0
        rc2, _, _ = rt.reduction(x, op, lifted=False)
        _check(x, op, out)
        rc, d = rt.reduction_diagnostics()
        assert rc == p.PROM_OK and d.initialized == 1 and d.production_enabled == 1
        assert d.total_requests == 13 and d.successful_requests == 13 and d.logical_failure_count == 0
        assert d.last_replay_id == res.replay_id and d.last_stage_count == res.stage_count and d.last_detail_code == 0
        assert d.last_gpu_duration_ns > 0 and d.configured_ring_depth == 1
        print(f"reduction benchmark op={op}: gpu median {res.gpu_median_ns / 1e3:.1f} us, "
              f"end-to-end median {res.end_to_end_median_ns / 1e3:.1f} us", flush=True)
    finally:
        rt.close()
