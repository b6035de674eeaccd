"""GPU parity of the MFMA SGEMM / GEMV / bf16 GEMM against the CPU oracle.

Bar: normwise relative error <= 1e-5 for fp32
against Oct's binary64 `@` on the same fp32 operands; <= 2e-2 for bf16
(against binary64 on the bf16 operands).  The reference's own tolerance
(abs 1e-4 and rel 1e-4, runtime.go:12-15) is checked on its corpora.
"""
import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu

FP32_NORMWISE = 1e-5
BF16_NORMWISE = 2e-2


def _sgemm(rt, a, b):
    m, k = a.shape
    n = b.shape[1]
    out, status = rt.sgemm(m, n, k, a, b)
    assert str(status) == "ok"
    return out.reshape(m, n)


def test_kat_2x2(gpu_runtime):
    out = _sgemm(gpu_runtime, np.array([[1, 2], [3, 4]], np.float32), np.array([[5, 6], [7, 8]], np.float32))
    np.testing.assert_array_equal(out, [[19, 22], [43, 50]])


def test_strict_path_a_at_a(gpu_runtime):
    # Language/Prometheus/gpu/matrix.octest:3-9
    out, env = p.run_compiled_matmul_mm_strict([[1.0, 2.0], [3.0, 4.0]], [[1.0, 2.0], [3.0, 4.0]])
    assert out[0][0] == 7.0 and env == "hardware_gpu_hip"


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (4, 4, 4), (16, 16, 16), (32, 32, 32), (3, 5, 7), (3, 7, 5),
                                   (1, 9, 4), (11, 1, 3), (2, 13, 3)])
def test_reference_corpora(gpu_runtime, m, n, k):
    # runtime.go:83-89 and reactor_stub_tests.cpp:205-253
    a = oracle.deterministic_matrix(m, k)
    b = oracle.deterministic_matrix(k, n)
    out, st, rc = gpu_runtime.sgemm_with_status(m, n, k, a, b)
    assert rc == p.PROM_OK and st.stage == p.STAGE_TRANSFER_OUT and st.detail > 0
    res = oracle.compare_against_oracle(oracle.cpu_sgemm_f32(a, b), out)
    assert res.pass_ == 1, (res.first_failing_index, res.first_expected, res.first_actual)
    assert oracle.normwise_rel_err(out, oracle.matmul_f64(a, b)) <= FP32_NORMWISE


def test_concept_corpus_binary64(gpu_runtime):
    # reactor_concept_sgemm_tests.cpp:17-29: 37x29x13 against binary64 within 1e-4
    m, n, k = 37, 29, 13
    a = oracle.concept_sgemm_matrix(m * k, 3).reshape(m, k)
    b = oracle.concept_sgemm_matrix(k * n, 5).reshape(k, n)
    out = _sgemm(gpu_runtime, a, b)
    assert np.max(np.abs(out - oracle.matmul_f64(a, b))) <= 1e-4


@pytest.mark.parametrize("m,n,k", [(2, 3, 1), (5, 3, 2), (7, 9, 3), (129, 127, 17), (128, 128, 16), (257, 130, 33),
                                   (64, 256, 4), (300, 200, 100), (1, 513, 257), (513, 1, 255), (130, 5, 1025)])
def test_exact_tail_shapes(gpu_runtime, m, n, k):
    a = oracle.uniform(100 + m, (m, k))
    b = oracle.uniform(200 + n, (k, n))
    out = _sgemm(gpu_runtime, a, b)
    assert oracle.normwise_rel_err(out, oracle.matmul_f64(a, b)) <= FP32_NORMWISE


# Every kernel variant, run explicitly through the variant entry (so the
# coverage does not depend on which variants the plan model picks): tiles
# 0-2 register-staged, 3-4 direct-to-LDS, 5-6 the 64x64 tile with the K tile
# split inside the workgroup; with and without split-K; ragged m and n.
VARIANT_SHAPES = [(200, 260, 512), (65, 128, 1024), (1, 4, 64)]


@pytest.mark.parametrize("tile", range(7))
@pytest.mark.parametrize("slices", [1, 4])
@pytest.mark.parametrize("shape", VARIANT_SHAPES)
def test_every_variant(gpu_runtime, tile, slices, shape):
    m, n, k = shape
    # K slices are whole granules (16; 32 and 64 for the 64x64 tiles): a
    # request that cannot give exactly `slices` slices is refused.
    g = {5: 32, 6: 64}.get(tile, 16)
    k_len = -(-(-(-k // slices)) // g) * g
    possible = slices == 1 or -(-k // k_len) == slices
    a = oracle.uniform(300 + m + tile, (m, k))
    b = oracle.uniform(400 + n + slices, (k, n))
    da, db, dc = gpu_runtime.upload_new(a), gpu_runtime.upload_new(b), gpu_runtime.alloc(m * n * 4)
    try:
        rc, st = gpu_runtime.sgemm_device_variant(da, db, dc, m, n, k, tile, slices)
        if not possible:
            assert rc == p.PROM_ERROR and st.detail == p.DETAIL_INVALID_ARGUMENT
            return
        assert rc == p.PROM_OK, (st.stage, st.detail)
        gpu_runtime.synchronize()
        out = gpu_runtime.download(np.empty((m, n), np.float32), dc)
    finally:
        for d in (da, db, dc):
            gpu_runtime.free(d)
    assert oracle.normwise_rel_err(out, oracle.matmul_f64(a, b)) <= FP32_NORMWISE


@pytest.mark.parametrize("tile", [5, 6])
@pytest.mark.parametrize("m,n,k", [(100, 260, 1000), (129, 64, 36), (64, 64, 4), (70, 68, 132)])
def test_k_tail_of_the_64x64_kernels(gpu_runtime, tile, m, n, k):
    """K not a multiple of the K tile: the last tile's A columns past K are
    filled from the next row by the transfers and must be cleared.  A NaN
    at the start of row 7 of A would poison row 6 if they were not."""
    a = oracle.uniform(700 + k, (m, k))
    b = oracle.uniform(800 + n, (k, n))
    a[7, 0] = np.nan
    da, db, dc = gpu_runtime.upload_new(a), gpu_runtime.upload_new(b), gpu_runtime.alloc(m * n * 4)
    try:
        rc, st = gpu_runtime.sgemm_device_variant(da, db, dc, m, n, k, tile, 1)
        assert rc == p.PROM_OK, (st.stage, st.detail)
        gpu_runtime.synchronize()
        out = gpu_runtime.download(np.empty((m, n), np.float32), dc)
    finally:
        for d in (da, db, dc):
            gpu_runtime.free(d)
    assert np.all(np.isnan(out[7]))
    rows = [r for r in range(m) if r != 7]
    ref = oracle.matmul_f64(np.delete(a, 7, axis=0), b)
    assert np.all(np.isfinite(out[rows]))
    assert oracle.normwise_rel_err(out[rows], ref) <= FP32_NORMWISE


@pytest.mark.parametrize("m,n,k", [(4097, 3001, 513), (130, 127, 65), (513, 1027, 131)])
def test_repacked_operands(gpu_runtime, m, n, k):
    """Unaligned operands copied to zero-padded buffers, then the direct kernels."""
    rc, plan = p.sgemm_plan(m, n, k)
    assert rc == p.PROM_OK and plan.repacked == 1, "the repack must be planned for this shape"
    a = oracle.uniform(900 + m, (m, k))
    b = oracle.uniform(901 + n, (k, n))
    out = _sgemm(gpu_runtime, a, b)
    rows = sorted({0, 1, m // 2, m - 2, m - 1})
    for r in rows:
        assert oracle.normwise_rel_err(out[r], oracle.matmul_f64(a, b, rows=(r, r + 1))[r]) <= FP32_NORMWISE, r


def test_staged_variants_cover_unaligned_shapes_and_direct_ones_refuse(gpu_runtime):
    m, n, k = 130, 127, 65  # n and k not multiples of 4: register-staged tiles only
    a = oracle.uniform(501, (m, k))
    b = oracle.uniform(502, (k, n))
    da, db, dc = gpu_runtime.upload_new(a), gpu_runtime.upload_new(b), gpu_runtime.alloc(m * n * 4)
    try:
        for tile in range(7):
            rc, st = gpu_runtime.sgemm_device_variant(da, db, dc, m, n, k, tile, 1)
            if tile >= 3:
                assert rc == p.PROM_ERROR and st.stage == p.STAGE_INIT and st.detail == p.DETAIL_INVALID_ARGUMENT, tile
                continue
            assert rc == p.PROM_OK, (tile, st.detail)
            gpu_runtime.synchronize()
            out = gpu_runtime.download(np.empty((m, n), np.float32), dc)
            assert oracle.normwise_rel_err(out, oracle.matmul_f64(a, b)) <= FP32_NORMWISE, tile
        rc, st = gpu_runtime.sgemm_device_variant(da, db, dc, m, n, k, 7, 1)
        assert rc == p.PROM_ERROR and st.detail == p.DETAIL_INVALID_ARGUMENT
    finally:
        for d in (da, db, dc):
            gpu_runtime.free(d)


# M past a multiple of 128 where the plan model runs the last rows as a second,
# K-split product after the full 128-row tiles: the rows either side of the
# seam and the last row.
@pytest.mark.parametrize("m,n,k", [(1056, 4096, 4096), (2049, 8192, 2048), (1056, 20480, 3840)])
def test_tail_row_split(gpu_runtime, m, n, k):
    rc, plan = p.sgemm_plan(m, n, k)
    assert rc == p.PROM_OK and plan.products == 2 and plan.head_rows == m - m % 128, "the split must be planned"
    a = oracle.uniform(500 + m, (m, k))
    b = oracle.uniform(600 + n, (k, n))
    out = _sgemm(gpu_runtime, a, b)
    head = m - m % 128
    for r in (0, head - 1, head, m - 1):
        assert oracle.normwise_rel_err(out[r], oracle.matmul_f64(a, b, rows=(r, r + 1))[r]) <= FP32_NORMWISE, r


def test_c1_1024_full(gpu_runtime):
    # M=N=K=1024, U[-1,1] seeded
    a = oracle.uniform(1, (1024, 1024))
    b = oracle.uniform(2, (1024, 1024))
    out = _sgemm(gpu_runtime, a, b)
    err = oracle.normwise_rel_err(out, oracle.matmul_f64(a, b))
    print(f"C1 1024^3 normwise rel err {err:.3e}")
    assert err <= FP32_NORMWISE


def test_c2_1000_full(gpu_runtime):
    a = oracle.uniform(3, (1000, 1000))
    b = oracle.uniform(4, (1000, 1000))
    out = _sgemm(gpu_runtime, a, b)
    assert oracle.normwise_rel_err(out, oracle.matmul_f64(a, b)) <= FP32_NORMWISE


def _rows_subset(m, count=64):
    rows = sorted(set(np.linspace(0, m - 1, count).astype(int).tolist()) | {m - 1, m - 2})
    return rows


def test_c2_ragged_4097_3001_513(gpu_runtime):
    m, n, k = 4097, 3001, 513
    a = oracle.uniform(5, (m, k))
    b = oracle.uniform(6, (k, n))
    out = _sgemm(gpu_runtime, a, b)
    # the last 129 rows (one full tile plus the ragged one) and a spread of others, exactly
    tail = oracle.matmul_f64(a, b, rows=(m - 129, m))
    assert oracle.normwise_rel_err(out[m - 129:], tail[m - 129:]) <= FP32_NORMWISE
    for r in _rows_subset(m, 32):
        ref = oracle.matmul_f64(a, b, rows=(r, r + 1))[r]
        assert oracle.normwise_rel_err(out[r], ref) <= FP32_NORMWISE
    # full-size property: C x = A (B x) for a random x (Freivalds)
    x = np.random.default_rng(0).standard_normal(n)
    lhs = out.astype(np.float64) @ x
    rhs = a.astype(np.float64) @ (b.astype(np.float64) @ x)
    assert np.linalg.norm(lhs - rhs) / np.linalg.norm(rhs) <= FP32_NORMWISE


def test_c2_gemv_8192x1x4096(gpu_runtime):
    m, n, k = 8192, 1, 4096
    a = oracle.uniform(7, (m, k))
    b = oracle.uniform(8, (k, n))
    out, st, rc = gpu_runtime.sgemm_with_status(m, n, k, a, b)
    assert rc == 0 and st.detail == p.DETAIL_PATH_HIP_GEMV_F32
    assert oracle.normwise_rel_err(out, oracle.matmul_f64(a, b)) <= FP32_NORMWISE


@pytest.mark.parametrize("m,k", [(1, 1), (3, 5), (7, 4097), (1000, 1000), (65, 3)])
def test_gemv_ragged(gpu_runtime, m, k):
    a = oracle.uniform(9 + m, (m, k))
    b = oracle.uniform(10 + k, (k, 1))
    out = _sgemm(gpu_runtime, a, b)
    assert oracle.normwise_rel_err(out, oracle.matmul_f64(a, b)) <= FP32_NORMWISE


def test_c2_4096_cubed_device_resident(gpu_runtime):
    """Full-size 4096^3 via the device-resident entry: subset rows exactly + Freivalds."""
    rt = gpu_runtime
    n = 4096
    a = oracle.uniform(11, (n, n))
    b = oracle.uniform(12, (n, n))
    da, db, dc = rt.alloc(a.nbytes), rt.alloc(b.nbytes), rt.alloc(a.nbytes)
    try:
        rt.upload(da, a)
        rt.upload(db, b)
        assert rt.sgemm_device(da, db, dc, n, n, n) == p.DETAIL_PATH_HIP_MFMA_F32
        rt.synchronize()
        out = rt.download(np.empty((n, n), np.float32), dc)
        # the host-pointer path gives bit-identical results (same kernel, deterministic)
        out2 = _sgemm(rt, a, b)
        np.testing.assert_array_equal(out, out2)
    finally:
        for d in (da, db, dc):
            rt.free(d)
    rows = _rows_subset(n, 24)
    for r in rows:
        ref = oracle.matmul_f64(a, b, rows=(r, r + 1))[r]
        assert oracle.normwise_rel_err(out[r], ref) <= FP32_NORMWISE, r
    x = np.random.default_rng(1).standard_normal(n)
    rhs = a.astype(np.float64) @ (b.astype(np.float64) @ x)
    assert np.linalg.norm(out.astype(np.float64) @ x - rhs) / np.linalg.norm(rhs) <= FP32_NORMWISE


def test_sgemm_deterministic(gpu_runtime):
    a = oracle.uniform(13, (300, 257))
    b = oracle.uniform(14, (257, 190))
    np.testing.assert_array_equal(_sgemm(gpu_runtime, a, b), _sgemm(gpu_runtime, a, b))


def test_injected_faults_report_reference_stages():
    # reactor_stub_tests.cpp:842-913: injected upload/dispatch/download failures
    for flag, stage, detail in ((p.TESTCFG_FAIL_UPLOAD, p.STAGE_TRANSFER_IN, p.DETAIL_INJECTED_UPLOAD_FAILURE),
                                (p.TESTCFG_FAIL_DISPATCH, p.STAGE_SUBMIT, p.DETAIL_INJECTED_DISPATCH_FAILURE),
                                (p.TESTCFG_FAIL_DOWNLOAD, p.STAGE_TRANSFER_OUT, p.DETAIL_INJECTED_DOWNLOAD_FAILURE)):
        with p.NativeRuntime(test_flags=flag) as rt:
            assert rt.available
            out, st, rc = rt.sgemm_with_status(2, 2, 2, np.ones(4), np.ones(4))
            assert rc == p.PROM_ERROR and (st.stage, st.detail) == (stage, detail) and out is None


# ------------------------------------------------------------------ bf16
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (5, 7, 3), (128, 128, 64), (129, 130, 65), (257, 513, 200),
                                   (1000, 1000, 1000), (64, 8, 8)])
def test_bf16_shapes(gpu_runtime, m, n, k):
    a = oracle.to_bf16(oracle.uniform(20 + m, (m, k)))
    b = oracle.to_bf16(oracle.uniform(30 + n, (k, n)))
    out = gpu_runtime.gemm_bf16(m, n, k, a, b).reshape(m, n)
    err = oracle.normwise_rel_err(out, oracle.matmul_f64(a, b))
    # products of bf16 values are exact in fp32; only fp32 accumulation rounds
    assert err <= 1e-5 and err <= BF16_NORMWISE


def test_bf16_4096_cubed(gpu_runtime):
    rt = gpu_runtime
    n = 4096
    a = oracle.to_bf16(oracle.uniform(41, (n, n)))
    b = oracle.to_bf16(oracle.uniform(42, (n, n)))
    da, db, dc = rt.alloc(a.nbytes), rt.alloc(b.nbytes), rt.alloc(n * n * 4)
    try:
        rt.upload(da, a)
        rt.upload(db, b)
        assert rt.gemm_bf16_device(da, db, dc, n, n, n) == p.DETAIL_PATH_HIP_MFMA_BF16
        rt.synchronize()
        out = rt.download(np.empty((n, n), np.float32), dc)
    finally:
        for d in (da, db, dc):
            rt.free(d)
    for r in _rows_subset(n, 16):
        ref = oracle.matmul_f64(a, b, rows=(r, r + 1))[r]
        assert oracle.normwise_rel_err(out[r], ref) <= BF16_NORMWISE
        assert oracle.normwise_rel_err(out[r], ref) <= 1e-5


@pytest.mark.parametrize("m,n,k", [(4224, 2056, 72), (600, 8200, 136), (1024, 4096, 8),
                                   (1100, 16400, 96), (2560, 3584, 8224)])
def test_bf16_large_tile_kernel_ragged(gpu_runtime, m, n, k):
    """Shapes with >= 128 256x256 tiles take the large-tile kernels; ragged m/n/k tails.
    (1100, 16400, 96) and (2560, 3584, 8224) take the four-stage kernel (more
    than 256 tiles, or K >= 8192; K a multiple of 32 but not of 64)."""
    a = oracle.to_bf16(oracle.uniform(50 + m, (m, k)))
    b = oracle.to_bf16(oracle.uniform(60 + n, (k, n)))
    out = gpu_runtime.gemm_bf16(m, n, k, a, b).reshape(m, n)
    ref = oracle.from_bf16(a).astype(np.float64) @ oracle.from_bf16(b).astype(np.float64)
    assert oracle.normwise_rel_err(out, ref) <= 1e-5
    rows = [0, m // 2, m - 1]
    for r in rows:
        ref_r = oracle.matmul_f64(a, b, rows=(r, r + 1))[r]
        # fp32 accumulation over k terms: absolute slack relative to the row's scale
        np.testing.assert_allclose(out[r], ref_r, rtol=1e-4, atol=2e-6 * np.abs(ref_r).max())


@pytest.mark.parametrize("m,n,k", [(1, 1, 3_000_000_000), (1, 2**31, 1), (70000, 70000, 1)])
def test_device_entry_rejects_oversized_shapes(gpu_runtime, m, n, k):
    """Admission runs before any launch: no operand memory is touched."""
    import ctypes

    stage, detail = ctypes.c_uint32(0), ctypes.c_int(0)
    dummy = gpu_runtime.alloc(256)
    try:
        rc = gpu_runtime.lib.prometheus_reactor_runtime_sgemm_device(gpu_runtime.handle, dummy, dummy, dummy, m, n, k,
                                                                     ctypes.byref(stage), ctypes.byref(detail))
    finally:
        gpu_runtime.free(dummy)
    assert rc == p.PROM_ERROR and stage.value == p.STAGE_TRANSFER_IN and detail.value == p.DETAIL_SIZE_OVERFLOW


def test_nonstrict_path_runs_on_the_device_and_passes_its_gate():
    """runtime.go:121-206 on the device: status ok, reactor backend, and the output
    within the gate of Oct's fp32 CPU reference (checked here by the oracle)."""
    from oct_amd import runtime as r

    runs = r.run_starter_corpus(r.BACKEND_PROMETHEUS)
    for run in runs:
        assert str(run.status) == "ok" and run.used_backend == "prometheus", run
        assert run.correctness.passed and run.detail_name in ("hip_mfma_f32", "hip_gemv_f32")
    m, n, k = 257, 129, 300
    a = oracle.uniform(71, (m, k))
    b = oracle.uniform(72, (k, n))
    out, res = r.run_sgemm_with_output(r.SGEMMRequest(r.BACKEND_PROMETHEUS, r.Shape(m, n, k), a, b))
    assert str(res.status) == "ok" and res.used_backend == "prometheus" and res.vulkan_env == "hardware_gpu_hip"
    gate = oracle.compare_against_oracle(oracle.cpu_sgemm_f32(a, b), out)
    assert gate.pass_ == 1 and res.correctness.passed
    assert oracle.normwise_rel_err(out.reshape(m, n), oracle.matmul_f64(a, b)) <= FP32_NORMWISE
    rows, res2 = r.run_compiled_matmul_mm([[1.0, 2.0], [3.0, 4.0]], [[5.0, 6.0], [7.0, 8.0]])
    assert rows == [[19.0, 22.0], [43.0, 50.0]] and str(res2.status) == "ok"
