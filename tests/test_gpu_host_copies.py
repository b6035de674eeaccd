"""Host-pointer entry points move caller-owned pageable buffers through a ring
of pinned chunks (8 MiB, four slots) once a copy reaches 4 MiB.  The results
must be exactly those of the device-pointer entries on the same operands:
chunk boundaries, ragged last chunks, more chunks than slots, and slots reused
between an upload and a later download."""
import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu


def _device_sgemm(rt, a, b):
    m, k = a.shape
    n = b.shape[1]
    da, db, dc = rt.upload_new(a), rt.upload_new(b), rt.alloc(m * n * 4)
    try:
        assert rt.sgemm_device(da, db, dc, m, n, k) > 0
        rt.synchronize()
        return rt.download(np.empty((m, n), np.float32), dc)
    finally:
        for d in (da, db, dc):
            rt.free(d)


# bytes of A / B / C: (6.3 MB, 12.5 MB, 8.5 MB): one short chunk, two chunks
# with a ragged tail; (8 MiB exactly, 36 MiB, 36 MiB): a whole chunk, and five
# chunks through four slots both ways
@pytest.mark.parametrize("m,n,k", [(1037, 2049, 1531), (1024, 4608, 2048)])
def test_sgemm_host_equals_device(gpu_runtime, m, n, k):
    a = oracle.uniform(200 + m, (m, k))
    b = oracle.uniform(300 + n, (k, n))
    out, status = gpu_runtime.sgemm(m, n, k, a, b)
    assert str(status) == "ok"
    host = out.reshape(m, n)
    np.testing.assert_array_equal(host, _device_sgemm(gpu_runtime, a, b))
    for r in (0, m // 2, m - 1):
        ref = oracle.matmul_f64(a, b, rows=(r, r + 1))[r]
        assert oracle.normwise_rel_err(host[r], ref) <= 1e-5


def test_softmax_host_many_chunks(gpu_runtime):
    # 3001 x 4099 fp32 = 49.2 MB in and out: six chunks, the last ragged
    x = oracle.normal(91, (3001, 4099))
    rc, res, out = gpu_runtime.reduction(x, p.OP_SOFTMAX)
    assert rc == 0 and res.detail_code == 0
    for r in (0, 1, 1500, 2999, 3000):
        row = x[r].astype(np.float64)
        e = np.exp(row - row.max())
        ref = e / e.sum()
        assert oracle.normwise_rel_err(out[r], ref) <= 1e-5
    rc, res, sums = gpu_runtime.reduction(x, p.OP_SUM)
    assert rc == 0
    np.testing.assert_allclose(sums, x.astype(np.float64).sum(axis=1), rtol=1e-5, atol=1e-3)


def test_alternating_host_calls(gpu_runtime):
    """Uploads and downloads of different sizes back to back reuse the slots."""
    rt = gpu_runtime
    for (m, n, k), seed in (((1536, 1536, 1536), 1), ((257, 8193, 1024), 2), ((1536, 1536, 1536), 3)):
        a = oracle.uniform(seed, (m, k))
        b = oracle.uniform(seed + 10, (k, n))
        out, status = rt.sgemm(m, n, k, a, b)
        assert str(status) == "ok"
        np.testing.assert_array_equal(out.reshape(m, n), _device_sgemm(rt, a, b))
        x = oracle.normal(seed + 20, (1000 + seed, 3000))
        rc, _, y = rt.reduction(x, p.OP_SOFTMAX)
        assert rc == 0
        row = x[-1].astype(np.float64)
        e = np.exp(row - row.max())
        assert oracle.normwise_rel_err(y[-1], e / e.sum()) <= 1e-5


def test_async_and_batch_copies_equal_device(gpu_runtime):
    """The async entry's copies into and out of its pinned staging and the
    batch's uploads (over 4 MiB: the pinned ring) leave the results exactly
    those of the device entry."""
    rt = gpu_runtime
    m, n, k = 1037, 2049, 1531
    a = oracle.uniform(501, (m, k))
    b = oracle.uniform(502, (k, n))
    want = _device_sgemm(rt, a, b)
    rc, task, _ = rt.submit_async(m, n, k, a, b)
    assert rc == p.PROM_OK
    st = rt.wait_async(task)
    assert st.lifecycle_state == p.ASYNC_READY
    out = np.empty((m, n), np.float32)
    rc, _ = rt.consume_async(task, out)
    assert rc == p.PROM_OK
    np.testing.assert_array_equal(out, want)
    a2 = oracle.uniform(503, (m, k))
    rc, _, outs = rt.sgemm_batch([(a, b), (a2, b)])
    assert rc == p.PROM_OK
    np.testing.assert_array_equal(outs[0], want)
    np.testing.assert_array_equal(outs[1], _device_sgemm(rt, a2, b))
