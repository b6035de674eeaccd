"""GPU tests of the asynchronous SGEMM lifecycle and the ordered-commit batch.

They restate the reference's Marionette facts for these entries
(reactor_stub_tests.cpp:1450-1636 for async; reactor_m29_fixed_double_tests.cpp:
126-348 for the batch) on the HIP runtime, and check every result against the
CPU oracle at the fp32 bar (normwise relative error <= 1e-5 against binary64).
"""
import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu

FP32_NORMWISE = 1e-5


def _check(out, a, b):
    assert oracle.normwise_rel_err(out, oracle.matmul_f64(a, b)) <= FP32_NORMWISE


@pytest.fixture
def rt():
    with p.NativeRuntime() as r:
        r.require_hardware_gpu()
        yield r


def test_deferred_completion_is_observable(rt):
    # reactor_stub_tests.cpp:1450-1494
    m = n = k = 32
    a, b = oracle.deterministic_matrix(m, k), oracle.deterministic_matrix(k, n)
    rc, task, cs = rt.submit_async(m, n, k, a, b)
    assert rc == p.PROM_OK and task > 0 and cs.stage == p.STAGE_SUBMIT and cs.detail == 0
    st = rt.wait_async(task)
    assert st.lifecycle_state == p.ASYNC_READY and st.ready == 1 and st.failed == 0
    assert st.stage == p.STAGE_TRANSFER_OUT and st.outstanding_tasks == 1
    out = np.zeros(m * n, np.float32)
    rc, cs = rt.consume_async(task, out)
    assert rc == p.PROM_OK and cs.stage == p.STAGE_TRANSFER_OUT and cs.detail == p.DETAIL_PATH_HIP_MFMA_F32
    ref = oracle.cpu_sgemm_f32(a, b)
    assert np.max(np.abs(out.reshape(m, n) - ref)) <= 1e-4
    _check(out.reshape(m, n), a, b)
    rc, st = rt.query_async(task)
    assert rc == p.PROM_OK and st.lifecycle_state == p.ASYNC_CONSUMED and st.consumed == 1
    assert st.outstanding_tasks == 0


def test_use_before_complete_and_double_consume_are_rejected(rt):
    # reactor_stub_tests.cpp:1496-1537.  A 2048^3 task (48 MiB of operands to move
    # and 17 GFLOP) cannot be complete when consume is called straight after submit.
    n = 2048
    a, b = oracle.uniform(71, (n, n)), oracle.uniform(72, (n, n))
    rc, task, _ = rt.submit_async(n, n, n, a, b)
    assert rc == p.PROM_OK
    out = np.zeros((n, n), np.float32)
    rc, cs = rt.consume_async(task, out)
    assert (rc, cs.stage, cs.detail) == (p.PROM_ERROR, p.STAGE_SUBMIT, p.DETAIL_ASYNC_NOT_READY)
    # a running task cannot be abandoned (reactor_sgemm.cpp:6485-6490)
    assert rt.abandon_async(task) == p.PROM_ERROR
    # the caller's inputs were captured at submit: clobbering them changes nothing
    a_copy = a.copy()
    a[:] = 0
    assert rt.wait_async(task).lifecycle_state == p.ASYNC_READY
    # too small an output buffer is refused without consuming the task
    rc, cs = rt.consume_async(task, out, c_len=n * n - 1)
    assert (rc, cs.stage, cs.detail) == (p.PROM_ERROR, p.STAGE_TRANSFER_OUT, p.PROM_ERROR)
    rc, cs = rt.consume_async(task, out)
    assert rc == p.PROM_OK
    rc, cs = rt.consume_async(task, out)
    assert (rc, cs.stage, cs.detail) == (p.PROM_ERROR, p.STAGE_TRANSFER_OUT, p.DETAIL_ASYNC_ALREADY_CONSUMED)
    for r in (0, 1023, n - 1):
        ref = oracle.matmul_f64(a_copy, b, rows=(r, r + 1))[r]
        assert oracle.normwise_rel_err(out[r], ref) <= FP32_NORMWISE


def test_in_flight_ownership_queue_full_and_abandonment(rt):
    # reactor_stub_tests.cpp:1539-1585 plus the two-slot admission limit
    # (reactor_sgemm.cpp:6322-6324) and the sync rejection (reactor_sgemm.cpp:4204-4211).
    m, n, k = 300, 200, 100
    a1, b1 = oracle.uniform(81, (m, k)), oracle.uniform(82, (k, n))
    a2, b2 = oracle.uniform(83, (m, k)), oracle.uniform(84, (k, n))
    rc1, t1, _ = rt.submit_async(m, n, k, a1, b1)
    rc2, t2, _ = rt.submit_async(m, n, k, a2, b2)
    assert rc1 == rc2 == p.PROM_OK and t1 != t2
    rc3, t3, cs = rt.submit_async(m, n, k, a1, b1)
    assert (rc3, cs.stage, cs.detail) == (p.PROM_ERROR, p.STAGE_SUBMIT, p.DETAIL_ASYNC_QUEUE_FULL)
    out, st, rc = rt.sgemm_with_status(2, 2, 2, np.ones(4), np.ones(4))
    assert rc == p.PROM_ERROR and (st.stage, st.detail) == (p.STAGE_SUBMIT, p.DETAIL_ASYNC_UNCONSUMED)
    assert rt.wait_async(t1).lifecycle_state == p.ASYNC_READY
    assert rt.abandon_async(t1) == p.PROM_OK
    rc, st = rt.query_async(t1)
    assert rc == p.PROM_ERROR and st.detail_code == p.DETAIL_ASYNC_NO_TASK
    assert rt.wait_async(t2).lifecycle_state == p.ASYNC_READY
    out2 = np.zeros((m, n), np.float32)
    assert rt.consume_async(t2, out2)[0] == p.PROM_OK
    _check(out2, a2, b2)
    d = rt.async_diagnostics()
    assert d.queue_full_count == 1 and d.max_in_flight == 2 and d.stale_id_rejection_count == 1
    # nothing outstanding: the synchronous path works again
    out, st, rc = rt.sgemm_with_status(2, 2, 2, np.ones(4), np.ones(4))
    assert rc == p.PROM_OK and np.all(out == 2.0)


def test_task_ids_carry_generations(rt):
    # reactor_sgemm.cpp:6028-6083: records are reused round-robin with a new generation
    m, n, k = 17, 9, 5
    a, b = oracle.uniform(85, (m, k)), oracle.uniform(86, (k, n))
    seen = []
    out = np.zeros(m * n, np.float32)
    for _ in range(6):
        rc, t, _ = rt.submit_async(m, n, k, a, b)
        assert rc == p.PROM_OK
        assert rt.wait_async(t).lifecycle_state == p.ASYNC_READY
        assert rt.consume_async(t, out)[0] == p.PROM_OK
        _check(out.reshape(m, n), a, b)
        seen.append(t)
    assert [t & 0xF for t in seen] == [1, 2, 3, 4, 1, 2]
    assert [t >> 4 for t in seen] == [1, 1, 1, 1, 2, 2]
    # the first id's record now belongs to a newer generation
    rc, st = rt.query_async(seen[0])
    assert rc == p.PROM_ERROR and st.detail_code == p.DETAIL_ASYNC_NO_TASK
    d = rt.async_diagnostics()
    live = [d.tasks[i] for i in range(4) if d.tasks[i].task_id in seen]
    assert all(t.timing_valid == 1 and t.gpu_duration_ns > 0 for t in live if t.task_id in seen[-2:])


def test_failure_remains_visible_until_explicit_abandon():
    # reactor_stub_tests.cpp:1587-1636 (PROM_TESTCFG_FAIL_ASYNC_POLL)
    with p.NativeRuntime(test_flags=p.TESTCFG_FAIL_ASYNC_POLL) as rt:
        rt.require_hardware_gpu()
        m = n = k = 32
        a, b = oracle.deterministic_matrix(m, k), oracle.deterministic_matrix(k, n)
        rc, first, _ = rt.submit_async(m, n, k, a, b)
        assert rc == p.PROM_OK
        rc, st = rt.query_async(first)
        assert rc == p.PROM_OK and st.lifecycle_state == p.ASYNC_FAILED and st.failed == 1
        assert st.detail_code == p.DETAIL_INJECTED_ASYNC_POLL_FAILURE
        out = np.zeros(m * n, np.float32)
        rc, cs = rt.consume_async(first, out)
        assert rc == p.PROM_ERROR and cs.detail == p.DETAIL_INJECTED_ASYNC_POLL_FAILURE
        assert cs.detail != p.DETAIL_ASYNC_NOT_READY
        rc, second, _ = rt.submit_async(m, n, k, a, b)
        assert rc == p.PROM_OK
        d = rt.async_diagnostics()
        assert d.quarantine_event_count >= 1
        assert rt.abandon_async(first) == p.PROM_OK
        assert second > first
        assert rt.wait_async(second).lifecycle_state == p.ASYNC_FAILED
        assert rt.abandon_async(second) == p.PROM_OK


# ------------------------------------------------------------------ batch
def _plan_entries(count):
    # make_plan_entries (reactor_m29_fixed_double_tests.cpp:70-90), with the
    # test's deterministic_matrix ((i % 19) - 9) / 5 (:20-28)
    def det(rows, cols):
        i = np.arange(rows * cols)
        return (((i % 19) - 9) / 5.0).astype(np.float32).reshape(rows, cols)
    return [(det(2 + i, 4), det(4, 3)) for i in range(count)]


@pytest.mark.parametrize("width", [1, 2, 4])
def test_batch_logical_widths_use_the_device(rt, width):
    # reactor_m29_fixed_double_tests.cpp:286-316
    probs = _plan_entries(8)
    rc, cs, outs = rt.sgemm_batch(probs, flags=width)
    assert rc == p.PROM_OK and (cs.stage, cs.detail) == (p.STAGE_TRANSFER_OUT, 0)
    d = rt.batch_diagnostics()
    assert d.requested_workers == width and d.effective_workers == width
    assert d.partition_policy == p.BATCH_PARTITION_ROUND_ROBIN
    assert d.total_submits == 8 and d.m31_completion_count == 8 and d.m31_commit_count == 8
    assert d.output_committed == 1 and d.batch_state == p.BATCH_STATE_SUCCEEDED
    assert d.physical_ring_depth_effective > 0 and d.real_worker_thread_count == 0
    assert d.execution_mode == p.BATCH_EXECUTION_SINGLE_WORKER
    assert [d.worker_assigned_count[lane] for lane in range(width)] == [8 // width] * width
    for (a, b), c in zip(probs, outs):
        assert np.max(np.abs(c - oracle.cpu_sgemm_f32(a, b))) <= 1e-3
    assert [d.m31_commit_order[i] for i in range(8)] == list(range(8))
    assert all(d.m31_submission_sequence[i] != 0 for i in range(8))


def test_batch_contiguous_partition_and_width_cap(rt):
    # reactor_m29_fixed_double_tests.cpp:148-162, 244-264, 318-329
    rc, _, _ = rt.sgemm_batch(_plan_entries(7), flags=3 | p.BATCH_FLAG_PARTITION_CONTIGUOUS)
    assert rc == p.PROM_OK
    d = rt.batch_diagnostics()
    assert d.partition_policy == p.BATCH_PARTITION_CONTIGUOUS
    # floor(entry * 3 / 7) -> lanes [0,0,0,1,1,2,2]
    assert [d.worker_assigned_count[i] for i in range(3)] == [3, 2, 2]
    rc, _, _ = rt.sgemm_batch(_plan_entries(3), flags=7)
    d = rt.batch_diagnostics()
    assert rc == p.PROM_OK and d.requested_workers == 7 and d.effective_workers == 3 and d.total_submits == 3


def test_batch_plan_validates_before_admission(rt):
    # reactor_m29_fixed_double_tests.cpp:164-190: entry 3 has no B
    probs = _plan_entries(4)
    entries = (p.PrometheusSgemmBatchEntry * 4)()
    outs = []
    for i, (a, b) in enumerate(probs):
        c = np.full((a.shape[0], 3), -1.0, np.float32)
        outs.append(c)
        entries[i] = p.PrometheusSgemmBatchEntry(a.ctypes.data, None if i == 3 else b.ctypes.data, c.ctypes.data,
                                                 a.shape[0], 3, 4)
    rc, cs = rt.sgemm_batch_raw(entries, 4)
    assert (rc, cs.stage, cs.detail) == (p.PROM_ERROR, p.STAGE_INIT, p.DETAIL_BATCH_PLAN_INVALID)
    d = rt.batch_diagnostics()
    assert d.total_submits == 0 and d.failed_entry_id == 3 and d.output_committed == 0
    assert all(np.all(c == -1.0) for c in outs)


@pytest.mark.parametrize("flags,failed_entry", [
    (p.BATCH_FLAG_FAIL_AFTER_FIRST_SUBMIT, 0),
    (3 << p.BATCH_FLAG_TEST_FAIL_ENTRY_SHIFT, 2),
    (p.BATCH_FLAG_TEST_DUAL_FAIL_FIRST_TWO, 0),
])
def test_batch_failure_commits_nothing(rt, flags, failed_entry):
    # reactor_batch.c:382-407 (test seams) and :514-545 (no partial output)
    rc, cs, outs = rt.sgemm_batch(_plan_entries(6), flags=flags, test_entry=True)
    assert (rc, cs.stage, cs.detail) == (p.PROM_ERROR, p.STAGE_SUBMIT, p.DETAIL_BATCH_EXECUTION_FAILED)
    assert all(np.all(c == -1.0) for c in outs)
    d = rt.batch_diagnostics()
    assert d.batch_state == p.BATCH_STATE_FAILED and d.failed_entry_id == failed_entry
    assert d.output_committed == 0 and d.m31_commit_count == 0
    assert d.total_submits == failed_entry + (2 if flags == p.BATCH_FLAG_TEST_DUAL_FAIL_FIRST_TWO else 1)
    # the runtime stays usable
    rc, _, outs = rt.sgemm_batch(_plan_entries(2))
    assert rc == p.PROM_OK and np.all(outs[0] != -1.0)


def test_batch_mixed_shapes_every_kernel_path(rt):
    """Ragged MFMA tiles, split-K, GEMV and a 1x1, each against the oracle."""
    shapes = [(300, 200, 100), (1, 513, 257), (513, 1, 255), (1, 1, 1), (129, 127, 1025), (64, 256, 4),
              (1024, 1024, 1024)]
    probs = [(oracle.uniform(90 + i, (m, k)), oracle.uniform(190 + i, (k, n))) for i, (m, n, k) in enumerate(shapes)]
    rc, cs, outs = rt.sgemm_batch(probs, flags=2)
    assert rc == p.PROM_OK
    for (a, b), c in zip(probs, outs):
        _check(c, a, b)
    d = rt.batch_diagnostics()
    assert all(d.m31_gpu_duration_ns[i] > 0 for i in range(len(shapes)))
    assert [d.m31_completion_order[i] for i in range(len(shapes))] == list(range(len(shapes)))


def test_batch_ring_depth_one_recycles(rt):
    # reactor_m29_fixed_double_tests.cpp:192-216 (batch_ring_depth = 1)
    with p.NativeRuntime(batch_ring_depth=1) as r1:
        probs = _plan_entries(8)
        rc, _, outs = r1.sgemm_batch(probs)
        assert rc == p.PROM_OK
        d = r1.batch_diagnostics()
        assert d.physical_ring_depth_configured == 1 and d.plan_generation == 1
        assert [d.m31_commit_order[i] for i in range(8)] == list(range(8))
        for (a, b), c in zip(probs, outs):
            assert np.max(np.abs(c - oracle.cpu_sgemm_f32(a, b))) <= 1e-3
