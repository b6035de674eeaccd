"""The allocation-free SGEMM entry (prometheus_reactor_runtime_sgemm_device_noalloc)
against the allocating device entry it mirrors: same plan, so the outputs must be
bit-identical, and both within the fp32 parity bar of the binary64 oracle.  Two
calls in a row, the second smaller, so a stale scratch array would show; a plan
whose scratch (split-K partials, padded copies) exceeds the array is refused
without touching C; and in a fresh process the entry makes no device
allocation."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu

FP32_NORMWISE = 1e-5


def _run_pair(rt, m, n, k, seed):
    a = oracle.uniform(seed, (m, k))
    b = oracle.uniform(seed + 1, (k, n))
    da, db = rt.upload_new(a), rt.upload_new(b)
    dc_ref, dc_new = rt.alloc(m * n * 4), rt.alloc(m * n * 4)
    try:
        rt.sgemm_device(da, db, dc_ref, m, n, k)
        rc, st = rt.sgemm_device_noalloc(da, db, dc_new, m, n, k)
        assert rc == p.PROM_OK and st.stage == p.STAGE_SUBMIT, st
        assert st.detail in (p.DETAIL_PATH_HIP_MFMA_F32, p.DETAIL_PATH_HIP_GEMV_F32), st
        rt.synchronize()
        ref = rt.download(np.empty((m, n), np.float32), dc_ref)
        new = rt.download(np.empty((m, n), np.float32), dc_new)
    finally:
        for d in (da, db, dc_ref, dc_new):
            rt.free(d)
    return a, b, ref, new


@pytest.mark.parametrize("shapes", [((1056, 2048, 16384), (520, 1000, 6000))])
def test_noalloc_matches_the_device_entry_on_two_calls(gpu_runtime, shapes):
    for i, (m, n, k) in enumerate(shapes):
        rc, plan = p.sgemm_plan(m, n, k)
        assert rc == p.PROM_OK and 0 < plan.partial_bytes <= p.SGEMM_NOALLOC_SCRATCH_BYTES, "scratch must be used"
        print(f"noalloc call {i}: {m}x{n}x{k}, partials {plan.partial_bytes >> 20} MiB", flush=True)
        a, b, ref, new = _run_pair(gpu_runtime, m, n, k, 900 + 10 * i)
        assert np.array_equal(ref.view(np.uint32), new.view(np.uint32))
        rows = sorted({0, m // 2, plan.head_rows - 1, min(plan.head_rows, m - 1), m - 1})
        for r in rows:
            got = oracle.normwise_rel_err(new[r], oracle.matmul_f64(a, b, rows=(r, r + 1))[r])
            assert got <= FP32_NORMWISE, (m, n, k, r, got)


@pytest.mark.parametrize("m,n,k", [(1280, 2048, 8192), (1056, 3840, 3841)])
def test_noalloc_refuses_a_plan_beyond_the_scratch(gpu_runtime, m, n, k):
    """Split-K partials of 80 MiB; or no partials but 72 MiB of padded copies."""
    rc, plan = p.sgemm_plan(m, n, k)
    assert rc == p.PROM_OK and plan.scratch_bytes > p.SGEMM_NOALLOC_SCRATCH_BYTES
    sentinel = np.full((m, n), 7.0, np.float32)
    da, db, dc = gpu_runtime.alloc(m * k * 4), gpu_runtime.alloc(k * n * 4), gpu_runtime.upload_new(sentinel)
    try:
        rc, st = gpu_runtime.sgemm_device_noalloc(da, db, dc, m, n, k)
        gpu_runtime.synchronize()
        after = gpu_runtime.download(np.empty((m, n), np.float32), dc)
    finally:
        for d in (da, db, dc):
            gpu_runtime.free(d)
    assert rc == p.PROM_ERROR and st.stage == p.STAGE_TRANSFER_IN and st.detail == p.DETAIL_SCRATCH_LIMIT
    assert np.array_equal(after, sentinel)


def test_noalloc_repacking_plan(gpu_runtime):
    """Unaligned operands: the padded copies live in the same array as the partials."""
    m, n, k = 513, 1027, 131
    rc, plan = p.sgemm_plan(m, n, k)
    assert rc == p.PROM_OK and plan.repacked == 1 and plan.repack_bytes > 0
    a = oracle.uniform(961, (m, k))
    b = oracle.uniform(962, (k, n))
    da, db = gpu_runtime.upload_new(a), gpu_runtime.upload_new(b)
    dc_ref, dc_new = gpu_runtime.alloc(m * n * 4), gpu_runtime.alloc(m * n * 4)
    try:
        gpu_runtime.sgemm_device(da, db, dc_ref, m, n, k)
        rc, st = gpu_runtime.sgemm_device_noalloc(da, db, dc_new, m, n, k)
        assert rc == p.PROM_OK, st
        gpu_runtime.synchronize()
        ref = gpu_runtime.download(np.empty((m, n), np.float32), dc_ref)
        new = gpu_runtime.download(np.empty((m, n), np.float32), dc_new)
    finally:
        for d in (da, db, dc_ref, dc_new):
            gpu_runtime.free(d)
    assert np.array_equal(ref.view(np.uint32), new.view(np.uint32))
    assert oracle.normwise_rel_err(new, oracle.matmul_f64(a, b)) <= FP32_NORMWISE


def test_noalloc_without_split_and_gemv(gpu_runtime):
    """Plans with no partials (the 4096-wide direct tile, the GEMV) run the same way."""
    for (m, n, k) in ((512, 4096, 256), (8192, 1, 4096)):
        a, b, ref, new = _run_pair(gpu_runtime, m, n, k, 950 + m)
        assert np.array_equal(ref.view(np.uint32), new.view(np.uint32))


_CHILD = r"""
import json, sys
sys.path.insert(0, sys.argv[1])
import numpy as np
from oct_amd import prometheus as p
rt = p.NativeRuntime()
assert rt.caps.available == 1
before = rt.device_diagnostics().staging_allocations
held, out = [], {"before": before, "calls": []}
for m, n, k in ((1056, 2048, 16384), (513, 1027, 131)):
    plan = p.sgemm_plan(m, n, k)[1]
    a, b, c = rt.alloc(m * k * 4), rt.alloc(k * n * 4), rt.alloc(m * n * 4)
    held += [a, b, c]
    rc, st = rt.sgemm_device_noalloc(a, b, c, m, n, k)
    rt.synchronize()
    out["calls"].append({"shape": [m, n, k], "rc": rc, "partial": plan.partial_bytes, "repack": plan.repack_bytes,
                         "staging_allocations": rt.device_diagnostics().staging_allocations})
rt.sgemm_device(held[0], held[1], held[2], 1056, 2048, 16384)  # the allocating entry, for contrast
rt.synchronize()
out["after_allocating_entry"] = rt.device_diagnostics().staging_allocations
for d in held:
    rt.free(d)
rt.close()
print(json.dumps(out), flush=True)
"""


def test_noalloc_allocates_nothing_in_a_fresh_process():
    """A new process whose first SGEMMs go through the allocation-free entry
    (a split-K plan and a repacking plan): the library's staging allocator
    makes no device allocation, while the allocating entry afterwards does."""
    repo = str(Path(__file__).resolve().parent.parent)
    proc = subprocess.run([sys.executable, "-c", _CHILD, repo], capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stderr[-2000:]
    out = json.loads(proc.stdout.strip().splitlines()[-1])
    print(out, flush=True)
    assert out["calls"][0]["partial"] > 0 and out["calls"][1]["repack"] > 0
    for call in out["calls"]:
        assert call["rc"] == p.PROM_OK, call
        assert call["staging_allocations"] == out["before"], call
    assert out["after_allocating_entry"] > out["before"]
