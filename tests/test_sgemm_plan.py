"""The SGEMM launch plan and shape admission, checked on the CPU through the
C ABI's plan query (``prometheus_reactor_sgemm_plan``: a pure function of the
shape, no device).  The GPU tests of the same shapes assert the plan too, so a
refit of the plan model that changes which variant a parity case covers shows
up here first."""
from __future__ import annotations

import ctypes

import pytest

from oct_amd import prometheus as p


def _plan(m, n, k):
    rc, info = p.sgemm_plan(m, n, k)
    return rc, info


def test_headline_plan_is_the_direct_128x128_tile():
    rc, i = _plan(4096, 4096, 4096)
    assert rc == p.PROM_OK and i.detail_code == p.DETAIL_PATH_HIP_MFMA_F32
    assert i.products == 1 and (i.tile_m[0], i.tile_n[0], i.direct_to_lds[0], i.k_slices[0]) == (128, 128, 1, 1)
    assert i.launches == 1 and i.partial_bytes == 0


def test_gemv_plan():
    for m, k in ((8192, 4096), (1, 1), (513, 255)):
        rc, i = _plan(m, 1, k)
        assert rc == p.PROM_OK and i.detail_code == p.DETAIL_PATH_HIP_GEMV_F32 and i.products == 0 and i.launches == 1


@pytest.mark.parametrize("m,n,k", [(2049, 8192, 2048), (1056, 20480, 3840), (1056, 4096, 4096),
                                   # the C4 layer at T = 1056: output and down projections
                                   (1056, 2048, 2048), (1056, 2048, 16384)])
def test_tail_split_is_planned_for_the_seam_cases(m, n, k):
    rc, i = _plan(m, n, k)
    assert rc == p.PROM_OK and i.products == 2
    assert i.head_rows == m - m % 128
    assert i.k_slices[1] > 1  # the tail product is K-split
    assert i.launches == sum(2 if s > 1 else 1 for s in i.k_slices[:2])


def test_split_k_plan_reports_its_partial_buffer():
    rc, i = _plan(512, 2048, 16384)  # the C4 down projection
    assert rc == p.PROM_OK and i.products == 1 and i.k_slices[0] > 1
    assert i.partial_bytes == i.k_slices[0] * 512 * 2048 * 4
    assert i.k_slice_len[0] * i.k_slices[0] >= 16384 and i.k_slice_len[0] % 16 == 0


def test_c1_runs_on_one_64x64_tile_per_cu():
    """1024^3: 256 tiles of 64x64 (one per CU), the K range split between two
    wave groups inside each workgroup instead of across workgroups."""
    rc, i = _plan(1024, 1024, 1024)
    assert rc == p.PROM_OK and i.products == 1 and (i.tile_m[0], i.tile_n[0]) == (64, 64)
    assert i.k_slices[0] == 1 and i.launches == 1 and i.partial_bytes == 0 and i.direct_to_lds[0] == 1


def test_unaligned_operands_are_repacked_for_the_direct_kernels():
    """k = 513 and n = 3001 leave rows unaligned: A and B are copied to zero-padded
    [m][516] and [516][3004] buffers and the direct-to-LDS kernels run on them."""
    rc, i = _plan(4097, 3001, 513)
    assert rc == p.PROM_OK and i.repacked == 1 and i.direct_to_lds[0] == 1
    assert i.repack_bytes == 4 * (4097 * 516 + 516 * 3004)
    assert i.launches == 2 + sum(2 if s > 1 else 1 for s in i.k_slices[:i.products])


def test_k_tail_runs_direct_when_rows_are_aligned():
    """k = 1000 (a multiple of 4, not of 16): the 64x64 kernels take the K tail."""
    rc, i = _plan(1000, 1000, 1000)
    assert rc == p.PROM_OK and i.repacked == 0 and i.direct_to_lds[0] == 1 and (i.tile_m[0], i.tile_n[0]) == (64, 64)


@pytest.mark.parametrize("m,n,k", [(1, 1, 3_000_000_000), (3_000_000_000, 1, 1), (1, 2**31, 1),
                                   (70000, 70000, 1), (2**16, 1, 2**16), (2**31 - 1, 3, 1)])
def test_oversized_shapes_are_rejected(m, n, k):
    rc, i = _plan(m, n, k)
    assert rc == p.PROM_ERROR and i.detail_code == p.DETAIL_SIZE_OVERFLOW


def test_largest_admitted_shapes():
    for m, n, k in ((2**31 - 1, 1, 1), (1, 2**31 - 1, 1), (65535, 65535, 1), (2**31 - 1, 2, 1)):
        rc, i = _plan(m, n, k)
        assert rc == p.PROM_OK, (m, n, k)


def test_zero_dimension_and_bad_struct():
    rc, i = _plan(0, 4, 4)
    assert rc == p.PROM_ERROR and i.detail_code == p.PROM_ERROR
    lib = p.shared_library()
    small = p.PrometheusSgemmPlanInfo()
    small.struct_size = 8
    assert lib.prometheus_reactor_sgemm_plan(4, 4, 4, ctypes.byref(small)) == p.PROM_ERROR
    assert lib.prometheus_reactor_sgemm_plan(4, 4, 4, None) == p.PROM_ERROR


def test_device_entries_apply_the_same_admission():
    """Without a device the SGEMM entry stops at INIT (availability comes first, as in
    reactor_sgemm.cpp:4152-4191); the plan query shows the same shape is refused."""
    rt = p.NativeRuntime(test_flags=p.TESTCFG_SKIP_VULKAN_INIT)
    try:
        stage, detail = ctypes.c_uint32(0), ctypes.c_int(0)
        buf = (ctypes.c_float * 4)()
        rc = rt.lib.prometheus_reactor_runtime_sgemm(rt.handle, buf, buf, buf, 1, 1, 3_000_000_000,
                                                     ctypes.byref(stage), ctypes.byref(detail))
        assert rc == p.PROM_ERROR and stage.value == p.STAGE_INIT and detail.value == p.DETAIL_HIP_UNAVAILABLE
    finally:
        rt.close()
    assert _plan(1, 1, 3_000_000_000)[1].detail_code == p.DETAIL_SIZE_OVERFLOW


def test_legacy_aliases_forward_to_the_runtime_entries():
    """reactor_api.h:2822-2825: prometheus_runtime_create / destroy / probe."""
    lib = p.shared_library()
    handle = ctypes.c_void_p()
    assert lib.prometheus_runtime_create(None, ctypes.byref(handle)) == p.PROM_OK and handle.value
    caps = p.PrometheusCaps()
    assert lib.prometheus_runtime_probe(handle, ctypes.byref(caps)) == p.PROM_OK
    # Same answer through the primary entry point.
    caps2 = p.PrometheusCaps()
    assert lib.prometheus_reactor_runtime_probe(handle, ctypes.byref(caps2)) == p.PROM_OK
    assert (caps.available, caps.backend_type, caps.reason_code) == \
        (caps2.available, caps2.backend_type, caps2.reason_code)
    assert lib.prometheus_runtime_destroy(handle) == p.PROM_OK
    assert lib.prometheus_runtime_destroy(handle) == p.PROM_INVALID_HANDLE
    assert lib.prometheus_runtime_probe(handle, ctypes.byref(caps)) == p.PROM_INVALID_HANDLE
    assert lib.prometheus_runtime_create(None, None) == p.PROM_ERROR


def test_scratch_bytes_is_what_the_noalloc_entry_needs():
    """scratch_bytes = split-K partials rounded up to 256 bytes + the padded
    copies of A and B: the exact rule of ..._sgemm_device_noalloc, which
    refuses a plan whose scratch_bytes exceeds its 64 MiB array even when it
    writes no partials (the repacking plans of large unaligned products)."""
    for m, n, k in ((4097, 4097, 4097), (1056, 3840, 3841), (1280, 2048, 8192), (513, 1027, 131),
                    (1056, 2048, 16384), (4096, 4096, 4096), (8192, 1, 4096)):
        rc, i = _plan(m, n, k)
        assert rc == p.PROM_OK
        assert i.scratch_bytes == (i.partial_bytes + 255) // 256 * 256 + i.repack_bytes, (m, n, k)
    rc, i = _plan(1056, 3840, 3841)
    assert i.partial_bytes == 0 and i.repacked == 1 and i.scratch_bytes > p.SGEMM_NOALLOC_SCRATCH_BYTES
    rc, i = _plan(8192, 1, 4096)  # the GEMV needs none
    assert i.scratch_bytes == 0


def test_plan_accepts_the_struct_without_scratch_bytes():
    """A caller's struct that ends at repack_bytes is still served, and the
    bytes past it are left alone."""
    lib = p.shared_library()
    short = p.PrometheusSgemmPlanInfo.scratch_bytes.offset
    buf = (ctypes.c_ubyte * ctypes.sizeof(p.PrometheusSgemmPlanInfo))()
    ctypes.memset(buf, 0xAB, len(buf))
    info = p.PrometheusSgemmPlanInfo.from_buffer(buf)
    info.struct_size = short
    assert lib.prometheus_reactor_sgemm_plan(1056, 3840, 3841, ctypes.byref(info)) == p.PROM_OK
    assert info.repacked == 1 and info.repack_bytes > 0
    assert bytes(buf[short:]) == b"\xab" * (len(buf) - short)
    info.struct_size = short - 1
    assert lib.prometheus_reactor_sgemm_plan(4, 4, 4, ctypes.byref(info)) == p.PROM_ERROR
