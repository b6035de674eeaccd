"""GPU parity of the bf16 flash attention (the DiT block's attention) against
the block oracle's attention, per head softmax_rows(Q K^T / sqrt(128)) V in
binary64 on the same bf16 inputs (oracle/blocks.py, as dit_block_bf16 uses it).

Bar: 1e-2 normwise per head (P and O are rounded to bf16 on the way, about
2^-9 relative each; the north_star bf16 bar is 2e-2).  Both kernels (the
DMA-fed one, which the DiT block runs, and the register-staged one) run on
every case and agree with each other to 5e-3.  Shapes cover one partial tile, exact tiles, a
ragged last tile and a partial last query block, padded leading dimensions,
and the full C5 attention (4224 tokens x 30 heads)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import blocks
from oct_amd import prometheus as p

pytestmark = pytest.mark.gpu

ATTN_BF16 = 1e-2
VARIANT_AGREE = 5e-3
VARIANTS = (0, 1)


def _inputs(seed, tokens, heads, ld, q_scale):
    q = oracle.to_bf16(oracle.normal(seed, (tokens, ld), 0.0, q_scale))
    k = oracle.to_bf16(oracle.normal(seed + 1, (tokens, ld)))
    v = oracle.to_bf16(oracle.normal(seed + 2, (tokens, ld)))
    return q, k, v


def _reference(q, k, v, h):
    cols = slice(128 * h, 128 * h + 128)
    qf = oracle.from_bf16(q[:, cols]).astype(np.float64)
    kf = oracle.from_bf16(k[:, cols]).astype(np.float64)
    vf = oracle.from_bf16(v[:, cols]).astype(np.float64)
    return blocks.softmax_rows(qf @ kf.T / np.sqrt(128.0)) @ vf


def _run(rt, q, k, v, tokens, heads, ld, variant):
    dq, dk, dv = rt.upload_new(q), rt.upload_new(k), rt.upload_new(v)
    do = rt.upload_new(np.full((tokens, ld), 0x7fc0, np.uint16))  # NaN fill: every output must be written
    try:
        rc, st = rt.attention_bf16_device(dq, dk, dv, do, tokens, heads, ld, variant)
        assert rc == p.PROM_OK, st
        rt.synchronize()
        out = rt.download(np.empty((tokens, ld), np.uint16), do)
    finally:
        for d in (dq, dk, dv, do):
            rt.free(d)
    return out


@pytest.mark.parametrize("tokens,heads,extra,q_scale", [(1, 1, 0, 1.0), (19, 1, 8, 3.0), (64, 1, 0, 3.0),
                                                        (65, 2, 0, 3.0), (130, 2, 16, 1.0), (300, 3, 8, 4.0),
                                                        (1056, 2, 0, 3.0)])
def test_attention_shapes(gpu_runtime, tokens, heads, extra, q_scale):
    ld = 128 * heads + extra
    q, k, v = _inputs(7 + tokens, tokens, heads, ld, q_scale)
    outs = [_run(gpu_runtime, q, k, v, tokens, heads, ld, variant) for variant in VARIANTS]
    for h in range(heads):
        ref = _reference(q, k, v, h)
        got = [oracle.from_bf16(o[:, 128 * h:128 * h + 128]).astype(np.float64) for o in outs]
        for variant, g in enumerate(got):
            assert np.all(np.isfinite(g)), (variant, h)
            err = oracle.normwise_rel_err(g, ref)
            print(f"T={tokens} head {h} variant {variant}: normwise rel err {err:.2e}", flush=True)
            assert err <= ATTN_BF16, (variant, h, err)
        for g in got[1:]:
            assert oracle.normwise_rel_err(got[0], g) <= VARIANT_AGREE
    # padding columns past the heads are left alone
    if extra:
        for o in outs:
            assert np.all(o[:, 128 * heads:] == 0x7fc0)


def test_attention_c5_full(gpu_runtime):
    """The C5 block's attention: 4224 tokens (64 x 64 image + 128 text), 30 heads of 128."""
    tokens, heads = 4224, 30
    ld = 128 * heads
    q, k, v = _inputs(55, tokens, heads, ld, 3.0)
    print("C5 attention on the GPU (all kernels) ...", flush=True)
    outs = [_run(gpu_runtime, q, k, v, tokens, heads, ld, variant) for variant in VARIANTS]
    for h in (0, 13, 29):
        ref = _reference(q, k, v, h)
        got = oracle.from_bf16(outs[0][:, 128 * h:128 * h + 128]).astype(np.float64)
        err = oracle.normwise_rel_err(got, ref)
        print(f"C5 head {h}: normwise rel err {err:.2e}", flush=True)
        assert err <= ATTN_BF16
    a = oracle.from_bf16(outs[0]).astype(np.float64)
    assert np.all(np.isfinite(a))
    for o in outs[1:]:
        assert oracle.normwise_rel_err(a, oracle.from_bf16(o).astype(np.float64)) <= VARIANT_AGREE


def test_attention_rejects_bad_arguments(gpu_runtime):
    rt = gpu_runtime
    buf = rt.alloc(64 * 256 * 2)
    try:
        for args in ((64, 2, 128, 0), (64, 1, 129, 0), (0, 1, 128, 0), (64, 1, 128, 2), (64, 0, 128, 0), (1, 1, 1 << 24, 0)):
            rc, st = rt.attention_bf16_device(buf, buf, buf, buf, *args)
            assert rc == p.PROM_ERROR and st.stage == p.STAGE_INIT and st.detail == p.DETAIL_INVALID_ARGUMENT, args
        rc, st = rt.attention_bf16_device(buf + 2, buf, buf, buf, 64, 1, 128, 0)
        assert rc == p.PROM_ERROR and st.detail == p.DETAIL_INVALID_ARGUMENT
    finally:
        rt.free(buf)
