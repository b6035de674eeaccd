"""Pins the wiring of the block oracles (oracle/blocks.py) with closed forms.

Each block function is evaluated on the closed-form inputs of
tests/closed_forms.py and must reproduce the stage recurrences there to
1e-12.  Then a copy of the oracle with one plausible misreading planted in
its source (a named edit of the function's text, applied in this process
only) must miss the closed form by more than five times the GPU parity bar
of that block, so the same closed form run through the HIP block in
tests/test_gpu_blocks.py and tests/test_gpu_model_block.py rejects the
misreading as well.
"""
import inspect
import textwrap

import numpy as np
import pytest

import oracle
from oracle import blocks
from tests import closed_forms as cf

BF16_BAR, F32_BAR = 2e-2, 1e-3


def planted(fn_name: str, edits, *also):
    """``blocks.<fn_name>`` with every (old, new) text edit applied; ``also``
    holds (helper name, edits) pairs for helpers it calls by name."""
    ns = dict(vars(blocks))
    for name, changes in (*also, (fn_name, edits)):
        src = textwrap.dedent(inspect.getsource(getattr(blocks, name)))
        for old, new in changes:
            assert src.count(old) == 1, f"{name}: the oracle text no longer holds {old!r}"
            src = src.replace(old, new)
        exec(compile(src, f"<planted {name}>", "exec"), ns)
    return ns[fn_name]


def rel(got, want):
    return float(np.linalg.norm(np.asarray(got, np.float64) - want) / np.linalg.norm(want))


# ----------------------------------------------------------------- DiT block
# Not listed: scaleA moved inside the attention pre-norm.  With identical
# tokens that only rescales every V row by one factor, which the post-attention
# RMSNorm removes, so no closed form of this kind can see it; the loop
# restatement on random tokens (test_oracle_blocks.py) covers the order.
DIT_MISREADINGS = {
    "gate inside the post-attention norm": ("dit_block_bf16", [(
        "gate_a * rmsnorm(proj, w.attn_norm2, eps)", "rmsnorm(gate_a * proj, w.attn_norm2, eps)")]),
    "post-attention norm dropped": ("dit_block_bf16", [(
        "gate_a * rmsnorm(proj, w.attn_norm2, eps)", "gate_a * proj")]),
    "FFN pre-norm dropped before scaleM": ("dit_block_bf16", [(
        "rmsnorm(r, w.ffn_norm1, eps) * scale_m", "r * scale_m")]),
    "gate and up swapped": ("dit_block_bf16", [(
        "silu(f @ w13[:, :F]) * (f @ w13[:, F:])", "silu(f @ w13[:, F:]) * (f @ w13[:, :F])")]),
    "GELU for SiLU": ("dit_block_bf16", [("silu(f @ w13", "gelu_tanh(f @ w13")]),
    "FFN output norm dropped": ("dit_block_bf16", [(
        "gate_m * rmsnorm(hdn @ wf(w.w_2), w.ffn_norm2, eps)", "gate_m * (hdn @ wf(w.w_2))")]),
    "residual taken from the modulated stream": ("dit_block_bf16", [("r = x[sel] + gate_a", "r = a[sel] + gate_a")]),
    "norm weights exchanged": ("dit_block_bf16", [("w.attn_norm2, eps", "w.ffn_norm2, eps"),
                                                  ("w.w_2), w.ffn_norm2, eps", "w.w_2), w.attn_norm2, eps")]),
}
ADALN_MISREADINGS = {
    "scale for 1 + scale": [("return 1.0 + chunks[0]", "return chunks[0]")],
    "gate without tanh": [("np.tanh(chunks[1])", "chunks[1]")],
    "adaLN chunks 1 and 2 exchanged": [("np.tanh(chunks[1]), 1.0 + chunks[2]", "np.tanh(chunks[2]), 1.0 + chunks[1]")],
}


def _dit_inputs():
    return cf.dit_case(tokens=5, heads=2, ffn=512, cond_dim=8)


def test_dit_block_closed_form():
    x, coords, cond, w = _dit_inputs()
    got = blocks.dit_block_bf16(x, coords, cond, w, heads=2)
    want = cf.dit_expected(5, 256)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
    assert np.ptp(want[0, :4]) > 1.0  # the four classes stay apart


@pytest.mark.parametrize("name", sorted(DIT_MISREADINGS))
def test_dit_block_closed_form_rejects(name):
    fn_name, edits = DIT_MISREADINGS[name]
    x, coords, cond, w = _dit_inputs()
    got = planted(fn_name, edits)(x, coords, cond, w, heads=2)
    assert rel(got, cf.dit_expected(5, 256)) > 5 * BF16_BAR, name


@pytest.mark.parametrize("name", sorted(ADALN_MISREADINGS))
def test_dit_block_closed_form_rejects_adaln(name):
    x, coords, cond, w = _dit_inputs()
    got = planted("dit_block_bf16", [], ("adaln_modulation", ADALN_MISREADINGS[name]))(x, coords, cond, w, heads=2)
    assert rel(got, cf.dit_expected(5, 256)) > 5 * BF16_BAR, name


def test_dit_closed_form_survives_uneven_scores():
    """At five different coordinates, with random W_q and W_k, a query's
    scores differ from key to key; the output is still the closed form."""
    x, coords, cond, w = _dit_inputs()
    coords = blocks.joint_coordinates(1, 3, 2)  # five different coordinates
    got = blocks.dit_block_bf16(x, coords, cond, w, heads=2)
    np.testing.assert_allclose(got, cf.dit_expected(5, 256), rtol=0, atol=1e-12)


# ---------------------------------------------------- resident Z-Image blocks
ZIMAGE_MISREADINGS = {
    "gate inside the post-attention norm": [(
        "gate_a * rmsnorm(proj, f(\"attn_norm2\"), eps)", "rmsnorm(gate_a * proj, f(\"attn_norm2\"), eps)")],
    "post-attention norm dropped": [("gate_a * rmsnorm(proj, f(\"attn_norm2\"), eps)", "gate_a * proj")],
    "FFN pre-norm dropped": [("fn = rmsnorm(r, f(\"ffn_norm1\"), eps)", "fn = r")],
    "scale for 1 + scale": [("scale_a, gate_a = 1.0 + raw[:D]", "scale_a, gate_a = raw[:D]")],
    "gate without tanh": [("gate_m = 1.0 + raw[2 * D:3 * D], np.tanh(raw[3 * D:])",
                           "gate_m = 1.0 + raw[2 * D:3 * D], raw[3 * D:]")],
    "gate and up swapped": [("hdn = silu(w1) * w3", "hdn = silu(w3) * w1")],
    "FFN output norm dropped": [("gate_m * rmsnorm(w2, f(\"ffn_norm2\"), eps)", "gate_m * w2")],
    "residual taken from the normed stream": [("r = x[sel] + gate_a", "r = normed[sel] + gate_a")],
    "scaleA also applied before the attention pre-norm": [(
        "normed = rmsnorm(x, f(\"attn_norm1\"), eps)", "normed = rmsnorm(x * scale_a, f(\"attn_norm1\"), eps)")],
}
# the ContextRefiner has no adaLN: scale and gate are 1, so only the misreadings
# that do not involve them apply
CONTEXT_MISREADINGS = ("post-attention norm dropped", "FFN pre-norm dropped", "gate and up swapped",
                       "FFN output norm dropped", "residual taken from the normed stream")


def _zimage_inputs(modulated, T=4, D=256, F=512):
    w = cf.zimage_case(modulated, D, F)
    x = np.tile(cf.tile(cf.X, D), (T, 1)).astype(np.float32)
    coords = blocks.image_coordinates(T) if modulated else blocks.context_coordinates(T)
    cond = np.random.default_rng(3).standard_normal(256).astype(np.float32) if modulated else None
    return x, coords, w, cond


@pytest.mark.parametrize("modulated", [True, False])
def test_zimage_block_closed_form(modulated):
    x, coords, w, cond = _zimage_inputs(modulated)
    got = blocks.zimage_block_f64(x, coords, w, cond, heads=2)
    np.testing.assert_allclose(got, cf.zimage_expected(4, modulated, 256), rtol=0, atol=1e-12)


@pytest.mark.parametrize("name", sorted(ZIMAGE_MISREADINGS))
def test_zimage_block_closed_form_rejects(name):
    x, coords, w, cond = _zimage_inputs(True)
    got = planted("zimage_block_f64", ZIMAGE_MISREADINGS[name])(x, coords, w, cond, heads=2)
    # the resident fp32 blocks are held to 5e-5; the margin asked here is the bf16 one
    assert rel(got, cf.zimage_expected(4, True, 256)) > 5 * BF16_BAR, name


@pytest.mark.parametrize("name", CONTEXT_MISREADINGS)
def test_context_refiner_closed_form_rejects(name):
    x, coords, w, cond = _zimage_inputs(False)
    got = planted("zimage_block_f64", ZIMAGE_MISREADINGS[name])(x, coords, w, cond, heads=2)
    assert rel(got, cf.zimage_expected(4, False, 256)) > 5 * BF16_BAR, name


def test_context_refiner_closed_form_is_unmodulated():
    """A ContextRefiner that applied the NoiseRefiner's modulation would be a
    different function: the two closed forms differ."""
    assert rel(cf.zimage_expected(1, True, 8), cf.zimage_expected(1, False, 8)) > 0.1


# ---------------------------------------------------------------- Gemma layer
DECODER_MISREADINGS = {
    "gate and up swapped": [("gelu_tanh(gu[:, :F]) * gu[:, F:]", "gelu_tanh(gu[:, F:]) * gu[:, :F]")],
    "FFN pre-norm dropped": [("n2 = rmsnorm(h, w.ffn_norm, eps)", "n2 = h")],
    "attention norm weight in the FFN norm": [("rmsnorm(h, w.ffn_norm, eps)", "rmsnorm(h, w.attn_norm, eps)")],
    "attention pre-norm dropped": [("n1 = rmsnorm(x, w.attn_norm, eps)", "n1 = x")],
    "attention residual from the normed stream": [("h = x + o @", "h = n1 + o @")],
    "FFN residual onto x": [("return h + a @", "return x + a @")],
    "SiLU for GELU": [("a = gelu_tanh(gu[:, :F])", "a = silu(gu[:, :F])")],
    "GELU on the up half": [("gelu_tanh(gu[:, :F]) * gu[:, F:]", "gu[:, :F] * gelu_tanh(gu[:, F:])")],
}


def _decoder_inputs(T=6, D=256, Hq=2, d=128, F=512):
    return cf.decoder_case(T, D, Hq, d, F)


def test_decoder_layer_closed_form():
    x, w = _decoder_inputs()
    got = blocks.decoder_layer_f32(x, w, 2, 128)
    np.testing.assert_allclose(got, cf.decoder_expected(6, 256), rtol=0, atol=1e-12)


@pytest.mark.parametrize("name", sorted(DECODER_MISREADINGS))
def test_decoder_layer_closed_form_rejects(name):
    x, w = _decoder_inputs()
    got = planted("decoder_layer_f32", DECODER_MISREADINGS[name])(x, w, 2, 128)
    assert rel(got, cf.decoder_expected(6, 256)) > 5 * F32_BAR, name


def test_planted_edit_must_apply():
    """A misreading whose text is not in the oracle fails loudly instead of
    testing the unmodified oracle."""
    with pytest.raises(AssertionError):
        planted("decoder_layer_f32", [("no such text", "x")])
