"""Pins the binary64 oracle of the resident fp32 Z-Image blocks
(oracle/blocks.py: zimage_block_f64, rope_canonical_f32).

* RoPE follows CanonicalRopeRotate (zimage/canonical_contract.go:66-87) and
  reproduces the reference's captured frame-33 witness pair
  (tests/golden/qkv_rope_selected.octagon).
* The modulated block equals the independently pinned bf16 DiT oracle when
  every weight is exactly representable in both FP16 and BF16 (the only
  difference left is the float32 RoPE angle, ~1e-7 relative).
* The unmodulated ContextRefiner equals a loop restatement written in the
  form of context_refiner_reference.go:230-311 (no adaLN, plain residual adds).
"""
import math

import numpy as np
import pytest

import oracle
from oracle import blocks
from tests.golden import octagon


def test_rope_canonical_matches_captured_witness():
    wit = octagon.load("qkv_rope_selected.octagon")
    x = np.zeros((1, 1, 128))
    x[0, 0, 8], x[0, 0, 9] = wit["QNormPair.Even"], wit["QNormPair.Odd"]
    out = blocks.rope_canonical_f32(x, np.array([[33.0, 0.0, 0.0]], np.float32))
    assert abs(out[0, 0, 8] - (-0.4407204)) <= 1e-6 and abs(out[0, 0, 9] - (-0.1587258)) <= 1e-6


def test_rope_canonical_angle_is_float32():
    # angle = float32(coord) * float32(freq), rounded to float32 before cos/sin
    x = np.zeros((1, 1, 128))
    x[0, 0, 34], x[0, 0, 35] = 1.0, 0.0  # axis 1 (width 48), pair 1
    out = blocks.rope_canonical_f32(x, np.array([[0.0, 31.0, 0.0]], np.float32))
    freq = np.float32(1.0 / math.pow(256.0, 2.0 / 48.0))
    angle = float(np.float32(np.float32(31.0) * freq))
    assert out[0, 0, 34] == math.cos(angle) and out[0, 0, 35] == math.sin(angle)
    # identity at the zero coordinate; norm preserved elsewhere
    x = np.random.default_rng(1).standard_normal((3, 2, 128))
    zero = blocks.rope_canonical_f32(x, np.zeros((3, 3), np.float32))
    np.testing.assert_array_equal(zero, x)
    rot = blocks.rope_canonical_f32(x, blocks.image_coordinates(3))
    np.testing.assert_allclose(np.linalg.norm(rot, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-13)


def test_coordinates_follow_the_canonical_contract():
    c = blocks.image_coordinates(1024)
    assert c.shape == (1024, 3) and (c[:, 0] == 33).all()
    assert tuple(c[33]) == (33.0, 1.0, 1.0) and tuple(c[1023]) == (33.0, 31.0, 31.0)
    k = blocks.context_coordinates(32)
    assert tuple(k[0]) == (1.0, 0.0, 0.0) and tuple(k[31]) == (32.0, 0.0, 0.0)
    # the joint sequence is image then context (zimage_main_transformer_canonical.py:146-155)
    j = blocks.joint_coordinates(32, 32, 15)
    np.testing.assert_array_equal(j[:1024], c)
    np.testing.assert_array_equal(j[1024:], blocks.context_coordinates(15))


def _shared_exact(a: np.ndarray) -> np.ndarray:
    """Round to BF16, then drop values FP16 cannot hold exactly (tiny magnitudes)."""
    b = oracle.from_bf16(oracle.to_bf16(a)).astype(np.float32)
    b[np.abs(b) < 2.0 ** -14] = 0.0
    assert np.array_equal(b.astype(np.float16).astype(np.float32), b)
    return b


@pytest.mark.parametrize("seed", [0, 1])
def test_modulated_block_equals_the_bf16_dit_oracle(seed):
    T, Dm, F, H = 9, 256, 64, 2
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, Dm)).astype(np.float32)
    cond = rng.standard_normal(256).astype(np.float32)
    w = blocks.make_zimage_weights(seed, True, Dm, F)
    w = {k: _shared_exact(v.astype(np.float32) * (8.0 if v.ndim == 2 else 1.0)) for k, v in w.items()}
    coords = blocks.image_coordinates(T)
    got = blocks.zimage_block_f64(x, coords, w, cond, heads=H)
    dw = blocks.DitBlockWeights(
        w_adaln=oracle.to_bf16(w["adaln_w"]), b_adaln=w["adaln_b"].astype(np.float64),
        attn_norm1=w["attn_norm1"], attn_norm2=w["attn_norm2"], ffn_norm1=w["ffn_norm1"],
        ffn_norm2=w["ffn_norm2"], q_norm=w["q_norm"], k_norm=w["k_norm"],
        w_qkv=oracle.to_bf16(w["w_qkv"]), w_out=oracle.to_bf16(w["w_out"]),
        w_13=oracle.to_bf16(np.concatenate((w["w1"], w["w3"]), axis=1)), w_2=oracle.to_bf16(w["w2"]))
    ref = blocks.dit_block_bf16(x, coords, cond, dw, heads=H)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)
    # a row subset evaluates exactly those rows
    np.testing.assert_allclose(blocks.zimage_block_f64(x, coords, w, cond, heads=H, rows=[0, 5]), got[[0, 5]],
                               rtol=1e-13, atol=1e-13)


def _context_loops(x, w, coords, heads, eps=1e-5):
    """context_refiner_reference.go:230-311 as written: row loops, channel
    loops, per-head attention loops (binary64)."""
    T, Dm = x.shape
    hd = Dm // heads
    F = w["w2"].shape[0]
    f = {k: np.asarray(v, np.float64) for k, v in w.items()}

    def norm_rows(v, scale):
        out = np.empty_like(v)
        for r in range(v.shape[0]):
            s = 0.0
            for c in range(v.shape[1]):
                s += v[r, c] * v[r, c]
            den = 1.0 / math.sqrt(s / v.shape[1] + eps)
            for c in range(v.shape[1]):
                out[r, c] = v[r, c] * den * scale[c]
        return out

    def linear(v, wt):
        out = np.zeros((v.shape[0], wt.shape[1]))
        for r in range(v.shape[0]):
            for c in range(wt.shape[0]):
                out[r] += v[r, c] * wt[c]
        return out

    def rotate(vec, coord):
        out = vec.copy()
        base = 0
        for axis, width in enumerate((32, 48, 48)):
            for pair in range(width // 2):
                freq = np.float32(1.0 / math.pow(256.0, 2.0 * pair / width))
                ang = float(np.float32(np.float32(coord[axis]) * freq))
                e, o = vec[base + 2 * pair], vec[base + 2 * pair + 1]
                out[base + 2 * pair] = e * math.cos(ang) - o * math.sin(ang)
                out[base + 2 * pair + 1] = e * math.sin(ang) + o * math.cos(ang)
            base += width
        return out

    norm = norm_rows(x.astype(np.float64), f["attn_norm1"])
    qkv = linear(norm, f["w_qkv"])
    q = norm_rows(qkv[:, :Dm].reshape(T * heads, hd), f["q_norm"]).reshape(T, heads, hd)
    k = norm_rows(qkv[:, Dm:2 * Dm].reshape(T * heads, hd), f["k_norm"]).reshape(T, heads, hd)
    v = qkv[:, 2 * Dm:].reshape(T, heads, hd)
    for t in range(T):
        for h in range(heads):
            q[t, h] = rotate(q[t, h], coords[t])
            k[t, h] = rotate(k[t, h], coords[t])
    attn = np.zeros((T, heads, hd))
    for t in range(T):
        for h in range(heads):
            scores = [float(np.dot(q[t, h], k[j, h])) / math.sqrt(hd) for j in range(T)]
            m = max(scores)
            p = [math.exp(s - m) for s in scores]
            tot = sum(p)
            for j in range(T):
                attn[t, h] += (p[j] / tot) * v[j, h]
    proj = linear(attn.reshape(T, Dm), f["w_out"])
    resid = x + norm_rows(proj, f["attn_norm2"])
    ffn = norm_rows(resid, f["ffn_norm1"])
    w1, w3 = linear(ffn, f["w1"]), linear(ffn, f["w3"])
    hidden = (w1 / (1.0 + np.exp(-w1))) * w3
    return resid + norm_rows(linear(hidden, f["w2"]), f["ffn_norm2"])


def test_unmodulated_block_matches_the_context_refiner_loops():
    T, Dm, F, H = 4, 256, 16, 2
    rng = np.random.default_rng(7)
    x = rng.standard_normal((T, Dm)).astype(np.float32)
    w = blocks.make_zimage_weights(7, False, Dm, F)
    w = {k: (v.astype(np.float32) * (6.0 if v.ndim == 2 else 1.0)).astype(np.float16) for k, v in w.items()}
    coords = blocks.context_coordinates(T)
    got = blocks.zimage_block_f64(x, coords, w, None, heads=H)
    ref = _context_loops(x, {k: v.astype(np.float64) for k, v in w.items()}, coords, H)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-10)


def test_stages_are_consistent_with_the_output():
    T, Dm, F, H = 6, 256, 32, 2
    rng = np.random.default_rng(3)
    x = rng.standard_normal((T, Dm)).astype(np.float32)
    cond = rng.standard_normal(256).astype(np.float32)
    w = blocks.make_zimage_weights(3, True, Dm, F)
    st = {}
    out = blocks.zimage_block_f64(x, blocks.image_coordinates(T), w, cond, heads=H, stages=st)
    np.testing.assert_array_equal(st["final_output"], out)
    np.testing.assert_allclose(st["ffn_gated_hidden"], st["w1"] / (1 + np.exp(-st["w1"])) * st["w3"], rtol=1e-14)
    raw = st["adaln_projection"]
    np.testing.assert_allclose(st["ffn_modulated"], st["ffn_norm"] * (1.0 + raw[2 * Dm:3 * Dm]), rtol=1e-14)
