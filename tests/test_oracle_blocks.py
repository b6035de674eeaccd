"""Pins the binary64 block oracles (oracle/blocks.py) with independent checks.

Each piece is compared with the pinned C oracle, a loop restatement written
in the reference's own formulation, a closed form, or an invariant that a
wrong sign, pairing or index would break.
"""
import math

import numpy as np
import pytest

import oracle
from oracle import blocks


def test_rmsnorm_matches_pinned_c_oracle():
    x = oracle.normal(5, (7, 96))
    w = oracle.normal(6, (96,), 1.0, 0.1)
    rc, y_c, _ = oracle.rmsnorm_reference(x, w, 1e-6)
    np.testing.assert_allclose(blocks.rmsnorm(x, w, 1e-6), y_c, rtol=2e-6, atol=1e-7)
    # uncentered: [2, 2] -> [1, 1] (zimage/canonical_contract_test.go:45-53)
    np.testing.assert_allclose(blocks.rmsnorm(np.array([[2.0, 2.0]]), np.ones(2), 1e-5), [[1.0, 1.0]], atol=1e-5)


def test_gelu_tanh_closed_form_values():
    x = np.array([0.0, 1.0, -1.0, 3.0])
    expect = [0.0, 0.8411919906082768, -0.15880800939172324, 2.99636281]
    np.testing.assert_allclose(blocks.gelu_tanh(x), expect, rtol=1e-7, atol=1e-12)


def test_silu_closed_form():
    np.testing.assert_allclose(blocks.silu(np.array([0.0, 1.0, -2.0])),
                               [0.0, 1 / (1 + math.exp(-1)), -2 / (1 + math.exp(2))], rtol=1e-15)


def _rope_component_loop(src, positions, base):
    """gemma4e2b_m1_rtx.go:834-861 formulation: component c, frequency c % (d/2),
    mate c +- d/2, first - second below d/2 and first + second above (no BF16)."""
    T, H, d = src.shape
    out = np.zeros_like(src)
    for t in range(T):
        for h in range(H):
            for c in range(d):
                f = c % (d // 2)
                mate = f + d // 2 if c < d // 2 else f
                ang = positions[t] * base ** (-2.0 * f / d)
                first = src[t, h, c] * math.cos(ang)
                second = src[t, h, mate] * math.sin(ang)
                out[t, h, c] = first - second if c < d // 2 else first + second
    return out


def test_rope_half_split_matches_reference_formulation():
    x = oracle.normal(1, (5, 2, 8)).astype(np.float64)
    pos = np.arange(3, 8)
    np.testing.assert_allclose(blocks.rope_half_split(x, pos, 10000.0), _rope_component_loop(x, pos, 10000.0),
                               rtol=1e-13, atol=1e-13)


def test_rope_identity_at_zero_and_relative_position_property():
    x = oracle.normal(2, (1, 1, 16)).astype(np.float64)
    np.testing.assert_array_equal(blocks.rope_half_split(x, np.array([0]), 10000.0), x)
    # <R(m) q, R(n) k> depends only on m - n
    q = oracle.normal(3, (1, 1, 16)).astype(np.float64)
    k = oracle.normal(4, (1, 1, 16)).astype(np.float64)
    dots = []
    for m, n in ((5, 2), (13, 10), (103, 100)):
        qm = blocks.rope_half_split(q, np.array([m]), 10000.0)
        kn = blocks.rope_half_split(k, np.array([n]), 10000.0)
        dots.append(float(np.sum(qm * kn)))
    np.testing.assert_allclose(dots, dots[0], rtol=1e-10)
    # each (i, i + d/2) pair keeps its magnitude
    r = blocks.rope_half_split(q, np.array([77]), 10000.0)
    np.testing.assert_allclose(r[..., :8] ** 2 + r[..., 8:] ** 2, q[..., :8] ** 2 + q[..., 8:] ** 2, rtol=1e-12)


def _layer_loops(x, w, Hq, d, eps, base):
    """Loop restatement of the layer for a tiny shape (independent of numpy broadcasting)."""
    T, D = x.shape
    F = w.w_down.shape[0]

    def rms_row(v, g):
        s = sum(float(a) * float(a) for a in v)
        inv = 1.0 / math.sqrt(s / len(v) + eps)
        return [float(a) * inv * float(b) for a, b in zip(v, g)]

    def matvec(v, W):
        return [sum(v[i] * float(W[i, j]) for i in range(len(v))) for j in range(W.shape[1])]

    n1 = [rms_row(x[t], w.attn_norm) for t in range(T)]
    qkv = [matvec(n1[t], w.w_qkv) for t in range(T)]
    q = np.array([[qkv[t][h * d:(h + 1) * d] for h in range(Hq)] for t in range(T)])
    k = np.array([[qkv[t][Hq * d:Hq * d + d]] for t in range(T)])
    v = np.array([qkv[t][Hq * d + d:Hq * d + 2 * d] for t in range(T)])
    pos = np.arange(T)
    q = _rope_component_loop(q, pos, base)
    k = _rope_component_loop(k, pos, base)[:, 0, :]
    o = np.zeros((T, Hq * d))
    for t in range(T):
        for h in range(Hq):
            s = [sum(q[t, h, c] * k[j, c] for c in range(d)) / math.sqrt(d) for j in range(t + 1)]
            m = max(s)
            e = [math.exp(a - m) for a in s]
            z = sum(e)
            for c in range(d):
                o[t, h * d + c] = sum(e[j] / z * v[j, c] for j in range(t + 1))
    h_ = [[float(x[t, i]) + matvec(list(o[t]), w.w_o)[i] for i in range(D)] for t in range(T)]
    out = []
    for t in range(T):
        n2 = rms_row(h_[t], w.ffn_norm)
        gu = matvec(n2, w.w_gate_up)
        a = [0.5 * g * (1 + math.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3))) * u
             for g, u in zip(gu[:F], gu[F:])]
        dn = matvec(a, w.w_down)
        out.append([h_[t][i] + dn[i] for i in range(D)])
    return np.array(out)


def test_decoder_layer_matches_loop_restatement():
    x, w = blocks.make_decoder_layer(10, tokens=4, hidden=6, q_heads=3, head_dim=4, ffn=5)
    # larger weights so every term matters
    for name in ("w_qkv", "w_o", "w_gate_up", "w_down"):
        setattr(w, name, getattr(w, name) * 25)
    got = blocks.decoder_layer_f32(x, w, q_heads=3, head_dim=4, eps=1e-6, rope_base=10000.0)
    ref = _layer_loops(x, w, 3, 4, 1e-6, 10000.0)
    np.testing.assert_allclose(got, ref, rtol=1e-11, atol=1e-11)


def test_decoder_layer_is_causal():
    x, w = blocks.make_decoder_layer(20, tokens=6, hidden=8, q_heads=2, head_dim=4, ffn=6)
    base = blocks.decoder_layer_f32(x, w, 2, 4)
    x2 = x.copy()
    x2[4] += 1.0
    moved = blocks.decoder_layer_f32(x2, w, 2, 4)
    np.testing.assert_array_equal(base[:4], moved[:4])
    assert np.max(np.abs(base[4:] - moved[4:])) > 1e-3


# ------------------------------------------------------------------ DiT pieces
from tests.golden import octagon  # noqa: E402


def test_adaln_transform_matches_captured_witness():
    # Experiments/ZImageTurboNoiseRefiner0/M2: lanes 0,2 -> 1 + x, lanes 1,3 -> tanh(x) (width 2), 1e-7
    wit = octagon.load("adaln_selected.octagon")
    raw = wit["Raw"]
    ones = oracle.to_bf16(np.ones((1, raw.size), np.float32))
    sa, ga, sm, gm = blocks.adaln_modulation(np.array([1.0]), ones, raw - 1.0, hidden=2)
    got = np.concatenate((sa, ga, sm, gm))
    assert np.max(np.abs(got - wit["Expected"])) <= 1e-7


def test_rope_pair_matches_captured_witness():
    # Experiments/ZImageTurboNoiseRefiner0/M3: frame-33 first-axis pair 4 of width 32
    wit = octagon.load("qkv_rope_selected.octagon")
    x = np.zeros((1, 1, 128))
    x[0, 0, 8], x[0, 0, 9] = wit["QNormPair.Even"], wit["QNormPair.Odd"]
    out = blocks.rope_interleaved(x, np.array([[33.0, 0.0, 0.0]]), (32, 48, 48), 256.0)
    assert abs(out[0, 0, 8] - (-0.4407204)) <= 1e-6 and abs(out[0, 0, 9] - (-0.1587258)) <= 1e-6
    assert abs((out[0, 0, 8] ** 2 + out[0, 0, 9] ** 2) - (x[0, 0, 8] ** 2 + x[0, 0, 9] ** 2)) <= 1e-6
    # the fused QKV witness: Q, K, V of token 0 sit at offsets 0, width, 2*width
    np.testing.assert_allclose(wit["FusedToken0"], [0.11094941, 43.58648, 54.267914])


def test_joint_coordinates_kat():
    # zimage/canonical_contract_test.go:11-31: 15 text tokens -> padding 17, frame 33
    assert blocks.text_padding(15) == 17 and blocks.text_padding(128) == 0
    c = blocks.joint_coordinates(32, 32, 15)
    for token, want in ((0, (33, 0, 0)), (31, (33, 0, 31)), (32, (33, 1, 0)), (1023, (33, 31, 31))):
        np.testing.assert_array_equal(c[token], want)
    np.testing.assert_array_equal(c[1024], (1, 0, 0))
    # C5 layout: 64x64 image grid then 128 text tokens; frame 129
    c5 = blocks.joint_coordinates(64, 64, 128)
    assert c5.shape == (4224, 3) and tuple(c5[4095]) == (129, 63, 63) and tuple(c5[4223]) == (128, 0, 0)


def test_rope_interleaved_zero_coordinate_is_identity():
    x = oracle.normal(1, (3, 2, 128)).astype(np.float64)
    np.testing.assert_array_equal(blocks.rope_interleaved(x, np.zeros((3, 3))), x)


def _dit_loops(x, coords, cond, w, heads, eps, theta, axes):
    """Loop restatement following canonical_reference.go:315-480 stage by stage."""
    T, D = x.shape
    hd = D // heads
    F = w.w_2.shape[0]
    wa = oracle.from_bf16(w.w_adaln).astype(np.float64)
    m = [sum(float(cond[k]) * wa[k, j] for k in range(len(cond))) + float(w.b_adaln[j]) for j in range(4 * D)]
    sa = [1 + v for v in m[:D]]
    ga = [math.tanh(v) for v in m[D:2 * D]]
    sm = [1 + v for v in m[2 * D:3 * D]]
    gm = [math.tanh(v) for v in m[3 * D:]]

    def rms(v, g):
        s = sum(a * a for a in v)
        inv = 1 / math.sqrt(s / len(v) + eps)
        return [a * inv * float(b) for a, b in zip(v, g)]

    def lin(v, bits):
        W = oracle.from_bf16(bits).astype(np.float64)
        return list(np.array(v) @ W)

    a = [[u * s for u, s in zip(rms(list(map(float, x[t])), w.attn_norm1), sa)] for t in range(T)]
    qkv = [lin(a[t], w.w_qkv) for t in range(T)]
    q = [[rms(qkv[t][h * hd:(h + 1) * hd], w.q_norm) for h in range(heads)] for t in range(T)]
    k = [[rms(qkv[t][D + h * hd:D + (h + 1) * hd], w.k_norm) for h in range(heads)] for t in range(T)]
    v = [[qkv[t][2 * D + h * hd:2 * D + (h + 1) * hd] for h in range(heads)] for t in range(T)]
    for t in range(T):
        for h in range(heads):
            base = 0
            for axis, width in enumerate(axes):
                for p in range(width // 2):
                    ang = float(coords[t][axis]) * (1.0 / theta ** (2 * p / width))
                    cs, sn = math.cos(ang), math.sin(ang)
                    for vec in (q[t][h], k[t][h]):
                        e, o = vec[base + 2 * p], vec[base + 2 * p + 1]
                        vec[base + 2 * p], vec[base + 2 * p + 1] = e * cs - o * sn, e * sn + o * cs
                base += width
    attn = [[0.0] * D for _ in range(T)]
    for t in range(T):
        for h in range(heads):
            s = [sum(q[t][h][c] * k[j][h][c] for c in range(hd)) / math.sqrt(hd) for j in range(T)]
            mx = max(s)
            e = [math.exp(z - mx) for z in s]
            z = sum(e)
            for c in range(hd):
                attn[t][h * hd + c] = sum(e[j] / z * v[j][h][c] for j in range(T))
    out = []
    for t in range(T):
        proj = lin(attn[t], w.w_out)
        r = [float(x[t][i]) + ga[i] * n for i, n in enumerate(rms(proj, w.attn_norm2))]
        f = [u * s for u, s in zip(rms(r, w.ffn_norm1), sm)]
        g13 = lin(f, w.w_13)
        hh = [g / (1 + math.exp(-g)) * u for g, u in zip(g13[:F], g13[F:])]
        y = rms(lin(hh, w.w_2), w.ffn_norm2)
        out.append([r[i] + gm[i] * y[i] for i in range(D)])
    return np.array(out)


def test_dit_block_matches_loop_restatement():
    x, cond, w = blocks.make_dit_block(3, tokens=4, hidden=256, ffn=16, cond_dim=8)
    # larger projection weights so attention and the FFN matter
    for name in ("w_qkv", "w_out", "w_13", "w_2", "w_adaln"):
        setattr(w, name, oracle.to_bf16(oracle.from_bf16(getattr(w, name)) * 40))
    coords = np.array([[5, 0, 1], [5, 1, 0], [1, 0, 0], [2, 0, 0]], np.float32)
    got = blocks.dit_block_bf16(x, coords, cond, w, heads=2)
    ref = _dit_loops(x, coords, cond, w, 2, 1e-5, 256.0, (32, 48, 48))
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-10)
    # the row-subset evaluation is exact for the chosen rows
    np.testing.assert_allclose(blocks.dit_block_bf16(x, coords, cond, w, heads=2, rows=[1, 3]), got[[1, 3]],
                               rtol=1e-13, atol=1e-13)


def test_dit_block_permutation_equivariant():
    x, cond, w = blocks.make_dit_block(5, tokens=6, hidden=256, ffn=32, cond_dim=8)
    coords = blocks.joint_coordinates(2, 2, 2)
    base = blocks.dit_block_bf16(x, coords, cond, w, heads=2)
    perm = np.array([3, 0, 5, 1, 4, 2])
    moved = blocks.dit_block_bf16(x[perm], coords[perm], cond, w, heads=2)
    np.testing.assert_allclose(moved, base[perm], rtol=1e-12, atol=1e-12)


def closed_form_attention_layer(q_heads: int, head_dim: int, c0_over_sqrt_d: float = np.log(3.0)):
    """A T = 2 layer whose output is known in closed form (conventions of
    gemma4e2b_m1_rtx.go:863-883: scores scaled by 1/sqrt(d), every query head on
    the single K/V head).  D = q_heads * head_dim; x0 = ones, x1 = alternating
    signs (orthogonal, RMS 1), so with unit norm weights RMSNorm is the identity
    up to 1/sqrt(1 + eps).  Token 0 has k = 0, so token 1's scores are 0 (key 0)
    and c_h / sqrt(d) (key 1) with c_h = (h + 1) * c0: head h puts weight
    3^(h+1) / (3^(h+1) + 1) on token 1 when c0 / sqrt(d) = ln 3.  W_o = I and a
    zero gate|up make the layer output x + attention output."""
    d, Hq = head_dim, q_heads
    D = Hq * d
    x = np.ones((2, D))
    x[1, 1::2] = -1.0
    a = 4.0
    b = c0_over_sqrt_d * np.sqrt(d) / a
    rng = np.random.default_rng(123)
    v0, v1 = rng.uniform(-1, 1, d), rng.uniform(-1, 1, d)
    cols = np.zeros((2, (Hq + 2) * d))  # per token: wanted q | k | v values
    for h in range(Hq):
        cols[1, h * d] = (h + 1) * a          # q head h at token 1 = (h+1) a e0; token 0's q = 0
    cols[1, Hq * d] = b                        # k1 = b e0, k0 = 0
    cols[0, (Hq + 1) * d:] = v0
    cols[1, (Hq + 1) * d:] = v1
    # column j = (val0 x0 + val1 x1) / D, then stored as float32
    w_qkv = ((cols[0][None, :] * x[0][:, None] + cols[1][None, :] * x[1][:, None]) / D).astype(np.float32)
    F = 4
    w = blocks.DecoderLayerWeights(
        attn_norm=np.ones(D, np.float32), w_qkv=w_qkv, w_o=np.eye(D, dtype=np.float32),
        ffn_norm=np.ones(D, np.float32), w_gate_up=np.zeros((D, 2 * F), np.float32),
        w_down=rng.uniform(-1, 1, (F, D)).astype(np.float32))
    # what the float32 weights actually hold
    qkv = x @ w_qkv.astype(np.float64)
    return x.astype(np.float32), w, qkv


def closed_form_expected(x, qkv, q_heads, head_dim, eps):
    d, Hq = head_dim, q_heads
    s2 = 1.0 / (1.0 + eps)          # both q and k carry the RMSNorm factor 1/sqrt(1+eps)
    s1 = np.sqrt(s2)
    v0 = qkv[0, (Hq + 1) * d:] * s1
    v1 = qkv[1, (Hq + 1) * d:] * s1
    k1 = qkv[1, Hq * d]
    out = x.astype(np.float64).copy()
    for h in range(Hq):
        c = qkv[1, h * d] * k1 * s2 / np.sqrt(d)
        p1 = 1.0 / (1.0 + np.exp(-c))  # two keys: softmax = sigmoid of the score difference
        out[0, h * d:(h + 1) * d] += v0
        out[1, h * d:(h + 1) * d] += p1 * v1 + (1.0 - p1) * v0
    return out


@pytest.mark.parametrize("q_heads,head_dim", [(8, 256), (3, 4)])
def test_decoder_layer_attention_closed_form(q_heads, head_dim):
    x, w, qkv = closed_form_attention_layer(q_heads, head_dim)
    got = blocks.decoder_layer_f32(x, w, q_heads, head_dim, eps=0.0)
    want = closed_form_expected(x, qkv, q_heads, head_dim, 0.0)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
    # the hand-computed weights: head h puts 3^(h+1)/(3^(h+1)+1) on token 1
    d = head_dim
    for h in range(q_heads):
        c = qkv[1, h * d] * qkv[1, q_heads * d] / np.sqrt(d)
        assert abs(1.0 / (1.0 + np.exp(-c)) - 3.0 ** (h + 1) / (3.0 ** (h + 1) + 1.0)) < 1e-6


def test_closed_form_rejects_plausible_convention_mistakes():
    """Each mistake the closed form is meant to catch moves the output well past its tolerance."""
    Hq, d = 8, 256
    x, w, qkv = closed_form_attention_layer(Hq, d)
    want = closed_form_expected(x, qkv, Hq, d, 0.0)
    # scale 1/d instead of 1/sqrt(d)
    wrong_scale = closed_form_expected(x, qkv * np.where(np.arange(qkv.shape[1]) < Hq * d, 1.0 / np.sqrt(d), 1.0),
                                       Hq, d, 0.0)
    assert np.max(np.abs(wrong_scale - want)) > 1e-2
    # per-head K (head h reading the columns after K, i.e. V, as its key) changes heads >= 1
    x2, w2, _ = closed_form_attention_layer(Hq, d)
    got = blocks.decoder_layer_f32(x2, w2, Hq, d, eps=0.0)
    v_as_key = closed_form_expected(x, qkv, Hq, d, 0.0)
    for h in range(1, Hq):
        kv = qkv[1, (Hq + 1) * d]  # the first V component would be head 1's "key" component
        c = qkv[1, h * d] * kv / np.sqrt(d)
        p1 = 1.0 / (1.0 + np.exp(-c))
        v0, v1 = qkv[0, (Hq + 1) * d:], qkv[1, (Hq + 1) * d:]
        v_as_key[1, h * d:(h + 1) * d] = x[1, h * d:(h + 1) * d] + p1 * v1 + (1 - p1) * v0
    assert np.max(np.abs(v_as_key - got)) > 1e-2
    # a causal mask transposed (token 0 sees token 1) changes token 0
    v0, v1 = qkv[0, (Hq + 1) * d:], qkv[1, (Hq + 1) * d:]
    assert np.max(np.abs(0.5 * (v0 + v1) - (got[0, :d] - x[0, :d]))) > 1e-2
