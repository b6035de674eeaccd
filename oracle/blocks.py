"""Binary64 numpy oracles for the transformer blocks ([4]).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Each step cites the
reference definition it restates.  The reference has no Gemma-2B layer (its
Gemma-4-E2B pieces fix the conventions) and its Z-Image block is fixed at
1024/1056 tokens; these oracles take the shapes as parameters.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """y = x / sqrt(mean(x^2) + eps) * w, no mean subtraction.

    reactor_vulkan_gemma4e2b.c:286-319; zimage/canonical_contract.go:91-105."""
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(w, dtype=np.float64)


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """Tanh-approximate GELU (Gemma's GeGLU activation; the reference has no implementation of it)."""
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def silu(x: np.ndarray) -> np.ndarray:
    """zimage/canonical_reference.go:459: x / (1 + exp(-x))."""
    return x / (1.0 + np.exp(-x))


def softmax_rows(s: np.ndarray) -> np.ndarray:
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / np.sum(e, axis=-1, keepdims=True)


# ------------------------------------------------------------- Gemma layer
@dataclass
class DecoderLayerWeights:
    attn_norm: np.ndarray  # [D]
    w_qkv: np.ndarray      # [D, (Hq+2)*d]
    w_o: np.ndarray        # [Hq*d, D]
    ffn_norm: np.ndarray   # [D]
    w_gate_up: np.ndarray  # [D, 2F]
    w_down: np.ndarray     # [F, D]


def rope_half_split(x: np.ndarray, positions: np.ndarray, base: float) -> np.ndarray:
    """Half-split pairing of gemma4e2b_m1_rtx.go:834-861 (component c pairs with
    c +- d/2; out = x*cos - mate*sin below d/2, x*cos + mate*sin above), without
    the BF16 storage rounding; angle = position * base^(-2i/d).  x: [T, H, d]."""
    d = x.shape[-1]
    half = d // 2
    inv = base ** (-2.0 * np.arange(half, dtype=np.float64) / d)
    ang = positions.astype(np.float64)[:, None] * inv[None, :]
    c = np.cos(ang)[:, None, :]
    s = np.sin(ang)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate((x1 * c - x2 * s, x2 * c + x1 * s), axis=-1)


def decoder_layer_f32(x: np.ndarray, w: DecoderLayerWeights, q_heads: int, head_dim: int, eps: float = 1e-6,
                      rope_base: float = 10000.0, position_offset: int = 0) -> np.ndarray:
    """Gemma-style decoder layer in binary64 (multi-query attention)."""
    x = np.asarray(x, dtype=np.float64)
    T, D = x.shape
    Hq, d = q_heads, head_dim
    F = w.w_down.shape[0]
    n1 = rmsnorm(x, w.attn_norm, eps)
    qkv = n1 @ w.w_qkv.astype(np.float64)
    q = qkv[:, :Hq * d].reshape(T, Hq, d)
    k = qkv[:, Hq * d:Hq * d + d].reshape(T, 1, d)
    v = qkv[:, Hq * d + d:Hq * d + 2 * d]
    pos = position_offset + np.arange(T)
    q = rope_half_split(q, pos, rope_base)
    k = rope_half_split(k, pos, rope_base)[:, 0, :]
    # every query head on KV head 0, scale 1/sqrt(d) (gemma4e2b_m1_rtx.go:863-883)
    scores = np.einsum("thd,sd->hts", q, k) / np.sqrt(d)
    causal = np.arange(T)[None, :] > np.arange(T)[:, None]
    scores = np.where(causal[None, :, :], -np.inf, scores)
    p = softmax_rows(scores)
    o = np.einsum("hts,sd->thd", p, v).reshape(T, Hq * d)
    h = x + o @ w.w_o.astype(np.float64)
    n2 = rmsnorm(h, w.ffn_norm, eps)
    gu = n2 @ w.w_gate_up.astype(np.float64)
    a = gelu_tanh(gu[:, :F]) * gu[:, F:]
    return h + a @ w.w_down.astype(np.float64)


def make_decoder_layer(seed: int, tokens: int, hidden: int, q_heads: int, head_dim: int, ffn: int):
    """Synthetic C4 inputs: x ~ N(0,1), projection weights ~ N(0,0.02), norm
    weights 1 + N(0,0.02) (RMSNorm scale multiplies, reactor_vulkan_gemma4e2b.c:313)."""
    import oracle

    nqkv = (q_heads + 2) * head_dim
    x = oracle.normal(seed, (tokens, hidden))
    w = DecoderLayerWeights(
        attn_norm=oracle.normal(seed + 1, (hidden,), 1.0, 0.02),
        w_qkv=oracle.normal(seed + 2, (hidden, nqkv), 0.0, 0.02),
        w_o=oracle.normal(seed + 3, (q_heads * head_dim, hidden), 0.0, 0.02),
        ffn_norm=oracle.normal(seed + 4, (hidden,), 1.0, 0.02),
        w_gate_up=oracle.normal(seed + 5, (hidden, 2 * ffn), 0.0, 0.02),
        w_down=oracle.normal(seed + 6, (ffn, hidden), 0.0, 0.02),
    )
    return x, w


# ---------------------------------------------------------------- DiT block
@dataclass
class DitBlockWeights:
    w_adaln: np.ndarray    # bf16 bits [C, 4D]
    b_adaln: np.ndarray    # f32 [4D]
    attn_norm1: np.ndarray
    attn_norm2: np.ndarray
    ffn_norm1: np.ndarray
    ffn_norm2: np.ndarray  # f32 [D] each
    q_norm: np.ndarray
    k_norm: np.ndarray     # f32 [head_dim]
    w_qkv: np.ndarray      # bf16 bits [D, 3D]
    w_out: np.ndarray      # bf16 bits [D, D]
    w_13: np.ndarray       # bf16 bits [D, 2F] (w1 | w3)
    w_2: np.ndarray        # bf16 bits [F, D]


def text_padding(raw_text_tokens: int) -> int:
    """zimage/canonical_contract.go:38-44: (-raw) % 32."""
    return (32 - raw_text_tokens % 32) % 32


def joint_coordinates(grid_h: int, grid_w: int, text_tokens: int) -> np.ndarray:
    """Image tokens first (frame = text + padding + 1, row-major grid), then text
    tokens at (1..text, 0, 0): zimage_main_transformer_canonical.py:146-155 and
    canonical_contract.go:46-65, generalised from a 32x32 grid to grid_h x grid_w."""
    frame = text_tokens + text_padding(text_tokens) + 1
    img = np.arange(grid_h * grid_w)
    image = np.stack((np.full(img.shape, frame, dtype=np.float64), img // grid_w, img % grid_w), axis=1)
    ctx = np.arange(1, text_tokens + 1, dtype=np.float64)
    text = np.stack((ctx, np.zeros_like(ctx), np.zeros_like(ctx)), axis=1)
    return np.concatenate((image, text), axis=0).astype(np.float32)


def rope_interleaved(x: np.ndarray, coords: np.ndarray, axes=(32, 48, 48), theta: float = 256.0) -> np.ndarray:
    """3-axis interleaved-pair RoPE (canonical_contract.go:66-87;
    zimage_main_transformer_canonical.py:124-140).  x: [T, H, hd]."""
    out = np.array(x, dtype=np.float64, copy=True)
    start = 0
    for axis, width in enumerate(axes):
        pairs = np.arange(width // 2, dtype=np.float64)
        freq = 1.0 / np.power(theta, 2.0 * pairs / width)
        ang = coords[:, axis:axis + 1].astype(np.float64) * freq[None, :]
        c = np.cos(ang)[:, None, :]
        s = np.sin(ang)[:, None, :]
        even = out[:, :, start:start + width:2].copy()
        odd = out[:, :, start + 1:start + width:2].copy()
        out[:, :, start:start + width:2] = even * c - odd * s
        out[:, :, start + 1:start + width:2] = even * s + odd * c
        start += width
    return out


def adaln_modulation(condition: np.ndarray, w_adaln_bits: np.ndarray, b_adaln: np.ndarray, hidden: int):
    """canonical_reference.go:363-383: four chunks; scale lanes 1 + m, gate lanes tanh(m)."""
    import oracle

    m = np.asarray(condition, np.float64) @ oracle.from_bf16(w_adaln_bits).astype(np.float64) + b_adaln
    chunks = [m[i * hidden:(i + 1) * hidden] for i in range(4)]
    return 1.0 + chunks[0], np.tanh(chunks[1]), 1.0 + chunks[2], np.tanh(chunks[3])


def dit_block_bf16(x, coords, condition, w: DitBlockWeights, heads: int, eps: float = 1e-5, theta: float = 256.0,
                   axes=(32, 48, 48), rows=None) -> np.ndarray:
    """The DiT block in binary64 on the bf16 weights (widened exactly).  When
    ``rows`` is given only those output tokens are evaluated (K and V still
    use every token), which is exact for those rows."""
    import oracle

    wf = lambda bits: oracle.from_bf16(bits).astype(np.float64)
    x = np.asarray(x, np.float64)
    T, D = x.shape
    hd = D // heads
    F = w.w_2.shape[0]
    scale_a, gate_a, scale_m, gate_m = adaln_modulation(condition, w.w_adaln, w.b_adaln, D)
    a = rmsnorm(x, w.attn_norm1, eps) * scale_a
    w_qkv = wf(w.w_qkv)
    sel = np.arange(T) if rows is None else np.asarray(rows)
    q = (a[sel] @ w_qkv[:, :D]).reshape(len(sel), heads, hd)
    k = (a @ w_qkv[:, D:2 * D]).reshape(T, heads, hd)
    v = (a @ w_qkv[:, 2 * D:]).reshape(T, heads, hd)
    q = rmsnorm(q, w.q_norm, eps)
    k = rmsnorm(k, w.k_norm, eps)
    q = rope_interleaved(q, coords[sel], axes, theta)
    k = rope_interleaved(k, coords, axes, theta)
    o = np.empty((len(sel), heads, hd))
    for h in range(heads):
        s = (q[:, h, :] @ k[:, h, :].T) / np.sqrt(hd)
        o[:, h, :] = softmax_rows(s) @ v[:, h, :]
    proj = o.reshape(len(sel), D) @ wf(w.w_out)
    r = x[sel] + gate_a * rmsnorm(proj, w.attn_norm2, eps)
    f = rmsnorm(r, w.ffn_norm1, eps) * scale_m
    w13 = wf(w.w_13)
    hdn = silu(f @ w13[:, :F]) * (f @ w13[:, F:])
    return r + gate_m * rmsnorm(hdn @ wf(w.w_2), w.ffn_norm2, eps)


def make_dit_block(seed: int, tokens: int, hidden: int, ffn: int, cond_dim: int = 256, head_dim: int = 128):
    """Synthetic C5 inputs: x ~ N(0,1) (fp32), condition ~ N(0,1), projection
    weights ~ N(0,0.02) rounded to bf16, adaLN bias ~ N(0,0.02), norm scales 1 + N(0,0.02)."""
    import oracle

    D, F, C = hidden, ffn, cond_dim
    x = oracle.normal(seed, (tokens, D))
    cond = oracle.normal(seed + 1, (C,))
    w = DitBlockWeights(
        w_adaln=oracle.to_bf16(oracle.normal(seed + 2, (C, 4 * D), 0.0, 0.02)),
        b_adaln=oracle.normal(seed + 3, (4 * D,), 0.0, 0.02),
        attn_norm1=oracle.normal(seed + 4, (D,), 1.0, 0.02),
        attn_norm2=oracle.normal(seed + 5, (D,), 1.0, 0.02),
        ffn_norm1=oracle.normal(seed + 6, (D,), 1.0, 0.02),
        ffn_norm2=oracle.normal(seed + 7, (D,), 1.0, 0.02),
        q_norm=oracle.normal(seed + 8, (head_dim,), 1.0, 0.02),
        k_norm=oracle.normal(seed + 9, (head_dim,), 1.0, 0.02),
        w_qkv=oracle.to_bf16(oracle.normal(seed + 10, (D, 3 * D), 0.0, 0.02)),
        w_out=oracle.to_bf16(oracle.normal(seed + 11, (D, D), 0.0, 0.02)),
        w_13=oracle.to_bf16(oracle.normal(seed + 12, (D, 2 * F), 0.0, 0.02)),
        w_2=oracle.to_bf16(oracle.normal(seed + 13, (F, D), 0.0, 0.02)),
    )
    return x, cond, w


# ------------------------------------------------- resident Z-Image blocks (fp32 path)
# Lexical cache-manifest order of one NoiseRefiner / MainTransformer layer
# (reactor_vulkan_model_block.c:158-161); the ContextRefiner omits the two
# adaLN tensors (:198-200).  Every tensor is FP16, linear weights [in, out].
ZIMAGE_TENSORS = ("adaln_b", "adaln_w", "k_norm", "w_out", "q_norm", "w_qkv", "attn_norm1", "attn_norm2",
                  "w1", "w2", "w3", "ffn_norm1", "ffn_norm2")
CONTEXT_TENSORS = ZIMAGE_TENSORS[2:]


def zimage_weight_shapes(width: int = 3840, ffn: int = 10240, cond: int = 256, head: int = 128) -> dict:
    return {"adaln_b": (4 * width,), "adaln_w": (cond, 4 * width), "k_norm": (head,), "w_out": (width, width),
            "q_norm": (head,), "w_qkv": (width, 3 * width), "attn_norm1": (width,), "attn_norm2": (width,),
            "w1": (width, ffn), "w2": (ffn, width), "w3": (width, ffn), "ffn_norm1": (width,),
            "ffn_norm2": (width,)}


def make_zimage_weights(seed: int, modulated: bool = True, width: int = 3840, ffn: int = 10240) -> dict:
    """Random FP16 weights of one layer: linear weights ~ N(0, 1/in), norm
    weights ~ 1 + N(0, 0.1^2), adaLN bias ~ N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in zimage_weight_shapes(width, ffn).items():
        if not modulated and name.startswith("adaln"):
            continue
        if len(shape) == 2:
            v = rng.standard_normal(shape, dtype=np.float32) * np.float32(1.0 / np.sqrt(shape[0]))
        elif name == "adaln_b":
            v = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.1)
        else:
            v = 1.0 + rng.standard_normal(shape, dtype=np.float32) * np.float32(0.1)
        out[name] = v.astype(np.float16)
    return out


def image_coordinates(tokens: int = 1024) -> np.ndarray:
    """NoiseRefiner token t: (frame 33, t // 32, t % 32) -- CanonicalImageTokenCoordinate(15, t),
    canonical_contract.go:36-64 (15 text tokens, 17 padding, +1)."""
    t = np.arange(tokens)
    return np.stack((np.full(tokens, 15 + text_padding(15) + 1), t // 32, t % 32), axis=1).astype(np.float32)


def context_coordinates(tokens: int = 32) -> np.ndarray:
    """ContextRefiner token t: (t + 1, 0, 0) -- context_refiner_reference.go:156-158."""
    t = np.arange(1, tokens + 1)
    return np.stack((t, np.zeros(tokens), np.zeros(tokens)), axis=1).astype(np.float32)


def rope_canonical_f32(x: np.ndarray, coords: np.ndarray, axes=(32, 48, 48), theta: float = 256.0) -> np.ndarray:
    """CanonicalRopeRotate (canonical_contract.go:66-87): frequency and angle are
    float32 values (freq = float32(1 / theta^(2p/w)), angle = float32(coord * freq)),
    cos/sin evaluated in binary64 on that angle; the rotation itself in binary64."""
    out = np.array(x, dtype=np.float64, copy=True)
    start = 0
    for axis, width in enumerate(axes):
        pairs = np.arange(width // 2, dtype=np.float64)
        freq = (1.0 / np.power(float(theta), 2.0 * pairs / width)).astype(np.float32)
        ang = (coords[:, axis:axis + 1].astype(np.float32) * freq[None, :]).astype(np.float64)
        c = np.cos(ang)[:, None, :]
        s = np.sin(ang)[:, None, :]
        even = out[:, :, start:start + width:2].copy()
        odd = out[:, :, start + 1:start + width:2].copy()
        out[:, :, start:start + width:2] = even * c - odd * s
        out[:, :, start + 1:start + width:2] = even * s + odd * c
        start += width
    return out


def zimage_block_f64(x, coords, w: dict, cond=None, heads: int = 30, eps: float = 1e-5, rows=None,
                     stages: dict | None = None) -> np.ndarray:
    """One Z-Image block in binary64 on FP16 weights widened exactly: the
    NoiseRefiner / MainTransformer (canonical_reference.go:358-480, with adaLN
    from ``cond``) or, with ``cond`` None, the unmodulated ContextRefiner
    (context_refiner_reference.go:230-311).  ``rows`` restricts the evaluated
    output tokens (K and V still use every token); ``stages`` (a dict) receives
    the canonical intermediate stages for those rows."""
    f = lambda name: np.asarray(w[name], dtype=np.float64)
    x = np.asarray(x, np.float64)
    T, D = x.shape
    hd = D // heads
    F = w["w2"].shape[0]
    sel = np.arange(T) if rows is None else np.asarray(rows)
    keep = stages if stages is not None else {}
    if cond is not None:
        raw = np.asarray(cond, np.float64) @ f("adaln_w") + f("adaln_b")
        keep["adaln_projection"] = raw
        scale_a, gate_a = 1.0 + raw[:D], np.tanh(raw[D:2 * D])
        scale_m, gate_m = 1.0 + raw[2 * D:3 * D], np.tanh(raw[3 * D:])
    else:
        scale_a = gate_a = scale_m = gate_m = np.ones(D)
    normed = rmsnorm(x, f("attn_norm1"), eps)
    keep["attention_norm"] = normed[sel]
    a = normed * scale_a
    keep["attention_modulated"] = a[sel]
    w_qkv = f("w_qkv")
    qkv = a @ w_qkv
    keep["qkv"] = qkv[sel]
    q = qkv[sel, :D].reshape(len(sel), heads, hd)
    k = qkv[:, D:2 * D].reshape(T, heads, hd)
    v = qkv[:, 2 * D:].reshape(T, heads, hd)
    q = rmsnorm(q, f("q_norm"), eps)
    k = rmsnorm(k, f("k_norm"), eps)
    keep["q_norm"] = q.reshape(len(sel), D)
    keep["k_norm"] = k[sel].reshape(len(sel), D)
    q = rope_canonical_f32(q, coords[sel])
    k = rope_canonical_f32(k, coords)
    keep["q_rope"] = q.reshape(len(sel), D)
    keep["k_rope"] = k[sel].reshape(len(sel), D)
    if stages is not None:  # every token's rotated key and value, for attention witnesses
        keep["k_rope_all"] = k.reshape(T, D)
        keep["v_all"] = v.reshape(T, D)
    o = np.empty((len(sel), heads, hd))
    for h in range(heads):
        s = (q[:, h, :] @ k[:, h, :].T) / np.sqrt(hd)
        o[:, h, :] = softmax_rows(s) @ v[:, h, :]
    o = o.reshape(len(sel), D)
    keep["attention_aggregation"] = o
    proj = o @ f("w_out")
    keep["attention_projection"] = proj
    r = x[sel] + gate_a * rmsnorm(proj, f("attn_norm2"), eps)
    keep["attention_residual"] = r
    fn = rmsnorm(r, f("ffn_norm1"), eps)
    keep["ffn_norm"] = fn
    fm = fn * scale_m
    keep["ffn_modulated"] = fm
    w1 = fm @ f("w1")
    w3 = fm @ f("w3")
    keep["w1"], keep["w3"] = w1, w3
    hdn = silu(w1) * w3
    keep["ffn_gated_hidden"] = hdn
    w2 = hdn @ f("w2")
    keep["w2"] = w2
    out = r + gate_m * rmsnorm(w2, f("ffn_norm2"), eps)
    keep["final_output"] = out
    return out
