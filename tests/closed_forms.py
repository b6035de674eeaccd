"""Closed-form cases of the transformer blocks: inputs for which every stage
is known from a few numbers, so the expected output is computed without any
matrix product, attention or reshaping.

Construction (shared by the CPU pinning tests and the GPU parity tests):

* Every activation is periodic in the channel index with period 4: channel j
  holds the value of its class j % 4.  A stage is therefore a 4-vector, and
  RMSNorm over a row of width D (a multiple of 4) is RMSNorm over the four
  class values, ``g * u / sqrt(mean(u^2) + eps)``.
* Weights are scaled selections that keep each channel's class: W_v selects
  channel j, W_out channel j + 4 (mod D), gate/up (W1 / W3) send hidden unit
  i to channel i % D, and down (W2) sends hidden unit j < D to channel j
  (F >= D; hidden units past D have zero rows).  The class values of the
  vectors (input, adaLN chunks, norm weights) all differ, so a misplaced
  scale or norm changes the shape of a stage, not only its size, and
  RMSNorm cannot hide it.
* All tokens are identical, so every token's V row is the same and
  attention returns it exactly, since the softmax weights of a query sum to
  one whatever W_q, W_k, the q/k norms, RoPE and the causal mask make of the
  scores (random W_q and W_k keep the scores uneven).

The stage recurrences restate the reference definitions:
  RMSNorm (no mean, no 1 + w)      canonical_contract.go:91-105
  adaLN 1 + scale, tanh(gate)      canonical_reference.go:366-383
  x + gateA * RMSNorm(proj)        canonical_reference.go:433-441 (canonicalAddGate :201-210)
  RMSNorm(r) * scaleM              canonical_reference.go:442-451
  silu(w1) * w3                    canonical_reference.go:456-464
  r + gateM * RMSNorm(w2)          canonical_reference.go:470-476
  ContextRefiner: no adaLN, plain residual adds (context_refiner_reference.go:230-311)
  Gemma layer: pre-norm attention and GeGLU FFN (the request definition in
  include/prometheus_reactor.h; tanh-approximate GELU).
"""
from __future__ import annotations

import numpy as np

import oracle
from oracle import blocks

# Class values, all exact in BF16 and FP16.  They were picked (from a seeded
# search over multiples of 1/8) so that every misreading listed in
# tests/test_oracle_closed_forms.py moves the block output by more than 0.2
# normwise, ten times the bf16 parity bar, with no scale (1 + m) or gate
# (m) smaller than 1/4 in magnitude.
X = np.array([-0.75, -1.5, 0.625, -1.75])
BETA = {  # adaLN chunk values per class: scaleA, gateA, scaleM, gateM (pre-activation)
    "scale_a": np.array([-0.625, 1.75, -0.375, -1.375]),
    "gate_a": np.array([1.625, 0.5, -1.0, 0.875]),
    "scale_m": np.array([1.5, -1.375, 0.875, -0.625]),
    "gate_m": np.array([-0.875, -1.25, 1.25, -0.375]),
}
GAMMA = {  # norm weights per class
    "attn_norm1": np.array([1.625, 0.5, 2.0, 2.75]),
    "attn_norm2": np.array([2.0, 1.125, 2.375, 1.875]),
    "ffn_norm1": np.array([1.75, 0.875, 1.25, 0.625]),
    "ffn_norm2": np.array([2.375, 1.625, 2.5, 2.0]),
}
S_V, S_O, S_1, S_3, S_2 = 0.5, 0.625, 0.75, -2.375, 0.5


def nu(u, g, eps):
    """RMSNorm of a row whose channels repeat the four class values ``u``."""
    return g * u / np.sqrt(np.mean(u * u) + eps)


def silu(v):
    return v / (1.0 + np.exp(-v))


def block_classes(modulated: bool, eps: float) -> np.ndarray:
    """The Z-Image / DiT block on the class values (attention output = V)."""
    if modulated:
        scale_a, gate_a = 1.0 + BETA["scale_a"], np.tanh(BETA["gate_a"])
        scale_m, gate_m = 1.0 + BETA["scale_m"], np.tanh(BETA["gate_m"])
    else:
        scale_a = gate_a = scale_m = gate_m = np.ones(4)
    a = nu(X, GAMMA["attn_norm1"], eps) * scale_a
    o = S_V * a
    proj = S_O * o
    r = X + gate_a * nu(proj, GAMMA["attn_norm2"], eps)
    f = nu(r, GAMMA["ffn_norm1"], eps) * scale_m
    hidden = silu(S_1 * f) * (S_3 * f)
    return r + gate_m * nu(S_2 * hidden, GAMMA["ffn_norm2"], eps)


def tile(classes: np.ndarray, width: int) -> np.ndarray:
    return np.tile(classes, width // 4)


def _selections(D: int, F: int):
    assert D % 4 == 0 and F >= D
    w_v = S_V * np.eye(D)
    w_out = S_O * np.roll(np.eye(D), 4, axis=0)  # column j reads channel (j + 4) % D
    sel = np.zeros((D, F))
    sel[np.arange(F) % D, np.arange(F)] = 1.0     # hidden i <- channel i % D
    w2 = np.zeros((F, D))
    w2[np.arange(D), np.arange(D)] = S_2          # channel j <- hidden j
    return w_v, w_out, S_1 * sel, S_3 * sel, w2


def dit_case(tokens: int, heads: int, ffn: int, cond_dim: int, head_dim: int = 128, seed: int = 0,
             coordinate=(33.0, 5.0, 7.0)):
    """Inputs of the bf16 DiT block (oracle.blocks.dit_block_bf16 conventions)."""
    D, F = heads * head_dim, ffn
    rng = np.random.default_rng(seed)
    w_v, w_out, w1, w3, w2 = _selections(D, F)
    w_qk = rng.uniform(-0.05, 0.05, (D, 2 * D))
    w = blocks.DitBlockWeights(
        w_adaln=oracle.to_bf16(np.zeros((cond_dim, 4 * D), np.float32)),
        b_adaln=np.concatenate([tile(BETA[k], D) for k in ("scale_a", "gate_a", "scale_m", "gate_m")]),
        attn_norm1=tile(GAMMA["attn_norm1"], D).astype(np.float32),
        attn_norm2=tile(GAMMA["attn_norm2"], D).astype(np.float32),
        ffn_norm1=tile(GAMMA["ffn_norm1"], D).astype(np.float32),
        ffn_norm2=tile(GAMMA["ffn_norm2"], D).astype(np.float32),
        q_norm=(1.0 + rng.uniform(-0.1, 0.1, head_dim)).astype(np.float32),
        k_norm=(1.0 + rng.uniform(-0.1, 0.1, head_dim)).astype(np.float32),
        w_qkv=oracle.to_bf16(np.concatenate((w_qk, w_v), axis=1).astype(np.float32)),
        w_out=oracle.to_bf16(w_out.astype(np.float32)),
        w_13=oracle.to_bf16(np.concatenate((w1, w3), axis=1).astype(np.float32)),
        w_2=oracle.to_bf16(w2.astype(np.float32)))
    x = np.tile(tile(X, D), (tokens, 1)).astype(np.float32)
    coords = np.tile(np.asarray(coordinate, np.float32), (tokens, 1))
    cond = rng.standard_normal(cond_dim).astype(np.float32)
    return x, coords, cond, w


def dit_expected(tokens: int, width: int, eps: float = 1e-5) -> np.ndarray:
    return np.tile(tile(block_classes(True, eps), width), (tokens, 1))


def zimage_case(modulated: bool, width: int = 3840, ffn: int = 10240, cond_dim: int = 256, seed: int = 0):
    """FP16 weights of a resident Z-Image block (oracle.blocks.zimage_block_f64
    conventions, cache-manifest names)."""
    D, F = width, ffn
    w_v, w_out, w1, w3, w2 = _selections(D, F)
    w_qkv = np.empty((D, 3 * D))
    w_qkv[:, :2 * D] = np.random.default_rng(seed).uniform(-0.05, 0.05, (D, 2 * D))
    w_qkv[:, 2 * D:] = w_v
    h16 = lambda a: np.asarray(a, np.float32).astype(np.float16)
    w = {"k_norm": h16(np.full(128, 0.75)), "q_norm": h16(np.full(128, 1.25)), "w_qkv": h16(w_qkv),
         "w_out": h16(w_out), "w1": h16(w1), "w2": h16(w2), "w3": h16(w3)}
    for name in ("attn_norm1", "attn_norm2", "ffn_norm1", "ffn_norm2"):
        w[name] = h16(tile(GAMMA[name], D))
    if modulated:
        w["adaln_w"] = h16(np.zeros((cond_dim, 4 * D)))
        w["adaln_b"] = h16(np.concatenate([tile(BETA[k], D) for k in ("scale_a", "gate_a", "scale_m", "gate_m")]))
    return {k: w[k] for k in (blocks.ZIMAGE_TENSORS if modulated else blocks.CONTEXT_TENSORS)}


def zimage_expected(tokens: int, modulated: bool, width: int = 3840, eps: float = 1e-5) -> np.ndarray:
    return np.tile(tile(block_classes(modulated, eps), width), (tokens, 1))


# --------------------------------------------------------------- Gemma layer
GEMMA_GAMMA = {"attn_norm": np.array([1.25, 0.5, 1.5, 0.75]), "ffn_norm": np.array([0.5, 1.75, 1.0, 1.25])}
G_A, G_B, G_V, G_O, G_D = 1.5, -1.25, 2.0, 0.75, 0.5


def gelu_tanh(v):
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


def decoder_classes(eps: float) -> np.ndarray:
    """Gemma layer on the class values: attention returns V (identical tokens),
    every query head carries the one K/V head's V."""
    n1 = nu(X, GEMMA_GAMMA["attn_norm"], eps)
    h = X + G_O * (G_V * n1)
    n2 = nu(h, GEMMA_GAMMA["ffn_norm"], eps)
    return h + G_D * gelu_tanh(G_A * n2) * (G_B * n2)


def decoder_case(tokens: int, hidden: int, q_heads: int, head_dim: int, ffn: int, seed: int = 0):
    """Inputs of the fp32 Gemma layer: the V head selects channels 0..d-1, W_o
    is a scaled identity over the q_heads * head_dim = hidden attention
    channels, gate and up are scaled selections of channel i % D, down sends
    hidden unit j < D to channel j."""
    D, d, F = hidden, head_dim, ffn
    assert q_heads * d == D and D % 4 == 0 and d % 4 == 0 and F >= D
    rng = np.random.default_rng(seed)
    w_qkv = np.zeros((D, (q_heads + 2) * d))
    w_qkv[:, :(q_heads + 1) * d] = rng.uniform(-0.05, 0.05, (D, (q_heads + 1) * d))
    w_qkv[np.arange(d), (q_heads + 1) * d + np.arange(d)] = G_V
    sel = np.zeros((D, F))
    sel[np.arange(F) % D, np.arange(F)] = 1.0
    w_down = np.zeros((F, D))
    w_down[np.arange(D), np.arange(D)] = G_D
    w = blocks.DecoderLayerWeights(
        attn_norm=tile(GEMMA_GAMMA["attn_norm"], D).astype(np.float32), w_qkv=w_qkv.astype(np.float32),
        w_o=(G_O * np.eye(D)).astype(np.float32), ffn_norm=tile(GEMMA_GAMMA["ffn_norm"], D).astype(np.float32),
        w_gate_up=np.concatenate((G_A * sel, G_B * sel), axis=1).astype(np.float32),
        w_down=w_down.astype(np.float32))
    x = np.tile(tile(X, D), (tokens, 1)).astype(np.float32)
    return x, w


def decoder_expected(tokens: int, hidden: int, eps: float = 1e-6) -> np.ndarray:
    return np.tile(tile(decoder_classes(eps), hidden), (tokens, 1))
