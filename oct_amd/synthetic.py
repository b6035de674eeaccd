"""Synthetic benchmark inputs (numpy PCG64), shaped like BASELINE.json's configs.

The benchmark's measured legs draw their data here; the CPU oracle (``oracle/``)
keeps its own generators and is only the checker.  Distributions:
SGEMM operands U[-1, 1]; activations N(0, 1); projection weights N(0, 0.02^2)
(N(0, 1/in) for the Z-Image layers); norm scales 1 + N(0, 0.02^2).
"""
from __future__ import annotations

import numpy as np


def uniform(seed: int, shape, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    return np.random.default_rng(seed).uniform(lo, hi, size=shape).astype(np.float32)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    return (mean + std * np.random.default_rng(seed).standard_normal(size=shape, dtype=np.float32)).astype(np.float32)


def to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (finite inputs)."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def joint_coordinates(grid_h: int, grid_w: int, text_tokens: int) -> np.ndarray:
    """Image tokens (frame = text + padding to 32 + 1, row, column) then text tokens (1..text, 0, 0)."""
    frame = text_tokens + (32 - text_tokens % 32) % 32 + 1
    img = np.arange(grid_h * grid_w)
    image = np.stack((np.full(img.shape, frame), img // grid_w, img % grid_w), axis=1)
    t = np.arange(1, text_tokens + 1)
    text = np.stack((t, np.zeros_like(t), np.zeros_like(t)), axis=1)
    return np.concatenate((image, text), axis=0).astype(np.float32)


def decoder_layer(seed: int, tokens: int, hidden: int, q_heads: int, head_dim: int, ffn: int) -> dict:
    """C4 inputs in the decoder-layer request's field names."""
    nqkv = (q_heads + 2) * head_dim
    return {"input": normal(seed, (tokens, hidden)),
            "attn_norm_weight": normal(seed + 1, (hidden,), 1.0, 0.02),
            "w_qkv": normal(seed + 2, (hidden, nqkv), 0.0, 0.02),
            "w_o": normal(seed + 3, (q_heads * head_dim, hidden), 0.0, 0.02),
            "ffn_norm_weight": normal(seed + 4, (hidden,), 1.0, 0.02),
            "w_gate_up": normal(seed + 5, (hidden, 2 * ffn), 0.0, 0.02),
            "w_down": normal(seed + 6, (ffn, hidden), 0.0, 0.02)}


def dit_block(seed: int, tokens: int, hidden: int, ffn: int, cond_dim: int, coords: np.ndarray,
              head_dim: int = 128) -> dict:
    """C5 inputs in the DiT request's field names (bf16 bits for the projections)."""
    D, F, C = hidden, ffn, cond_dim
    return {"input": normal(seed, (tokens, D)), "coordinates": coords, "condition": normal(seed + 1, (C,)),
            "w_adaln": to_bf16(normal(seed + 2, (C, 4 * D), 0.0, 0.02)),
            "b_adaln": normal(seed + 3, (4 * D,), 0.0, 0.02),
            "attn_norm1": normal(seed + 4, (D,), 1.0, 0.02), "attn_norm2": normal(seed + 5, (D,), 1.0, 0.02),
            "ffn_norm1": normal(seed + 6, (D,), 1.0, 0.02), "ffn_norm2": normal(seed + 7, (D,), 1.0, 0.02),
            "q_norm": normal(seed + 8, (head_dim,), 1.0, 0.02), "k_norm": normal(seed + 9, (head_dim,), 1.0, 0.02),
            "w_qkv": to_bf16(normal(seed + 10, (D, 3 * D), 0.0, 0.02)),
            "w_out": to_bf16(normal(seed + 11, (D, D), 0.0, 0.02)),
            "w_13": to_bf16(normal(seed + 12, (D, 2 * F), 0.0, 0.02)),
            "w_2": to_bf16(normal(seed + 13, (F, D), 0.0, 0.02))}


ZIMAGE_SHAPES = {"adaln_b": (15360,), "adaln_w": (256, 15360), "k_norm": (128,), "w_out": (3840, 3840),
                 "q_norm": (128,), "w_qkv": (3840, 11520), "attn_norm1": (3840,), "attn_norm2": (3840,),
                 "w1": (3840, 10240), "w2": (10240, 3840), "w3": (3840, 10240), "ffn_norm1": (3840,),
                 "ffn_norm2": (3840,)}


def zimage_weights(seed: int, modulated: bool = True) -> dict:
    """One Z-Image Turbo layer's FP16 tensors ([in, out] linear weights)."""
    out = {}
    for i, (name, shape) in enumerate(ZIMAGE_SHAPES.items()):
        if not modulated and name.startswith("adaln"):
            continue
        if len(shape) == 2:
            v = normal(seed * 16 + i, shape, 0.0, float(1.0 / np.sqrt(shape[0])))
        else:
            v = normal(seed * 16 + i, shape, 1.0, 0.1)
        out[name] = v.astype(np.float16)
    return out
