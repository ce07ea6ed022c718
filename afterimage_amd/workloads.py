"""Seeded synthetic BF16 weights for the decode workloads.

Values come from numpy's PCG64 ``default_rng(seed)`` as float32 and are
rounded to bf16 by torch's round-to-nearest-even conversion. Shapes are those
of a Qwen3 MLP / 14B-class decoder block; no real checkpoint is involved.
"""
from __future__ import annotations

import numpy as np
import torch

from .runtime.compressed_store import CompressedLayer, compress_group, compress_layer


def bf16_normal(shape, seed: int, scale: float = 0.02, outlier_frac: float = 0.0,
                outlier_scale: float = 0.5, center: float = 0.0) -> torch.Tensor:
    """bf16 tensor of N(center, scale); a fraction ``outlier_frac`` of entries
    (chosen by the same generator) are replaced by N(0, outlier_scale)."""
    rng = np.random.default_rng(seed)
    n = int(np.prod(shape))
    w = rng.standard_normal(n, dtype=np.float32)
    w *= np.float32(scale)
    if center:
        w += np.float32(center)
    if outlier_frac:
        mask = rng.random(n) < outlier_frac
        k = int(mask.sum())
        w[mask] = rng.standard_normal(k, dtype=np.float32) * np.float32(outlier_scale)
    return torch.from_numpy(w).to(torch.bfloat16).reshape(shape)


# One dense decoder block of a 14B-class model (Qwen3-14B shapes), [out, in].
BLOCK_14B = (
    ("q_proj", (5120, 5120), "attn_qo"),
    ("k_proj", (1024, 5120), "attn_kv"),
    ("v_proj", (1024, 5120), "attn_kv"),
    ("o_proj", (5120, 5120), "attn_qo"),
    ("gate_proj", (17408, 5120), "mlp_in"),
    ("up_proj", (17408, 5120), "mlp_in"),
    ("down_proj", (5120, 17408), "mlp_out"),
    ("input_layernorm", (5120,), "norm"),
    ("post_attention_layernorm", (5120,), "norm"),
)


def single_layer(seed: int = 2, rows: int = 5120, cols: int = 17408,
                 chunk_size: int = 65536) -> tuple[torch.Tensor, CompressedLayer]:
    """The 5120x17408 MLP weight with 0.1% N(0, 0.5) outliers, one codebook."""
    w = bf16_normal((rows, cols), seed, 0.02, outlier_frac=1e-3)
    return w, compress_layer(w, chunk_size=chunk_size)


def small_layer(seed: int = 1, rows: int = 1024, cols: int = 3072,
                chunk_size: int = 4096) -> tuple[torch.Tensor, CompressedLayer]:
    """The 1024x3072 MLP up-projection of a 0.6B model, N(0, 0.02)."""
    w = bf16_normal((rows, cols), seed, 0.02)
    return w, compress_layer(w, chunk_size=chunk_size)


def block_14b(seed: int = 3, chunk_size: int = 65536, scale: float = 1.0
              ) -> list[tuple[str, torch.Tensor, CompressedLayer]]:
    """One 14B-class decoder block: weights N(0, 0.02), RMSNorm weights
    N(1.0, 0.05), tensor i seeded with seed * 100 + i. Tensors of one role
    share one codebook built from their pooled exponent histogram. ``scale``
    < 1 shrinks every row count (for quick checks); 1.0 is the real block."""
    weights = []
    for i, (name, shape, role) in enumerate(BLOCK_14B):
        if scale != 1.0:
            shape = (max(1, int(round(shape[0] * scale))),) + tuple(shape[1:])
        if role == "norm":
            w = bf16_normal(shape, seed * 100 + i, 0.05, center=1.0)
        else:
            w = bf16_normal(shape, seed * 100 + i, 0.02)
        weights.append((name, w, role))
    layers: dict[str, CompressedLayer] = {}
    for role in dict.fromkeys(r for _, _, r in weights):
        group = [(name, w) for name, w, r in weights if r == role]
        for (name, _), layer in zip(group, compress_group([w for _, w in group],
                                                          chunk_size=chunk_size)):
            layers[name] = layer
    return [(name, w, layers[name]) for name, w, _ in weights]

