"""Synthetic symbol distributions that reach particular decoder paths."""
from __future__ import annotations

import numpy as np


def many_escape_windows(seed: int, n: int) -> np.ndarray:
    """16 common symbols and 240 rare ones (p = 1.2e-4 each). The rare
    symbols get 13-bit codes, two per 12-bit prefix, so the decode table has
    about 112 windows whose first codeword is longer than 12 bits: more
    escape blocks than a workgroup keeps in LDS (64)."""
    rng = np.random.default_rng(seed)
    p_rare = 1.2e-4
    p = np.concatenate([np.full(16, (1 - 240 * p_rare) / 16), np.full(240, p_rare)])
    return rng.choice(256, size=n, p=p).astype(np.int64)
