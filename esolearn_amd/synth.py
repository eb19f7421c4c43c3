"""Seeded synthetic inputs with fastrand 2.3.0's generator (wyrand), as the
reference draws them (fastrand::Rng::with_seed; tests/llama_smoke.rs:26-28).

Prompt ids are a build-defined choice: n draws of Rng::with_seed(seed).u64()
taken modulo the vocabulary size.
"""
from __future__ import annotations

import numpy as np

_M64 = (1 << 64) - 1
_W0 = 0x2D358DCCAA6C78A5
_W1 = 0x8BB84B93962EACC9


def rng_u64(seed: int, n: int) -> list[int]:
    s = seed & _M64
    out = []
    for _ in range(n):
        s = (s + _W0) & _M64
        t = s * (s ^ _W1)
        out.append((t & _M64) ^ (t >> 64))
    return out


def prompt_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    return np.array([u % vocab for u in rng_u64(seed, n)], dtype=np.int64)
