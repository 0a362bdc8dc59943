"""Deterministic input generators shared by the golden-vector script and tests.

``fill_random`` is the linear congruential generator the reference's model
tests use for their inputs (tools/test_model.c:29-39): state = state*1664525 +
1013904223 (mod 2^32), value = (state >> 8) / 2^23 - 1, in [-1, 1).  Fixtures
store the seed and shape of every input drawn from it, plus an input checksum,
so the inputs are rebuilt bit for bit instead of being committed.
"""
from __future__ import annotations

import numpy as np


def fill_random(n: int, seed: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    state = seed & 0xFFFFFFFF
    inv = np.float32(1.0 / (1 << 23))
    one = np.float32(1.0)
    sc = np.float32(scale)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        # (float)(state >> 8) / (float)(1u << 23) - 1.0f, then * scale, in fp32
        out[i] = (np.float32(state >> 8) * inv - one) * sc
    return out


def normal(n: int, seed: int) -> np.ndarray:
    """N(0,1) fp32 from numpy's PCG64 (bench / large-shape tests)."""
    return np.random.default_rng(seed).standard_normal(n, dtype=np.float32)


def checksum(a: np.ndarray) -> int:
    """Order-dependent 64-bit checksum of an array's bytes."""
    b = np.frombuffer(np.ascontiguousarray(a).tobytes(), dtype=np.uint8).astype(np.uint64)
    w = (np.arange(b.size, dtype=np.uint64) % np.uint64(251)) + np.uint64(1)
    return int((b * w).sum() & np.uint64(0xFFFFFFFFFFFF))
