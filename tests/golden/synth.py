"""Deterministic synthetic data for fixtures and tests.

counter_uniform(seed, n) is a counter-based SplitMix64 stream mapped to
float32 in [-1, 1) using 24 random bits, so every value is exactly
representable and the stream is reproducible bit-for-bit from (seed, index)
with integer arithmetic alone — the golden fixtures store the seed, not the
pool contents.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64_at(seed: int, idx: np.ndarray) -> np.ndarray:
    """z_i = SplitMix64 output for state seed + (i+1)*golden (wrapping uint64)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + (idx.astype(np.uint64) + np.uint64(1)) * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def counter_uniform(seed: int, n: int) -> np.ndarray:
    z = splitmix64_at(seed, np.arange(n, dtype=np.uint64))
    return ((z >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -23)
            - np.float32(1.0)).astype(np.float32)


def counter_pool(seed: int, pages: int, layers: int, kv_dim: int) -> np.ndarray:
    n = pages * layers * 16 * kv_dim
    return counter_uniform(seed, n).reshape(pages, layers, 16, kv_dim)


def rope_tables(seq_len: int, head_dim: int, base: float = 10000.0):
    """Llama-style RoPE tables: angle(pos, i) = pos * base^(-2i/head_dim), i < head_dim/2,
    evaluated in float64 and rounded to float32 (real = cos, imag = sin)."""
    i = np.arange(head_dim // 2, dtype=np.float64)
    theta = base ** (-2.0 * i / head_dim)
    ang = np.arange(seq_len, dtype=np.float64)[:, None] * theta[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
