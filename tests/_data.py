"""Seeded synthetic inputs shared by tests and bench (numpy PCG64 streams).

N(0, sigma) weights and activations as the benchmark configs describe them;
bf16 values are produced with the oracle's bit-exact fp32 -> bf16 rounding.
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def normal(shape, sigma: float, seed: int) -> np.ndarray:
    return (rng(seed).standard_normal(shape) * sigma).astype(np.float32)


def uniform(shape, lo: float, hi: float, seed: int) -> np.ndarray:
    return rng(seed).uniform(lo, hi, shape).astype(np.float32)


def to_bf16_bits(oracle, x: np.ndarray) -> np.ndarray:
    return oracle.f32_to_bf16_n(np.ascontiguousarray(x, np.float32))


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def with_outliers(x: np.ndarray, frac: float, mag: float, seed: int) -> np.ndarray:
    """Replace a fraction of entries by +-mag at seeded positions (config 3)."""
    g = rng(seed)
    y = x.copy().ravel()
    n = max(1, int(round(frac * y.size)))
    pos = g.choice(y.size, size=n, replace=False)
    y[pos] = np.where(g.random(n) < 0.5, -mag, mag).astype(np.float32)
    return y.reshape(x.shape)


def moe_routing(tokens: int, experts: int, topk: int, seed: int) -> np.ndarray:
    """Top-k DISTINCT experts per token drawn uniformly (config 4)."""
    g = rng(seed)
    ids = np.empty((tokens, topk), np.int32)
    for t in range(tokens):
        ids[t] = g.choice(experts, size=topk, replace=False)
    return ids
