"""Seeded synthetic inputs shared bit-exactly by the GPU run and its CPU check.

Values come from numpy's Philox4x32-10 bit generator (Salmon et al., SC'11) with a caller-chosen
seed, so the same (seed, shape) gives the same float32 values on every host; bf16 inputs are those
values rounded to nearest even.
"""
from __future__ import annotations

import numpy as np

from .dtypes import bf16_bits_to_f32, f32_to_bf16_bits


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.Philox(seed))


def normal(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """float32 N(0, std^2) samples."""
    x = rng(seed).standard_normal(size=shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    return x


def uniform(seed: int, shape, low: float, high: float) -> np.ndarray:
    return rng(seed).uniform(low, high, size=shape).astype(np.float32)


def bf16(x: np.ndarray) -> np.ndarray:
    """(bits uint16, values float32) of x rounded to bf16."""
    bits = f32_to_bf16_bits(x)
    return bits, bf16_bits_to_f32(bits).reshape(x.shape)


def randint(seed: int, shape, low: int, high: int) -> np.ndarray:
    return rng(seed).integers(low, high, size=shape, dtype=np.int64).astype(np.int32)
