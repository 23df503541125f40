"""Shared helpers for the GPU parity tests (not collected by pytest)."""
import numpy as np

from kandle_amd import Tensor
from kandle_amd import synthetic as syn


def dev(x, dtype="float32"):
    """Upload a float32 array (rounded to bf16 when dtype is bfloat16) as a HIP tensor."""
    return Tensor(np.asarray(x), dtype=dtype)


def seeded(seed, shape, dtype="float32", std=1.0):
    """(device tensor, host float32 values exactly as stored) for a seeded N(0, std^2) input."""
    x = syn.normal(seed, shape, std)
    if dtype == "bfloat16":
        bits, vals = syn.bf16(x)
        return Tensor(bits, dtype="bfloat16"), vals
    return Tensor(x, dtype="float32"), x


def max_rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))
