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


def assert_close_elem(a, b, rtol=1e-4, atol=1e-5, what=""):
    """Element-wise |a - b| <= rtol * |b| + atol (atol: the floor for elements near zero, where an
    fp32 sum's absolute error dominates), reporting the worst element."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    excess = np.abs(a - b) - (rtol * np.abs(b) + atol)
    i = int(np.argmax(excess))
    assert excess.flat[i] <= 0, (f"{what}: element {np.unravel_index(i, b.shape)} differs by "
                                 f"{abs(a.flat[i] - b.flat[i]):.3e} (value {b.flat[i]:.4e}; "
                                 f"bound {rtol * abs(b.flat[i]) + atol:.3e})")
