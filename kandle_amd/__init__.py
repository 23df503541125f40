"""kandle_amd — MI355X (gfx950) backend for Kandle's transformer hot path.

Host side: a Python mirror of Kandle's backend plugin interface (HipBackend, kernel registry,
tensor handles, dispatch functions).  Device side: hand-written HIP kernels behind the C ABI in
include/kandle_hip.h (libkandle_hip.so, built by `python -m kandle_amd.build`).

    from kandle_amd import HipBackend, Tensor, functional as F
    HipBackend.create()
    q = Tensor(np_q, dtype="bfloat16"); ...
    o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
"""
from . import env, functional
from ._lib import KandleHipError
from .memory import is_in_tidy_scope, keep, tidy
from .backend import HipBackend, register_hip_kernels
from .registry import SimpleOperatorRegistry
from .tensor import HipStorage, HipTensorHandle, Tensor

__all__ = [
    "env",
    "functional",
    "HipBackend",
    "HipStorage",
    "HipTensorHandle",
    "KandleHipError",
    "SimpleOperatorRegistry",
    "Tensor",
    "register_hip_kernels",
    "tidy",
    "keep",
    "is_in_tidy_scope",
]
