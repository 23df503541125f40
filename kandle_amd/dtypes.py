"""DTypes of the HIP backend and host-side conversions.

The reference DType set (packages/types/src/base.ts:5-25) has no bfloat16; this backend adds
'bfloat16' as a first-class storage dtype (16 high bits of a float32, round to nearest even) and
keeps 'float32' and 'int32'.  Host data for a bfloat16 tensor is accepted as float32 values (rounded
here) or as raw uint16 bit patterns; readback widens exactly, as the reference's safetensors loader
widens BF16 (packages/core/src/io/safetensor/dtypes.ts:82-94).
"""
from __future__ import annotations

import numpy as np

from ._lib import KH_BF16, KH_F32, KH_I32

FLOAT32 = "float32"
BFLOAT16 = "bfloat16"
INT32 = "int32"

DTYPES = (FLOAT32, BFLOAT16, INT32)
ITEMSIZE = {FLOAT32: 4, BFLOAT16: 2, INT32: 4}
KH_CODE = {FLOAT32: KH_F32, BFLOAT16: KH_BF16, INT32: KH_I32}
STORAGE_NP = {FLOAT32: np.float32, BFLOAT16: np.uint16, INT32: np.int32}


def check_dtype(dtype: str) -> str:
    if dtype not in DTYPES:
        raise ValueError(f"unsupported dtype {dtype!r}: the HIP backend stores {DTYPES}")
    return dtype


def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even, NaN kept quiet.

    Works through the array in cache-sized chunks with in-place integer ops (the weights of a
    0.6B-parameter model convert in about a second)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    flat = a.reshape(-1)
    out = np.empty(flat.size, np.uint16)
    chunk = 1 << 22
    for s in range(0, flat.size, chunk):
        u = flat[s:s + chunk].view(np.uint32)
        t = u >> np.uint32(16)
        t &= np.uint32(1)
        t += u
        t += np.uint32(0x7FFF)
        t >>= np.uint32(16)
        out[s:s + chunk] = t
        nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
        if nan.any():
            out[s:s + chunk][nan] = (u[nan] >> np.uint32(16)) | np.uint32(0x40)
    return out.reshape(a.shape)


def bf16_bits_to_f32(b) -> np.ndarray:
    """Exact widening of bf16 bit patterns to float32."""
    u = np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return u.view(np.float32)


def to_storage_array(data, dtype: str) -> np.ndarray:
    """Host data -> contiguous array of the storage element type of `dtype`."""
    a = np.asarray(data)
    if dtype == BFLOAT16:
        if a.dtype == np.uint16:
            return np.ascontiguousarray(a)
        return f32_to_bf16_bits(a.astype(np.float32, copy=False))
    return np.ascontiguousarray(a, dtype=STORAGE_NP[dtype])


def from_storage_array(raw: np.ndarray, dtype: str) -> np.ndarray:
    """Storage array -> logical host values (bf16 widened to float32)."""
    if dtype == BFLOAT16:
        return bf16_bits_to_f32(raw)
    return raw
