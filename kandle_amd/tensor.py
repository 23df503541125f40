"""Device storage, tensor handles and the user-level Tensor of the HIP backend.

Mirrors the reference contract:
  * HipStorage ~ WebGPUStorage: device bytes with a reference count; views incRef, dispose decRefs,
    the last decRef returns the block to the caching allocator; incRef after free is an error
    (reference: packages/backend-webgpu/src/base/storage.ts:60-245, :114-117).
  * HipTensorHandle ~ ITensorHandle / WebGPUTensor: shape, dtype, element strides and element offset
    over a shared storage; dataAsync returns the logical contiguous data
    (reference: packages/types/src/tensor.ts:6-55; packages/backend-webgpu/src/base/tensor.ts:55-202).
  * Tensor ~ core Tensor: a thin user object over a handle with data_async / dispose
    (reference: packages/core/src/tensor.ts:8-414).
Python's garbage collector is the safety net that the reference gets from FinalizationRegistry.
"""
from __future__ import annotations

import ctypes as C
import itertools
from typing import Optional, Sequence

import numpy as np

from . import _lib
from .dtypes import ITEMSIZE, KH_CODE, STORAGE_NP, check_dtype, from_storage_array, to_storage_array

_ids = itertools.count(1)


def contiguous_strides(shape: Sequence[int]) -> list:
    strides, acc = [], 1
    for s in reversed(list(shape)):
        strides.append(acc)
        acc *= max(int(s), 1)
    return list(reversed(strides))


def numel_of(shape: Sequence[int]) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


class HipStorage:
    """Reference-counted device allocation from the library's caching allocator."""

    def __init__(self, nbytes: int):
        _lib.init_check()
        self.nbytes = int(nbytes)
        self.id = next(_ids)
        self.ptr = _lib.alloc(max(self.nbytes, 1))
        self._refs = 1

    @property
    def ref_count(self) -> int:
        return self._refs

    @property
    def is_freed(self) -> bool:
        return self._refs <= 0

    def inc_ref(self) -> None:
        if self._refs <= 0:
            raise RuntimeError(f"storage {self.id}: incRef after the storage was freed")
        self._refs += 1

    def dec_ref(self) -> None:
        if self._refs <= 0:
            return
        self._refs -= 1
        if self._refs == 0:
            _lib.free(self.ptr)
            self.ptr = 0

    def upload(self, host: np.ndarray, byte_offset: int = 0) -> None:
        h = np.ascontiguousarray(host)
        if byte_offset + h.nbytes > self.nbytes:
            raise ValueError("upload exceeds storage size")
        _lib.call("kh_memcpy_h2d", C.c_void_p(self.ptr + byte_offset), C.c_void_p(h.ctypes.data), h.nbytes)

    def download(self, nbytes: int, byte_offset: int = 0) -> bytes:
        buf = np.empty(nbytes, np.uint8)
        _lib.call("kh_memcpy_d2h", C.c_void_p(buf.ctypes.data), C.c_void_p(self.ptr + byte_offset), nbytes)
        return buf


def check_extent(storage: "HipStorage", shape, strides, offset: int, dtype: str, what: str = "view") -> None:
    """Refuse a view whose element offsets (offset + sum of index * stride over `shape`) leave its
    storage: every kernel addresses device memory from these numbers."""
    if int(offset) != offset or offset < 0:
        raise ValueError(f"{what}: offset {offset} is not a non-negative integer")
    if len(strides) != len(shape):
        raise ValueError(f"{what}: {len(strides)} strides for a {len(shape)}-d shape")
    lo = hi = int(offset)
    for n, st in zip(shape, strides):
        if n < 0:
            raise ValueError(f"{what}: negative extent {n}")
        if n == 0:
            return
        span = (int(n) - 1) * int(st)
        if span < 0:
            lo += span
        else:
            hi += span
    capacity = storage.nbytes // ITEMSIZE[dtype]
    if lo < 0 or hi >= capacity:
        raise ValueError(f"{what}: reaches elements [{lo}, {hi}] of a storage holding {capacity}")


class HipTensorHandle:
    """Shape / dtype / element strides / element offset over a HipStorage."""

    device = "hip"

    def __init__(self, storage: HipStorage, shape, dtype: str, strides=None, offset: int = 0):
        self.storage = storage
        self.shape = tuple(int(s) for s in shape)
        self.dtype = check_dtype(dtype)
        self.strides = tuple(int(s) for s in (strides if strides is not None else contiguous_strides(self.shape)))
        self.offset = int(offset)
        check_extent(storage, self.shape, self.strides, self.offset, self.dtype)
        self.id = next(_ids)
        self._disposed = False

    # -- construction ---------------------------------------------------------------------------
    @classmethod
    def create_new(cls, shape, dtype: str, data=None) -> "HipTensorHandle":
        check_dtype(dtype)
        n = numel_of(shape)
        storage = HipStorage(n * ITEMSIZE[dtype])
        h = cls(storage, shape, dtype)
        if data is not None:
            arr = to_storage_array(data, dtype).reshape(-1)
            if arr.size != n:
                raise ValueError(f"data has {arr.size} elements, shape {tuple(shape)} needs {n}")
            storage.upload(arr)
        return h

    @classmethod
    def create_view(cls, storage: HipStorage, shape, dtype: str, strides, offset: int) -> "HipTensorHandle":
        storage.inc_ref()
        return cls(storage, shape, dtype, strides, offset)

    # -- properties ---------------------------------------------------------------------------
    @property
    def numel(self) -> int:
        return numel_of(self.shape)

    @property
    def itemsize(self) -> int:
        return ITEMSIZE[self.dtype]

    @property
    def kh_dtype(self) -> int:
        return KH_CODE[self.dtype]

    @property
    def is_disposed(self) -> bool:
        return self._disposed

    @property
    def storage_id(self) -> int:
        return self.storage.id

    def data_ptr(self) -> int:
        """Device address of element 0 of this view (storage base + offset)."""
        if self._disposed or self.storage.is_freed:
            raise RuntimeError(f"tensor {self.id} used after dispose")
        return self.storage.ptr + self.offset * self.itemsize

    def is_contiguous(self) -> bool:
        expected = contiguous_strides(self.shape)
        return all(sz == 1 or st == ex for sz, st, ex in zip(self.shape, self.strides, expected))

    # -- data -----------------------------------------------------------------------------------
    def data_async(self) -> np.ndarray:
        """Logical contiguous host copy (bf16 widened to float32); waits for the device."""
        n = self.numel
        if n == 0:
            return np.zeros(self.shape, STORAGE_NP[self.dtype] if self.dtype != "bfloat16" else np.float32)
        if self.is_contiguous():
            raw = self.storage.download(n * self.itemsize, self.offset * self.itemsize)
            arr = raw.view(STORAGE_NP[self.dtype]).reshape(self.shape)
            return from_storage_array(arr, self.dtype).reshape(self.shape)
        tmp = HipTensorHandle.create_new(self.shape, self.dtype)
        try:
            copy_into(self, tmp)
            return tmp.data_async()
        finally:
            tmp.dispose()

    def raw_bits(self) -> np.ndarray:
        """Storage-typed host copy (bf16 as uint16 bit patterns)."""
        if not self.is_contiguous():
            tmp = HipTensorHandle.create_new(self.shape, self.dtype)
            try:
                copy_into(self, tmp)
                return tmp.raw_bits()
            finally:
                tmp.dispose()
        raw = self.storage.download(self.numel * self.itemsize, self.offset * self.itemsize)
        return raw.view(STORAGE_NP[self.dtype]).reshape(self.shape).copy()

    def dispose(self) -> None:
        if not self._disposed:
            self._disposed = True
            self.storage.dec_ref()

    def __del__(self):
        try:
            if not self._disposed and _lib.is_initialized():
                self.dispose()
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"HipTensorHandle(id={self.id}, shape={self.shape}, dtype={self.dtype}, strides={self.strides}, offset={self.offset})"


def copy_into(src: HipTensorHandle, dst: HipTensorHandle) -> None:
    """dst (contiguous) <- src (any strided view), casting float32 <-> bfloat16 as needed."""
    if src.shape != dst.shape:
        raise ValueError(f"copy shape mismatch {src.shape} vs {dst.shape}")
    if not dst.is_contiguous():
        raise ValueError("copy destination must be contiguous")
    shape, strides = _coalesce(src.shape, src.strides)
    if len(shape) > 6:
        raise ValueError(f"strided copy supports up to 6 non-mergeable dims, got {len(shape)}")
    _lib.call(
        "kh_copy_strided",
        C.c_void_p(src.storage.ptr),
        src.offset,
        C.c_void_p(dst.data_ptr()),
        len(shape),
        _lib.i64_array(shape),
        _lib.i64_array(strides),
        src.kh_dtype,
        dst.kh_dtype,
    )


def _coalesce(shape, strides):
    """Drop size-1 dims and merge dims that are contiguous with their inner neighbour."""
    dims = [(s, st) for s, st in zip(shape, strides) if s != 1]
    if not dims:
        return [1], [1]
    out = [list(dims[-1])]
    for s, st in reversed(dims[:-1]):
        inner_s, inner_st = out[0]
        if st == inner_s * inner_st:
            out[0] = [s * inner_s, inner_st]
        else:
            out.insert(0, [s, st])
    return [d[0] for d in out], [d[1] for d in out]


class Tensor:
    """User-level tensor over a HipTensorHandle (reference: packages/core/src/tensor.ts)."""

    def __init__(self, data=None, *, dtype: str = "float32", shape=None, handle: Optional[HipTensorHandle] = None):
        if handle is None:
            from .env import get_backend

            arr = None if data is None else np.asarray(data)
            if shape is None:
                if arr is None:
                    raise ValueError("Tensor needs data or a shape")
                shape = arr.shape
            handle = get_backend("hip").create_tensor_handle(shape, dtype, arr)
        self.handle = handle
        from .memory import _track

        _track(self)

    @property
    def shape(self):
        return self.handle.shape

    @property
    def dtype(self) -> str:
        return self.handle.dtype

    @property
    def strides(self):
        return self.handle.strides

    @property
    def offset(self) -> int:
        return self.handle.offset

    @property
    def device(self) -> str:
        return self.handle.device

    @property
    def numel(self) -> int:
        return self.handle.numel

    def data_async(self) -> np.ndarray:
        return self.handle.data_async()

    def numpy(self) -> np.ndarray:
        return self.handle.data_async()

    def dispose(self) -> None:
        self.handle.dispose()

    @property
    def is_disposed(self) -> bool:
        return self.handle.is_disposed

    def __repr__(self) -> str:
        return f"Tensor(shape={self.shape}, dtype={self.dtype}, device=hip)"
