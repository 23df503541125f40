"""HipBackend: the MI355X plugin behind Kandle's backend interface.

Mirrors IBackend (reference: packages/types/src/backend/index.ts:33-55) and the way
WebGPUBackend.create() initialises the device, registers its kernels by name and is installed with
env.setBackend / env.setDefaultDevice (packages/backend-webgpu/src/index.ts:15-87;
packages/core/src/env.ts:8-30).
"""
from __future__ import annotations

from typing import Optional

from . import _lib, env
from .dtypes import check_dtype
from .kernels import KERNELS
from .registry import SimpleOperatorRegistry
from .tensor import HipStorage, HipTensorHandle


class HipBackend:
    name = "hip"

    def __init__(self):
        self.operators = SimpleOperatorRegistry()
        register_hip_kernels(self.operators)

    def create_tensor_handle(self, shape=None, dtype: Optional[str] = None, data=None, *, storage: HipStorage = None,
                             strides=None, offset: int = 0, options: dict = None) -> HipTensorHandle:
        """Allocate a new tensor (shape, dtype[, data]) or build a view sharing `storage`.

        Accepts both the options form ({shape, dtype, storage?, data?, strides?, offset?}) and the
        positional (shape, dtype, data) form of the reference's createTensorHandle."""
        if options is not None:
            shape = options.get("shape", shape)
            dtype = options.get("dtype", dtype)
            data = options.get("data", data)
            storage = options.get("storage", storage)
            strides = options.get("strides", strides)
            offset = options.get("offset", offset)
        check_dtype(dtype)
        if storage is not None:
            if data is not None:
                raise ValueError("create_tensor_handle: data cannot be given with a shared storage")
            return HipTensorHandle.create_view(storage, shape, dtype,
                                               strides if strides is not None else None, offset)
        return HipTensorHandle.create_new(shape, dtype, data)

    @classmethod
    def create(cls, device: int = 0, make_default: bool = True) -> "HipBackend":
        """Initialise the HIP device and stream, register kernels, install as the 'hip' backend."""
        _lib.load()
        _lib.init(device)
        backend = cls()
        env.set_backend(backend)
        if make_default:
            env.set_default_device(cls.name)
        return backend

    # -- observability (mirrors the reference storage statistics) --------------------------------
    @staticmethod
    def memory_stats() -> dict:
        return _lib.alloc_stats()

    @staticmethod
    def synchronize() -> None:
        _lib.synchronize()


def register_hip_kernels(registry: SimpleOperatorRegistry) -> None:
    """Register every HIP kernel under the reference kernel names (plus the new fused names)."""
    for name, fn in KERNELS.items():
        registry.register(name, fn)
