"""Backend registry and default device (reference: packages/core/src/env.ts:3-44)."""
from __future__ import annotations

_backends = {}
_default_device = None


def set_backend(backend) -> None:
    _backends[backend.name] = backend


def get_backend(device: str = None):
    name = device or _default_device
    if name is None or name not in _backends:
        raise RuntimeError(f"no backend registered for device {name!r}; call HipBackend.create() first")
    return _backends[name]


def set_default_device(device: str) -> None:
    global _default_device
    if device not in _backends:
        raise RuntimeError(f"backend {device!r} is not registered")
    _default_device = device


def get_default_device() -> str:
    return _default_device
