"""Kernel registry of a backend: a plain name -> callable map looked up at every call.

Mirrors SimpleOperatorRegistry / IBackendOpsRegister (reference: packages/utils/src/registry/index.ts:3-17;
packages/types/src/backend/register.ts:128-144).
"""
from __future__ import annotations

from typing import Callable, Dict, Optional


class SimpleOperatorRegistry:
    def __init__(self):
        self._kernels: Dict[str, Callable] = {}

    def register(self, op_name: str, kernel_func: Callable) -> None:
        self._kernels[op_name] = kernel_func

    def find(self, op_name: str) -> Optional[Callable]:
        return self._kernels.get(op_name)

    def has(self, op_name: str) -> bool:
        return op_name in self._kernels

    def names(self):
        return sorted(self._kernels)
