"""Rotary position embedding tables (reference: packages/model-utils/src/rope.ts:120-273).

The inverse frequencies are computed exactly as RotaryEmbedding._computeInvFreqDirect does
(rope.ts:159-171): 1 / base^(i / (dim/2)) evaluated in float64 and stored as float32.  The angles
float32(position) * inv_freq and their cos/sin are formed inside the fused qk-norm + RoPE kernel, so
no [seq, dim] cos/sin tables are materialised in HBM.
"""
from __future__ import annotations

import numpy as np

from ..tensor import Tensor


class RotaryEmbedding:
    def __init__(self, dim: int, base: float = 10000.0):
        if dim % 2:
            raise ValueError("rotary dim must be even")
        self.dim = dim
        self.base = float(base)
        half = dim // 2
        self.inv_freq_host = np.array([1.0 / (self.base ** (i / half)) for i in range(half)],
                                      dtype=np.float64).astype(np.float32)
        self.inv_freq = Tensor(self.inv_freq_host, dtype="float32")

    @staticmethod
    def get_position_ids(seq_len: int, start_pos: int = 0) -> Tensor:
        """arange(start, start + seq_len) as int32 (rope.ts:270-272)."""
        return Tensor(np.arange(start_pos, start_pos + seq_len, dtype=np.int32), dtype="int32")
