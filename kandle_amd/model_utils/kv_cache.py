"""Static KV cache (reference: packages/model-utils/src/kv-cache.ts:92-309).

Per layer, keys and values are preallocated as [batch, num_kv_heads, max_seq_len, head_dim].  New
rows are written at [start, end) -- here directly by the fused qk-norm + RoPE kernel, which writes
K (rotated) and V (copied) into the cache slice in the same launch -- and attention reads the
[:, :, :end, :] slice in place (update returns strided views, kv-cache.ts:197-211).  rollback only
moves the seen-token counter; later writes overwrite (kv-cache.ts:264-274).
"""
from __future__ import annotations

from typing import List, Tuple

from .. import functional as F
from ..tensor import Tensor


class StaticKVCache:
    def __init__(self, num_layers: int, batch: int, num_kv_heads: int, max_seq_len: int, head_dim: int,
                 dtype: str = "bfloat16"):
        self.num_layers = num_layers
        self.batch = batch
        self.num_kv_heads = num_kv_heads
        self.max_seq_len = max_seq_len
        self.head_dim = head_dim
        self.key_cache: List[Tensor] = []
        self.value_cache: List[Tensor] = []
        for _ in range(num_layers):
            self.key_cache.append(F.zeros((batch, num_kv_heads, max_seq_len, head_dim), dtype))
            self.value_cache.append(F.zeros((batch, num_kv_heads, max_seq_len, head_dim), dtype))
        self.seen_tokens = 0

    def check_write(self, start_pos: int, new_len: int) -> int:
        """Validate a write of new_len rows at start_pos (kv-cache.ts:169-174); return the end."""
        end = start_pos + new_len
        if end > self.max_seq_len:
            raise ValueError(f"Cache overflow: trying to write to position {start_pos}-{end}, "
                             f"but maxSeqLen is {self.max_seq_len}")
        return end

    def write_slices(self, layer: int, start_pos: int, new_len: int) -> Tuple[Tensor, Tensor]:
        """[:, :, start:start+new_len, :] views of layer `layer` (the fused kernel's destinations)."""
        self.check_write(start_pos, new_len)
        return (F.narrow(self.key_cache[layer], 2, start_pos, new_len),
                F.narrow(self.value_cache[layer], 2, start_pos, new_len))

    def valid_slices(self, layer: int, end: int) -> Tuple[Tensor, Tensor]:
        """[:, :, :end, :] views (what attention reads)."""
        return F.narrow(self.key_cache[layer], 2, 0, end), F.narrow(self.value_cache[layer], 2, 0, end)

    def mark_written(self, end: int) -> None:
        if end > self.seen_tokens:
            self.seen_tokens = end

    def rollback(self, position: int) -> None:
        if position < 0 or position > self.seen_tokens:
            raise ValueError(f"rollback to {position} outside [0, {self.seen_tokens}]")
        self.seen_tokens = position

    def reset(self) -> None:
        self.seen_tokens = 0

    def dispose(self) -> None:
        for t in self.key_cache + self.value_cache:
            t.dispose()
        self.key_cache, self.value_cache = [], []
