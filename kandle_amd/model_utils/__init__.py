"""Model-side callers of the hot path (Kandle's packages/model-utils): rotary tables, the static KV
cache and the Qwen3 causal LM, built on the HIP backend's kernels."""
from .kv_cache import StaticKVCache
from .qwen3 import (LoadStateDictResult, Qwen3Config, Qwen3ForCausalLM, init_qwen3_weights,
                    qwen3_weights_from_safetensor)
from .rope import RotaryEmbedding

__all__ = ["StaticKVCache", "Qwen3Config", "Qwen3ForCausalLM", "init_qwen3_weights", "RotaryEmbedding",
           "LoadStateDictResult", "qwen3_weights_from_safetensor"]
