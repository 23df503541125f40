"""Model-side callers of the hot path (Kandle's packages/model-utils): rotary tables, the static KV
cache, the Qwen3 causal LM and token sampling, built on the HIP backend's kernels."""
from .kv_cache import StaticKVCache
from .qwen3 import (GenerationStep, GeneratorConfig, LoadStateDictResult, Qwen3Config, Qwen3ForCausalLM,
                    init_qwen3_weights, qwen3_weights_from_safetensor)
from .rope import RotaryEmbedding
from .sampling import SampleResult, SamplerConfig, sample, sample_greedy

__all__ = ["StaticKVCache", "Qwen3Config", "Qwen3ForCausalLM", "init_qwen3_weights", "RotaryEmbedding",
           "LoadStateDictResult", "qwen3_weights_from_safetensor", "SamplerConfig", "SampleResult", "sample",
           "sample_greedy", "GeneratorConfig", "GenerationStep"]
