"""Qwen3 causal LM on the HIP backend (reference: packages/model-utils/src/qwen3/{model,decoder_layer,
for_causal_lm}.ts, attention/gqa.ts, mlp/swiglu.ts).

Data flow per decoder layer (pre-norm, decoder_layer.ts:191-241), batch 1, S new tokens at cache
position p:
  h   = rms_norm(x, input_layernorm)                          [S, hidden]          (rms_norm)
  qkv = h W_qkv^T                                              [S, (Hq+2Hkv) D]    (matmul; q/k/v rows
        concatenated -- each output element is the same dot product as the separate projections)
  q, k -> per-head RMSNorm + RoPE, q written heads-first, k written into the KV cache at [p, p+S),
        v copied into the V cache in the same launch                                (rms_norm_rope)
  o   = SDPA(q, K[:, :, :p+S], V[:, :, :p+S], causal = S > 1)  written as [S, Hq D] (flash_attention;
        the caller turns causal off for 1-token decode, gqa.ts:333-336; GQA is native, no repeat_kv)
  x   = x + o W_o^T                                            (matmul, residual in the epilogue)
  h   = rms_norm(x, post_attention_layernorm)
  a   = silu(h W_gate^T) * (h W_up^T)                          [S, I] (linear_swiglu: one GEMM over
        the gate/up weight interleaved in blocks of 8 rows, silu*mul in its epilogue)
  x   = x + a W_down^T                                          (matmul + residual)
then x = rms_norm(x, norm) and logits = x[last] E^T in fp32 with the tied embedding E
(for_causal_lm.ts:121-125, 184-185); greedy = argmax, lowest index among maxima (:475-508).
The residual stream x is float32 (embedding rows widened on gather; the o_proj and down GEMMs add
into it in their fp32 epilogue).  The other activations (h, q/k/v, the K/V cache, attention
output, the SwiGLU product) are stored between kernels in the model's activation dtype:
  "float32" (default): every activation in fp32, as the reference computes (its bf16 checkpoints
      are widened to float32 on load, io/safetensor/dtypes.ts:17-31, and every op runs in f32);
      the weights stay bf16 in HBM and the MFMA GEMMs take each fp32 activation as a bf16 hi + lo
      pair (kh_gemm_ex), the decode GEMVs multiply in fp32, attention runs in fp32;
  "bfloat16": rounded to bf16 at each store (half the activation bytes, the fastest path).
Math inside kernels is fp32 either way.
"""
from __future__ import annotations

import time
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from .. import env
from .. import functional as F
from .. import synthetic as syn
from .._lib import KandleHipError
from ..kernels import gemm_split_count
from ..graphs import HipGraph
from ..kernels import TensorIterator, interleave_gate_up
from ..tensor import HipTensorHandle, Tensor
from .kv_cache import StaticKVCache
from .rope import RotaryEmbedding


@dataclass
class Qwen3Config:
    """Qwen3-0.6B architecture (reference defaults: qwen3/model.ts:45-84, 183-197;
    playground-node/src/qwen3/utils.ts:19-33)."""

    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_position_embeddings: int = 40960
    tie_word_embeddings: bool = True

    @classmethod
    def from_dict(cls, d: dict) -> "Qwen3Config":
        """From a Hugging Face config.json mapping (unknown keys ignored; head_dim defaults to
        hidden_size / num_attention_heads as in the transformers Qwen3 config)."""
        kw = {f: d[f] for f in cls.__dataclass_fields__ if f in d and d[f] is not None}
        if "head_dim" not in kw and "hidden_size" in kw and "num_attention_heads" in kw:
            kw["head_dim"] = kw["hidden_size"] // kw["num_attention_heads"]
        return cls(**kw)

    @classmethod
    def from_json_file(cls, path: str) -> "Qwen3Config":
        import json

        with open(path, "r", encoding="utf-8") as fh:
            return cls.from_dict(json.load(fh))


def weight_names(cfg: Qwen3Config) -> List[str]:
    names = ["model.embed_tokens.weight"]
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        names += [p + "input_layernorm.weight", p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight",
                  p + "self_attn.v_proj.weight", p + "self_attn.o_proj.weight", p + "self_attn.q_norm.weight",
                  p + "self_attn.k_norm.weight", p + "post_attention_layernorm.weight", p + "mlp.gate_proj.weight",
                  p + "mlp.up_proj.weight", p + "mlp.down_proj.weight"]
    names.append("model.norm.weight")
    return names


def weight_shape(cfg: Qwen3Config, name: str):
    H, I, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    q, kv = cfg.num_attention_heads * D, cfg.num_key_value_heads * D
    table = {"embed_tokens": (cfg.vocab_size, H), "input_layernorm": (H,), "post_attention_layernorm": (H,),
             "q_proj": (q, H), "k_proj": (kv, H), "v_proj": (kv, H), "o_proj": (H, q), "q_norm": (D,),
             "k_norm": (D,), "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I), "norm": (H,)}
    key = name.split(".")[-2]
    return table[key]


def init_qwen3_weights(cfg: Qwen3Config, seed: int = 0, std: float = 0.02) -> Dict[str, np.ndarray]:
    """Random-init weights as bf16 bit patterns (uint16): projections and the embedding ~ N(0, std^2)
    from a seeded Philox stream per tensor; RMSNorm weights = 1 (the usual initialisation, which keeps
    activations O(1) through 28 layers)."""
    out = {}
    for idx, name in enumerate(weight_names(cfg)):
        shape = weight_shape(cfg, name)
        if name.endswith("norm.weight"):
            out[name] = np.full(shape, 0x3F80, np.uint16)  # 1.0 in bf16
        else:
            out[name] = syn.bf16(syn.normal(seed * 100003 + idx, shape, std))[0]
    return out


@dataclass
class LoadStateDictResult:
    """Outcome of loading a checkpoint (reference: nn/module.ts LoadStateDictResult)."""

    loaded_keys: List[str]
    missing_keys: List[str]
    unexpected_keys: List[str]


def qwen3_weights_from_safetensor(group, cfg: Qwen3Config, strict: bool = True, key_mapper=None):
    """(weights, result): the model's tensors from a safetensors group as bf16 bit patterns (uint16
    arrays; BF16 layers are views of the file's memory map, F32/F16 layers are rounded to nearest
    even), keyed by the Hugging Face names of weight_names(cfg), plus "lm_head.weight" for an untied
    head.  Follows Module.loadFromSafetensor (nn/module.ts:572-660): key_mapper maps checkpoint names
    to model names; strict raises on missing or unexpected keys, with the same message."""
    from ..io.safetensors import host_array

    key_mapper = key_mapper or (lambda k: k)
    expected = weight_names(cfg)
    if not cfg.tie_word_embeddings:
        expected = expected + ["lm_head.weight"]
    expected_set = set(expected)
    tied_extra = {"lm_head.weight"} if cfg.tie_word_embeddings else set()   # a tied head may be stored too
    by_model_key = {}
    unexpected = []
    for name in group.layers:
        mk = key_mapper(name)
        if mk in expected_set:
            by_model_key.setdefault(mk, name)
        elif mk not in tied_extra:
            unexpected.append(name)
    weights, loaded, missing = {}, [], []
    for key in expected:
        name = by_model_key.get(key)
        if name is None:
            missing.append(key)
            continue
        layer = group.get_layer(name)
        want = tuple(weight_shape(cfg, key)) if key != "lm_head.weight" else (cfg.vocab_size, cfg.hidden_size)
        if tuple(layer.shape) != want:
            raise ValueError(f"{name}: checkpoint shape {list(layer.shape)} does not match the model's {list(want)}")
        weights[key] = host_array(layer, "bfloat16")
        loaded.append(key)
    if strict and (missing or unexpected):
        raise ValueError("Error(s) in loading state_dict:\n"
                         f"  Missing keys: [{', '.join(missing)}]\n"
                         f"  Unexpected keys: [{', '.join(unexpected)}]")
    return weights, LoadStateDictResult(loaded, missing, unexpected)


ACTIVATION_DTYPES = ("float32", "bfloat16")


class Qwen3ForCausalLM:
    def __init__(self, cfg: Qwen3Config, weights: Dict[str, np.ndarray], max_seq_len: int = 1024,
                 activations: str = "float32", f32_attention: str = "split"):
        """activations: "float32" (the reference's f32 arithmetic over bf16 weights) or "bfloat16"
        (activations and KV caches rounded to bf16).  f32_attention (float32 mode): "split" runs the
        prefill attention as three bf16 MFMAs per product on hi/lo operands (flash_attention_split,
        within about 2^-15 of the fp32 products), "fp32" on the fp32 MFMA (flash_attention)."""
        if activations not in ACTIVATION_DTYPES:
            raise ValueError(f"activations must be one of {ACTIVATION_DTYPES}, not {activations!r}")
        if f32_attention not in ("split", "fp32"):
            raise ValueError(f"f32_attention must be 'split' or 'fp32', not {f32_attention!r}")
        self.cfg = cfg
        self.max_seq_len = max_seq_len
        self.act = activations
        self._flash_name = "flash_attention_split" if (activations == "float32" and f32_attention == "split") \
            else "flash_attention"
        self.ops = env.get_backend("hip").operators
        up = lambda a: Tensor(a, dtype="bfloat16")  # noqa: E731  (uint16 bits -> bf16 tensor)
        self.embed = up(weights["model.embed_tokens.weight"])
        # Tied embeddings (for_causal_lm.ts:121-125): the lm_head is the embedding matrix itself.
        untied = not cfg.tie_word_embeddings and "lm_head.weight" in weights
        self.lm_head = up(weights["lm_head.weight"]) if untied else self.embed
        self.final_norm = up(weights["model.norm.weight"])
        self.layers = []
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            w = lambda n: weights[p + n]  # noqa: E731
            self.layers.append({
                "in_norm": up(w("input_layernorm.weight")),
                "w_qkv": up(np.concatenate([w("self_attn.q_proj.weight"), w("self_attn.k_proj.weight"),
                                            w("self_attn.v_proj.weight")], axis=0)),
                "q_norm": up(w("self_attn.q_norm.weight")),
                "k_norm": up(w("self_attn.k_norm.weight")),
                "w_o": up(w("self_attn.o_proj.weight")),
                "post_norm": up(w("post_attention_layernorm.weight")),
                # gate and up rows interleaved in blocks of 8 (kernels.interleave_gate_up): the fused
                # SwiGLU GEMM's layout, whose decode GEMV output the down projection reads in place
                "w_gu": up(interleave_gate_up(w("mlp.gate_proj.weight"), w("mlp.up_proj.weight"))),
                "w_down": up(w("mlp.down_proj.weight")),
            })
        # Norm weights in the activation dtype for the kernels whose weight shares the output's
        # dtype (rms_norm, linear_add_rms_norm, rms_norm_rope): with float32 activations, the
        # bf16 values widened exactly (as the reference widens its checkpoint).
        f32 = lambda t: F.cast(t, "float32")  # noqa: E731
        for L in self.layers:
            for k in ("in_norm", "post_norm", "q_norm", "k_norm"):
                L[k + "_a"] = f32(L[k]) if self.act == "float32" else L[k]
        self.final_norm_a = f32(self.final_norm) if self.act == "float32" else self.final_norm
        self.rope = RotaryEmbedding(cfg.head_dim, cfg.rope_theta)
        self.cache = StaticKVCache(cfg.num_hidden_layers, 1, cfg.num_key_value_heads, max_seq_len, cfg.head_dim,
                                   dtype=self.act)
        self.scale = 1.0 / np.sqrt(cfg.head_dim)
        # prompt length -> (graph, ids, positions, logits), least recently used first.  Each captured
        # prefill keeps its activations (sized by the prompt length) in the graph's private pool, so
        # at most max_prefill_graphs lengths are kept; the least recently used is disposed first.
        self._prefill_graphs: "OrderedDict[int, tuple]" = OrderedDict()
        self.max_prefill_graphs = 4
        # Decode steps run each layer's attention block (qk-norm, RoPE, K/V write, attention, o_proj)
        # as one library call (head_dim 128); False runs the separate launches (the prefill's path
        # at S = 1).
        self.fused_decode = cfg.head_dim == 128
        # Chunks whose QKV projection kh_gemm would run on MFMA tiles without a K split run it with
        # qk-norm, RoPE and the K/V cache write in its epilogue (linear_qk_norm_rope, head_dim 128;
        # the same values); False always runs the projection and rms_norm_rope as two launches.
        self.fused_qkv_rope = cfg.head_dim == 128

    # -- decoder body shared by the prefill and the device-resident decode step -------------------
    @classmethod
    def from_pretrained(cls, path: str, max_seq_len: int = 1024, cfg: Optional[Qwen3Config] = None,
                        strict: bool = True, activations: str = "float32",
                        f32_attention: str = "split") -> "Qwen3ForCausalLM":
        """A model from a Hugging Face-layout checkpoint: `path` is a directory holding config.json and
        model.safetensors (or model.safetensors.index.json and its shards), or a .safetensors /
        index file with `cfg` given.  Weights go to the device as bf16 without an fp32 copy."""
        import os

        from ..io.safetensors import load_safetensor

        if cfg is None:
            root = path if os.path.isdir(path) else os.path.dirname(os.path.abspath(path))
            cfg = Qwen3Config.from_json_file(os.path.join(root, "config.json"))
        with load_safetensor(path) as group:
            weights, result = qwen3_weights_from_safetensor(group, cfg, strict=strict)
            model = cls(cfg, weights, max_seq_len=max_seq_len, activations=activations, f32_attention=f32_attention)
            del weights   # views of the memory maps: released before the files close
        model.load_result = result
        return model

    def _decoder(self, x: Tensor, S: int, positions: Tensor, attend, decode_block: bool = False) -> Tensor:
        """Runs every decoder layer over the fp32 residual rows x [S, hidden] in place and returns
        the fp32 logits of the last position [1, vocab].  positions: int32 [S] device tensor
        (RoPE angles and KV-cache rows); attend(layer, q_heads, out_view) writes attention for
        q_heads [1, Hq, S, D] into out_view [1, Hq, S, D].  A single row (decode) runs each norm
        and the SwiGLU product inside the projection that consumes it (linear_fused); with
        decode_block the whole attention block after the QKV projection (qk-norm, RoPE, K/V cache
        write, attention over rows [0, position], o_proj and the residual add) is one library call
        (decode_attention_block) and `attend` is not used."""
        cfg = self.cfg
        Hd = cfg.hidden_size
        eps = cfg.rms_norm_eps
        act = self.act
        one = S == 1
        n_layers = len(self.layers)
        # Multi-token rows: each residual add is fused with the RMSNorm after it
        # (linear_add_rms_norm), so h -- the normed input of the next projection, in the activation
        # dtype -- is carried from one sub-block to the next; the last down projection normalises
        # only the last row, with the final norm, for the lm_head.
        h = None if one else F.rms_norm(x, [Hd], self.layers[0]["in_norm_a"], eps, out_dtype=act)
        # The fused QKV projection sums each output over all of K, as kh_gemm does when it takes
        # its MFMA tiles (more than 8 rows) without splitting K: only then are the values the same.
        nqkv = (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim
        fuse_qkv = (self.fused_qkv_rope and not one and S > 8
                    and gemm_split_count(S, nqkv, Hd) == 1)
        # the RoPE angles of these positions, once for every layer's fused projection
        rope_tab = self.ops.find("rope_table")(positions.handle, self.rope.inv_freq.handle) if fuse_qkv else None
        for li, L in enumerate(self.layers):
            if one and decode_block:
                qkv = F.linear_fused("rms_norm", x, L["w_qkv"], L["in_norm"], eps, act_dtype=act)  # [1, nq + 2 nkv]
                self.ops.find("decode_attention_block")(qkv.handle, {
                    "q_norm": L["q_norm"].handle, "k_norm": L["k_norm"].handle, "inv_freq": self.rope.inv_freq.handle,
                    "eps": eps, "position": positions.handle, "k_cache": self.cache.key_cache[li].handle,
                    "v_cache": self.cache.value_cache[li].handle, "w_o": L["w_o"].handle, "x": x.handle,
                    "scale": self.scale})                                                # x += o W_o^T
                qkv.dispose()
            elif one:
                qkv = F.linear_fused("rms_norm", x, L["w_qkv"], L["in_norm"], eps, act_dtype=act)  # [1, nq + 2 nkv]
                attn_t = self._attention_heads(li, L, qkv, S, positions, attend)
                F.linear_fused("none", attn_t, L["w_o"], residual=x, act_dtype=act)     # x += o W_o^T
                attn_t.dispose()
            elif fuse_qkv:
                attn_t = self._attention_heads_fused(li, L, h, S, positions, attend, rope_tab)
                h.dispose()
                h = F.linear_add_rms_norm(attn_t, L["w_o"], x, L["post_norm_a"], eps)   # x += o W_o^T
                attn_t.dispose()
            else:
                qkv = F.linear(h, L["w_qkv"])                                          # [S, nq + 2 nkv]
                h.dispose()
                attn_t = self._attention_heads(li, L, qkv, S, positions, attend)
                h = F.linear_add_rms_norm(attn_t, L["w_o"], x, L["post_norm_a"], eps)   # x += o W_o^T
                attn_t.dispose()
            if one:
                a = F.linear_swiglu_row("rms_norm", x, L["w_gu"], L["post_norm"], eps,
                                        act_dtype=act)                                 # [1, I] = silu(g) * u
                F.linear_fused("none", a, L["w_down"], residual=x, act_dtype=act)      # x += a W_d^T
                a.dispose()
            else:
                a = F.linear_swiglu(h, L["w_gu"])                                      # [S, I]
                h.dispose()
                if li + 1 < n_layers:
                    h = F.linear_add_rms_norm(a, L["w_down"], x, self.layers[li + 1]["in_norm_a"], eps)
                else:
                    h = F.linear_add_rms_norm(a, L["w_down"], x, self.final_norm_a, eps, rows=(S - 1, S))
                a.dispose()
        if rope_tab is not None:
            rope_tab.dispose()
        if one:
            last = F.narrow(x, 0, S - 1, 1)
            logits = F.linear_fused("rms_norm", last, self.lm_head, self.final_norm, eps, out_dtype="float32",
                                    act_dtype=act)
            last.dispose()
        else:
            logits = F.linear(h, self.lm_head, out_dtype="float32")                    # [1, vocab] fp32
            h.dispose()
        return logits

    def _attention_heads_fused(self, li: int, L: dict, h: Tensor, S: int, positions: Tensor, attend,
                               rope_tab=None) -> Tensor:
        """As _attention_heads from the normed rows h [S, hidden] instead of their projection: one
        launch projects q/k/v and applies qk-norm + RoPE with the K/V cache write
        (linear_qk_norm_rope; the angles from rope_tab when given), then attend(); returns the
        heads [S, nq] in the activation dtype."""
        cfg = self.cfg
        Hq, D = cfg.num_attention_heads, cfg.head_dim
        nq = Hq * D
        q_heads = HipTensorHandle.create_new((1, Hq, S, D), self.act)
        self.ops.find("linear_qk_norm_rope")(h.handle, L["w_qkv"].handle, {
            "q_weight": L["q_norm"].handle, "k_weight": L["k_norm"].handle, "inv_freq": self.rope.inv_freq.handle,
            "positions": positions.handle, "eps": cfg.rms_norm_eps, "q_out": q_heads,
            "k_out": self.cache.key_cache[li].handle, "v_out": self.cache.value_cache[li].handle,
            "rope_table": rope_tab})
        attn = HipTensorHandle.create_new((S, nq), self.act)
        attn_view = HipTensorHandle.create_view(attn.storage, (1, Hq, S, D), self.act, (S * nq, D, nq, 1), 0)
        attend(li, q_heads, attn_view)
        attn_view.dispose()
        q_heads.dispose()
        return Tensor(handle=attn)

    def _attention_heads(self, li: int, L: dict, qkv: Tensor, S: int, positions: Tensor, attend) -> Tensor:
        """The attention of layer li from its QKV projection qkv [S, nq + 2 nkv] (disposed here):
        qk-norm + RoPE with the K/V cache write, then attend(); returns the heads [S, nq] bf16."""
        cfg = self.cfg
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        nq, nkv = Hq * D, Hkv * D
        q = _split_heads(qkv, 0, S, Hq, D)
        k = _split_heads(qkv, nq, S, Hkv, D)
        v = _split_heads(qkv, nq + nkv, S, Hkv, D)
        q_heads = HipTensorHandle.create_new((1, Hq, S, D), self.act)
        # K (normed + rotated) and V land in the cache rows given by `positions`.
        self.ops.find("rms_norm_rope")(q.handle, k.handle, {
            "q_weight": L["q_norm_a"].handle, "k_weight": L["k_norm_a"].handle, "inv_freq": self.rope.inv_freq.handle,
            "positions": positions.handle, "eps": cfg.rms_norm_eps, "q_out": q_heads,
            "k_out": self.cache.key_cache[li].handle, "v": v.handle, "v_out": self.cache.value_cache[li].handle,
            "cache_positions": True})
        for t in (q, k, v, qkv):
            t.dispose()
        attn = HipTensorHandle.create_new((S, nq), self.act)
        # [1, Hq, S, D] view of the [S, Hq*D] buffer: o_proj then reads it as a plain matrix.
        attn_view = HipTensorHandle.create_view(attn.storage, (1, Hq, S, D), self.act, (S * nq, D, nq, 1), 0)
        attend(li, q_heads, attn_view)
        attn_view.dispose()
        q_heads.dispose()
        return Tensor(handle=attn)

    # -- one forward over S new tokens at cache position `pos` -------------------------------------
    def _forward_dev(self, ids: Tensor, positions: Tensor, end: int) -> Tensor:
        """Forward over the device token ids [S] at device positions [S] (cache rows), attending
        over the first `end` cache rows; returns fp32 logits of the last position [1, vocab]."""
        S = ids.shape[0]
        x = F.embedding(ids, self.embed, out_dtype="float32")     # [S, Hd] fp32 residual stream

        def attend(li, q_heads, out_view):
            kc, vc = self.cache.valid_slices(li, end)
            # causal for a multi-token chunk; off for one new token (gqa.ts:333-336)
            self.ops.find(self._flash_name)(q_heads, kc.handle, vc.handle, out_view, self.scale, S > 1)
            kc.dispose()
            vc.dispose()

        logits = self._decoder(x, S, positions, attend)
        x.dispose()
        return logits

    def forward(self, input_ids: np.ndarray, pos: int) -> Tensor:
        """Runs the decoder over input_ids (int32 [S]) appended at `pos`; returns fp32 logits of the
        last position [1, vocab] (the only row greedy decoding reads)."""
        S = int(len(input_ids))
        end = self.cache.check_write(pos, S)
        ids = Tensor(np.asarray(input_ids, np.int32), dtype="int32")
        positions = RotaryEmbedding.get_position_ids(S, pos)
        logits = self._forward_dev(ids, positions, end)
        self.cache.mark_written(end)
        for t in (ids, positions):
            t.dispose()
        return logits

    def _prefill(self, prompt_ids: np.ndarray, use_graph: bool):
        """(logits, owned) of the prompt at position 0.  With use_graph, the first prompt of a given
        length runs eagerly and is then captured; later prompts of that length are copied into the
        graph's device ids buffer and replayed (owned = False: the logits buffer is the graph's)."""
        S = int(len(prompt_ids))
        if not use_graph:
            return self.forward(prompt_ids, 0), True
        entry = self._prefill_graphs.get(S)
        if entry is None:
            logits = self.forward(prompt_ids, 0)
            if self.max_prefill_graphs < 1:
                return logits, True
            while len(self._prefill_graphs) >= self.max_prefill_graphs:
                self._dispose_prefill_graph(next(iter(self._prefill_graphs)))
            ids_buf = Tensor(np.zeros(S, np.int32), dtype="int32")
            pos_buf = RotaryEmbedding.get_position_ids(S, 0)
            graph = HipGraph()
            try:
                with graph.capture():
                    g_logits = self._forward_dev(ids_buf, pos_buf, S)
            except KandleHipError:
                # e.g. device memory exhausted inside the capture (where the allocator cannot empty
                # its cache): drop every captured prefill and keep this prompt's eager result
                ids_buf.dispose()
                pos_buf.dispose()
                for key in list(self._prefill_graphs):
                    self._dispose_prefill_graph(key)
                return logits, True
            self._prefill_graphs[S] = (graph, ids_buf, pos_buf, g_logits)
            return logits, True
        self._prefill_graphs.move_to_end(S)
        graph, ids_buf, _, g_logits = entry
        ids_buf.handle.storage.upload(np.ascontiguousarray(prompt_ids, dtype=np.int32))
        graph.replay()
        self.cache.mark_written(S)
        return g_logits, False

    # -- device-resident greedy decode step ---------------------------------------------------------
    def _step_logits(self, st: "DecodeState") -> Tensor:
        """The fp32 logits [1, vocab] of the token st.ids at position st.pos, attending over st.lens
        cached rows (its K/V row is written at st.pos); every changing value is read from device
        memory, so the same launches run eagerly or replayed from a captured graph."""
        x = F.embedding(st.ids, self.embed, out_dtype="float32")  # [1, Hd]

        def attend(li, q_heads, out_view):
            self.ops.find("decode_attention")(q_heads, self.cache.key_cache[li].handle,
                                               self.cache.value_cache[li].handle, st.lens.handle, out_view,
                                               self.scale)

        logits = self._decoder(x, 1, st.pos, attend, decode_block=self.fused_decode)
        x.dispose()
        return logits

    def _decode_step(self, st: "DecodeState") -> Tensor:
        """One greedy step on device state: the logits of st.ids (_step_logits), whose argmax
        overwrites st.ids, and greedy_advance logs it and moves st.pos / st.lens on.  Returns the
        step's fp32 logits [1, vocab]."""
        logits = self._step_logits(st)
        self.ops.find("argmax")(TensorIterator.reduction_op(logits.handle, [-1], False, st.ids.handle))
        self.ops.find("greedy_advance")(st.ids.handle, st.pos.handle, st.lens.handle, st.log.handle, st.base)
        return logits

    def greedy(self, logits: Tensor) -> int:
        tok = F.argmax(logits)
        v = int(tok.numpy().reshape(-1)[0])
        tok.dispose()
        return v

    def generate(self, prompt_ids: np.ndarray, max_new_tokens: int, return_logits: bool = False,
                 use_graph: bool = True, timing: Optional[dict] = None):
        """Prefill the prompt, then greedy-decode (for_causal_lm.ts:475-508): max_new_tokens token
        ids, each the lowest-index argmax of the previous logits, after max_new_tokens decode
        forwards as in the reference loop.  The decode steps run on device state; with use_graph
        the step is captured once and replayed.  return_logits adds the fp32 logits of every forward:
        the prefill's last position and each of the max_new_tokens decode steps (the last of which
        follows the last token), max_new_tokens + 1 rows.  timing (a dict) receives wall times: prefill_ms, decode_ms (all decode steps,
        including the eager first step and the capture) and, with a graph, replay_ms over the
        replay_steps = max_new_tokens - 1 replayed steps."""
        from .. import _lib

        P, N = int(len(prompt_ids)), int(max_new_tokens)
        self.cache.reset()
        self.cache.check_write(0, P + N)
        t0 = time.perf_counter()
        logits, owned = self._prefill(prompt_ids, use_graph)
        st = DecodeState.start(logits, P, N + 1, self.ops)
        if timing is not None:
            _lib.synchronize()
            timing["prefill_ms"] = (time.perf_counter() - t0) * 1e3
            timing["prefill_issue"] = "eager" if owned else "hip graph replay"
        all_logits = [logits.numpy()[0]] if return_logits else []
        if owned:
            logits.dispose()
        graph, g_logits = None, None
        t1 = time.perf_counter()
        t_replay = None
        try:
            for i in range(N):
                if not use_graph or i == 0:
                    lg = self._decode_step(st)
                    if return_logits:
                        all_logits.append(lg.numpy()[0])
                    lg.dispose()
                    if use_graph and N > 1:
                        # Capture records the step without running it; replays 1..N-1 run it.
                        graph = HipGraph()
                        with graph.capture():
                            g_logits = self._decode_step(st)
                        if timing is not None:
                            _lib.synchronize()
                            t_replay = time.perf_counter()
                else:
                    graph.replay()
                    if return_logits:
                        all_logits.append(g_logits.numpy()[0])
            toks = st.log.numpy()[:N].tolist()   # waits for the last step
            t2 = time.perf_counter()
        finally:
            if g_logits is not None:
                g_logits.dispose()
            if graph is not None:
                graph.dispose()
            st.dispose()
        if timing is not None:
            timing["decode_ms"] = (t2 - t1) * 1e3
            if t_replay is not None:
                timing["replay_ms"] = (t2 - t_replay) * 1e3
                timing["replay_steps"] = N - 1
        self.cache.mark_written(P + N)
        return (toks, all_logits) if return_logits else toks

    def generate_stream(self, input_ids, config: Optional["GeneratorConfig"] = None, seed: int = 0,
                        use_graph: bool = True):
        """generateStream (for_causal_lm.ts:354-440): a generator that prefills the prompt, then per
        step samples a token on the device (sample(), temperature / top-k / top-p or greedy) and
        yields a GenerationStep with the token, its log-probability and the display_top_k most
        likely ids.  `generator.send(token_id)` overrides the token fed back (None keeps the
        sampled one); generation stops after max_new_tokens steps or at an EOS token.

        The draw of step i uses r = philox4x32-10(seed, counter = i), so a (seed, prompt, config)
        triple replays the same tokens (the reference draws with Math.random()).  The token fed
        back, its position, the KV length and the counter live in one device buffer written with
        one copy per step; the step's outputs are read back with one copy.  With use_graph the
        one-token forward and the draw are captured together once and replayed (except for top-p
        without top-k and prefixes over 1024 ids, whose full sort is not capturable: then only the
        forward is captured).  The reference's extra forward after the last step (its result
        unused) is not run."""
        from .sampling import SampleOutputs, SamplerConfig, sample_device

        cfg = config or GeneratorConfig()
        prompt = np.asarray(input_ids, np.int32).reshape(-1)
        P, N = int(prompt.size), int(cfg.max_new_tokens)
        eos = set(int(t) for t in cfg.eos_token_ids)
        k = min(int(cfg.display_top_k), self.cfg.vocab_size)
        sampler = SamplerConfig(cfg.temperature, cfg.top_k, cfg.top_p, cfg.do_sample)
        top_p_only = cfg.do_sample and cfg.top_p < 1.0 and not 0 < cfg.top_k < self.cfg.vocab_size
        capture_draw = not top_p_only and k <= 1024 and not (cfg.do_sample and cfg.top_k > 1024)
        self.cache.reset()
        self.cache.check_write(0, P + max(N, 1))
        logits, owned = self._prefill(prompt, use_graph)
        state = Tensor(np.zeros(4, np.int32), dtype="int32")   # token, position, KV length, counter
        ids, pos, lens, ctr = (F.narrow(state, 0, i, 1) for i in range(4))
        st = DecodeState(ids, pos, lens, None, P)
        out = SampleOutputs(k)
        draw = lambda lg: sample_device(lg, sampler, seed, ctr, out.token, k, out.logprob, out.ids,  # noqa: E731
                                        out.probs)
        graph, g_logits = None, None
        try:
            for i in range(N):
                if logits is not None:   # eager step (or a replay whose draw is not captured)
                    draw(logits)
                    if owned:
                        logits.dispose()
                    logits, owned = None, False
                res = out.read()
                override = yield GenerationStep(res.token_id, res.log_prob, res.top_k_token_ids, res.top_k_probs,
                                                res.token_id in eos, P + i, i + 1)
                tok = int(override) if override is not None else res.token_id
                if tok in eos or i + 1 == N:
                    break
                if not 0 <= tok < self.cfg.vocab_size:
                    raise ValueError(f"generate_stream: token id {tok} outside [0, {self.cfg.vocab_size})")
                state.handle.storage.upload(np.array([tok, P + i, P + i + 1, i + 1], np.int32))
                if not use_graph or graph is None:
                    logits, owned = self._step_logits(st), True
                    if use_graph:   # capture records without running: replays serve the next steps
                        graph = HipGraph()
                        with graph.capture():
                            g_logits = self._step_logits(st)
                            if capture_draw:
                                draw(g_logits)
                else:
                    graph.replay()
                    logits = None if capture_draw else g_logits
                self.cache.mark_written(P + i + 1)
        finally:
            if owned and logits is not None:
                logits.dispose()
            if g_logits is not None:
                g_logits.dispose()
            if graph is not None:
                graph.dispose()
            out.dispose()
            for t in (ids, pos, lens, ctr, state):
                t.dispose()

    def _dispose_prefill_graph(self, length: int) -> None:
        graph, ids_buf, pos_buf, g_logits = self._prefill_graphs.pop(length)
        g_logits.dispose()
        graph.dispose()
        ids_buf.dispose()
        pos_buf.dispose()

    def dispose(self) -> None:
        for key in list(self._prefill_graphs):
            self._dispose_prefill_graph(key)
        self.cache.dispose()
        heads = [self.lm_head] if self.lm_head is not self.embed else []
        extra = [self.final_norm_a] if self.final_norm_a is not self.final_norm else []
        owned = {}
        for L in self.layers:
            for v in L.values():
                owned[id(v)] = v   # the *_a norm entries alias the bf16 ones with bf16 activations
        for t in [self.embed, self.final_norm] + heads + extra + list(owned.values()):
            t.dispose()


@dataclass
class GeneratorConfig:
    """GeneratorConfig and DEFAULT_GENERATOR_CONFIG (for_causal_lm.ts:47-78)."""

    max_new_tokens: int = 256
    eos_token_ids: List[int] = field(default_factory=list)
    display_top_k: int = 10
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    do_sample: bool = True


@dataclass
class GenerationStep:
    """One yielded step of generate_stream (for_causal_lm.ts:24-41)."""

    token_id: int
    log_prob: float
    top_k_token_ids: List[int]
    top_k_probs: np.ndarray
    is_eos: bool
    cache_position: int
    generated_count: int


def _split_heads(qkv: Tensor, col0: int, S: int, H: int, D: int) -> Tensor:
    """[1, S, H, D] view of columns [col0, col0 + H*D) of the [S, ncols] projection output."""
    ncols = qkv.shape[1]
    h = HipTensorHandle.create_view(qkv.handle.storage, (1, S, H, D), qkv.dtype, (S * ncols, ncols, D, 1),
                                    qkv.offset + col0)
    return Tensor(handle=h)


class DecodeState:
    """Device-resident greedy-loop state: ids (int32 [1], the token to feed), pos (int32 [1], its
    position), lens (int32 [1], KV rows attended = pos + 1) and log (int32 [cap], the generated
    tokens; log[i] is the token for position base + i)."""

    def __init__(self, ids: Tensor, pos: Tensor, lens: Tensor, log: Tensor, base: int):
        self.ids, self.pos, self.lens, self.log, self.base = ids, pos, lens, log, base

    @classmethod
    def start(cls, prefill_logits: Tensor, prompt_len: int, cap: int, ops) -> "DecodeState":
        """State after the prefill: ids = argmax(prefill logits) (also log[0]), pos = prompt_len."""
        ids = F.zeros((1,), "int32")
        log = F.zeros((cap,), "int32")
        ops.find("argmax")(TensorIterator.reduction_op(prefill_logits.handle, [-1], False, ids.handle))
        head = F.narrow(log, 0, 0, 1)
        F.copy_(head, ids)
        head.dispose()
        pos = Tensor(np.array([prompt_len], np.int32), dtype="int32")
        lens = Tensor(np.array([prompt_len + 1], np.int32), dtype="int32")
        return cls(ids, pos, lens, log, prompt_len)

    def dispose(self) -> None:
        for t in (self.ids, self.pos, self.lens, self.log):
            t.dispose()
