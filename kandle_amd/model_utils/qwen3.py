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
  gu  = h W_gu^T                                               [S, 2 I] (gate rows then up rows)
  x   = x + silu(gu[:, :I]) * gu[:, I:] W_down^T                (silu_mul, matmul + residual)
then x = rms_norm(x, norm) and logits = x[last] E^T in fp32 with the tied embedding E
(for_causal_lm.ts:121-125, 184-185); greedy = argmax, lowest index among maxima (:475-508).
The residual stream x is float32 (embedding rows widened on gather; the o_proj and down GEMMs add
into it in their fp32 epilogue); every other activation is stored in bf16 between kernels (the norms
read fp32 x and write bf16 h); math inside kernels is fp32.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from .. import env
from .. import functional as F
from .. import synthetic as syn
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


class Qwen3ForCausalLM:
    def __init__(self, cfg: Qwen3Config, weights: Dict[str, np.ndarray], max_seq_len: int = 1024):
        self.cfg = cfg
        self.max_seq_len = max_seq_len
        self.ops = env.get_backend("hip").operators
        up = lambda a: Tensor(a, dtype="bfloat16")  # noqa: E731  (uint16 bits -> bf16 tensor)
        self.embed = up(weights["model.embed_tokens.weight"])
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
                "w_gu": up(np.concatenate([w("mlp.gate_proj.weight"), w("mlp.up_proj.weight")], axis=0)),
                "w_down": up(w("mlp.down_proj.weight")),
            })
        self.rope = RotaryEmbedding(cfg.head_dim, cfg.rope_theta)
        self.cache = StaticKVCache(cfg.num_hidden_layers, 1, cfg.num_key_value_heads, max_seq_len, cfg.head_dim)
        self.scale = 1.0 / np.sqrt(cfg.head_dim)

    # -- one forward over S new tokens at cache position `pos` -------------------------------------
    def forward(self, input_ids: np.ndarray, pos: int) -> Tensor:
        """Runs the decoder over input_ids (int32 [S]) appended at `pos`; returns fp32 logits of the
        last position [1, vocab] (the only row greedy decoding reads)."""
        cfg = self.cfg
        S = int(len(input_ids))
        Hq, Hkv, D, Hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.hidden_size
        nq, nkv = Hq * D, Hkv * D
        end = self.cache.check_write(pos, S)
        ids = Tensor(np.asarray(input_ids, np.int32), dtype="int32")
        x = F.embedding(ids, self.embed, out_dtype="float32")     # [S, Hd] fp32 residual stream
        positions = RotaryEmbedding.get_position_ids(S, pos)
        eps = cfg.rms_norm_eps
        for li, L in enumerate(self.layers):
            h = F.rms_norm(x, [Hd], L["in_norm"], eps, out_dtype="bfloat16")
            qkv = F.linear(h, L["w_qkv"])                          # [S, nq + 2 nkv]
            h.dispose()
            q = _split_heads(qkv, 0, S, Hq, D)
            k = _split_heads(qkv, nq, S, Hkv, D)
            v = _split_heads(qkv, nq + nkv, S, Hkv, D)
            k_dst, v_dst = self.cache.write_slices(li, pos, S)
            q_heads = HipTensorHandle.create_new((1, Hq, S, D), "bfloat16")
            self.ops.find("rms_norm_rope")(q.handle, k.handle, {
                "q_weight": L["q_norm"].handle, "k_weight": L["k_norm"].handle, "inv_freq": self.rope.inv_freq.handle,
                "positions": positions.handle, "eps": eps, "q_out": q_heads, "k_out": k_dst.handle,
                "v": v.handle, "v_out": v_dst.handle})
            for t in (q, k, v, k_dst, v_dst):
                t.dispose()
            qkv.dispose()
            kc, vc = self.cache.valid_slices(li, end)
            attn = HipTensorHandle.create_new((S, nq), "bfloat16")
            # [1, Hq, S, D] view of the [S, Hq*D] buffer: o_proj then reads it as a plain matrix.
            attn_view = HipTensorHandle.create_view(attn.storage, (1, Hq, S, D), "bfloat16", (S * nq, D, nq, 1), 0)
            self.ops.find("flash_attention")(q_heads, kc.handle, vc.handle, attn_view, self.scale, S > 1)
            attn_view.dispose()
            q_heads.dispose()
            kc.dispose()
            vc.dispose()
            attn_t = Tensor(handle=attn)
            F.dispatch_matmul(attn_t, L["w_o"], c=x, beta=1.0, out=x, transpose_b=True)   # x += o W_o^T
            attn_t.dispose()
            h = F.rms_norm(x, [Hd], L["post_norm"], eps, out_dtype="bfloat16")
            gu = F.linear(h, L["w_gu"])                            # [S, 2I]
            h.dispose()
            I = cfg.intermediate_size
            a = F.silu_mul(F.narrow(gu, 1, 0, I), F.narrow(gu, 1, I, I))
            gu.dispose()
            F.dispatch_matmul(a, L["w_down"], c=x, beta=1.0, out=x, transpose_b=True)     # x += a W_d^T
            a.dispose()
        self.cache.mark_written(end)
        last = F.narrow(x, 0, S - 1, 1)
        xf = F.rms_norm(last, [Hd], self.final_norm, eps, out_dtype="bfloat16")
        logits = F.linear(xf, self.embed, out_dtype="float32")     # [1, vocab] fp32
        for t in (last, xf, x, ids, positions):
            t.dispose()
        return logits

    def greedy(self, logits: Tensor) -> int:
        tok = F.argmax(logits)
        v = int(tok.numpy().reshape(-1)[0])
        tok.dispose()
        return v

    def generate(self, prompt_ids: np.ndarray, max_new_tokens: int, return_logits: bool = False):
        """Prefill the prompt, then greedy-decode max_new_tokens tokens (for_causal_lm.ts:475-508)."""
        self.cache.reset()
        logits = self.forward(prompt_ids, 0)
        pos = len(prompt_ids)
        out, all_logits = [], []
        for _ in range(max_new_tokens):
            if return_logits:
                all_logits.append(logits.numpy()[0])
            nxt = self.greedy(logits)
            logits.dispose()
            out.append(nxt)
            logits = self.forward(np.array([nxt], np.int32), pos)
            pos += 1
        logits.dispose()
        return (out, all_logits) if return_logits else out

    def dispose(self) -> None:
        self.cache.dispose()
        for t in [self.embed, self.final_norm] + [v for L in self.layers for v in L.values()]:
            t.dispose()


def _split_heads(qkv: Tensor, col0: int, S: int, H: int, D: int) -> Tensor:
    """[1, S, H, D] view of columns [col0, col0 + H*D) of the [S, ncols] projection output."""
    ncols = qkv.shape[1]
    h = HipTensorHandle.create_view(qkv.handle.storage, (1, S, H, D), qkv.dtype, (S * ncols, ncols, D, 1),
                                    qkv.offset + col0)
    return Tensor(handle=h)
