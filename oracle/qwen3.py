"""CPU restatement of the Qwen3 causal-LM forward — TEST INFRASTRUCTURE ONLY (the checker of the
GPU model path; never imported by kandle_amd).

Follows the reference module order: Qwen3Model.forwardWithLayerOutputs (packages/model-utils/src/
qwen3/model.ts:265-347), Qwen3DecoderLayer.forward (qwen3/decoder_layer.ts:191-241),
GroupedQueryAttention.forward (attention/gqa.ts:246-430: projections, per-head q_norm/k_norm,
RoPE, KV-cache update, SDPA with causal off for a single new token, o_proj), SwiGLUMLP.forward
(mlp/swiglu.ts:119-134), tied lm_head (qwen3/for_causal_lm.ts:121-125, 184-185) and greedy argmax
(for_causal_lm.ts:475-508).

Rounding points mirror the GPU path: the residual stream x stays float32 (embedding rows widened,
projection outputs added in fp32); every other tensor that the GPU stores between kernels is rounded
to bf16 here too (norm outputs, q/k/v projections, q/k after norm+RoPE, attention output, gate/up,
silu*mul); math between those points is fp32 (GEMMs, numpy sgemm) or double (norms, RoPE, softmax);
logits are fp32.
"""
from __future__ import annotations

import numpy as np

from . import bf16_round, from_bf16_bits, qk_norm_rope, rms_norm, rope_inv_freq


ROUNDING_POINTS = ("norm", "qkv", "qk_rope", "attn", "gate_up", "act", "final_norm")


class Qwen3Oracle:
    """exact=True drops the bf16 rounding points (every intermediate stays float32/float64): the
    form checked against an independent float32 implementation of the architecture.  `rounding`
    names the points that are rounded to bf16 (a subset of ROUNDING_POINTS; default: all of them
    unless exact)."""

    def __init__(self, cfg, weights_bits, max_seq_len: int = 1024, exact: bool = False, rounding=None):
        self.cfg = cfg
        if rounding is None:
            rounding = () if exact else ROUNDING_POINTS
        unknown = set(rounding) - set(ROUNDING_POINTS)
        if unknown:
            raise ValueError(f"unknown rounding points {sorted(unknown)}")
        self.rounding = frozenset(rounding)
        f = lambda n: from_bf16_bits(weights_bits[n])  # noqa: E731
        self.embed = f("model.embed_tokens.weight")
        self.final_norm = f("model.norm.weight")
        self.layers = []
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            self.layers.append({k: f(p + n) for k, n in (
                ("in_norm", "input_layernorm.weight"), ("q", "self_attn.q_proj.weight"),
                ("k", "self_attn.k_proj.weight"), ("v", "self_attn.v_proj.weight"), ("o", "self_attn.o_proj.weight"),
                ("q_norm", "self_attn.q_norm.weight"), ("k_norm", "self_attn.k_norm.weight"),
                ("post_norm", "post_attention_layernorm.weight"), ("gate", "mlp.gate_proj.weight"),
                ("up", "mlp.up_proj.weight"), ("down", "mlp.down_proj.weight"))})
        self.inv_freq = rope_inv_freq(cfg.head_dim, cfg.rope_theta)
        Hkv, D = cfg.num_key_value_heads, cfg.head_dim
        self.k_cache = [np.zeros((Hkv, max_seq_len, D), np.float32) for _ in range(cfg.num_hidden_layers)]
        self.v_cache = [np.zeros((Hkv, max_seq_len, D), np.float32) for _ in range(cfg.num_hidden_layers)]

    def r(self, a, point: str):
        """a as float32, rounded to bf16 when `point` is one of the active rounding points."""
        return bf16_round(a) if point in self.rounding else np.asarray(a, np.float32)

    @staticmethod
    def _sdpa(q, k, v, scale, causal):
        """q [Hq, S, D], k/v [Hkv, L, D] -> [Hq, S, D]; GQA h -> h // (Hq / Hkv); top-left causal."""
        Hq, S, D = q.shape
        Hkv, L, _ = k.shape
        G = Hq // Hkv
        out = np.empty((Hq, S, D), np.float64)
        mask = np.triu(np.ones((S, L), bool), k=1) if causal else None
        for h in range(Hq):
            s = (q[h].astype(np.float64) @ k[h // G].astype(np.float64).T) * scale
            if causal:
                s[mask] = -np.inf
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            out[h] = (p / p.sum(axis=1, keepdims=True)) @ v[h // G].astype(np.float64)
        return out

    def forward(self, ids, pos: int) -> np.ndarray:
        """fp32 logits of the last position after appending ids at cache position pos."""
        cfg = self.cfg
        S = len(ids)
        Hq, Hkv, D, Hd, eps = (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.hidden_size,
                               cfg.rms_norm_eps)
        end = pos + S
        x = self.embed[np.asarray(ids)].astype(np.float32)                    # fp32 residual [S, Hd]
        positions = np.arange(pos, end, dtype=np.int32)
        for li, L in enumerate(self.layers):
            h = self.r(rms_norm(x, L["in_norm"], eps), "norm")
            q = self.r(h @ L["q"].T, "qkv").reshape(S, Hq, D)
            k = self.r(h @ L["k"].T, "qkv").reshape(S, Hkv, D)
            v = self.r(h @ L["v"].T, "qkv").reshape(S, Hkv, D)
            qh = self.r(qk_norm_rope(q, L["q_norm"], positions, self.inv_freq, eps), "qk_rope").transpose(1, 0, 2)
            kh = self.r(qk_norm_rope(k, L["k_norm"], positions, self.inv_freq, eps), "qk_rope").transpose(1, 0, 2)
            self.k_cache[li][:, pos:end] = kh
            self.v_cache[li][:, pos:end] = v.transpose(1, 0, 2)
            o = self._sdpa(qh, self.k_cache[li][:, :end], self.v_cache[li][:, :end], 1.0 / np.sqrt(D), S > 1)
            o = self.r(o.transpose(1, 0, 2).reshape(S, Hq * D), "attn")
            x = (x + (o @ L["o"].T)).astype(np.float32)
            h = self.r(rms_norm(x, L["post_norm"], eps), "norm")
            g = h @ L["gate"].T
            u = h @ L["up"].T
            g = self.r(g, "gate_up")
            u = self.r(u, "gate_up")
            c = np.clip(g.astype(np.float64), -88.0, 88.0)
            a = self.r(g / (1.0 + np.exp(-c)) * u, "act")
            x = (x + (a @ L["down"].T)).astype(np.float32)
        xf = self.r(rms_norm(x[-1:], self.final_norm, eps), "final_norm")
        return (xf @ self.embed.T)[0].astype(np.float32)

    def generate(self, prompt_ids, max_new_tokens: int):
        """(token ids, logits of every forward) for greedy decoding; argmax keeps the lowest index on
        ties.  The logits are the prefill's last position and each decode step's, the last one
        after the last token: max_new_tokens + 1 rows."""
        logits = self.forward(prompt_ids, 0)
        pos = len(prompt_ids)
        toks, all_logits = [], []
        for _ in range(max_new_tokens):
            all_logits.append(logits)
            nxt = int(np.argmax(logits))
            toks.append(nxt)
            logits = self.forward([nxt], pos)
            pos += 1
        all_logits.append(logits)
        return toks, all_logits
