"""Writes tests/golden/qwen3_tiny.npz: a tiny Qwen3 causal LM run by Hugging Face transformers'
Qwen3ForCausalLM (CPU, float32, eager attention) -- an implementation of the architecture that is
independent of both the reference and this repository's oracle.

The reference's Qwen3 module chain (packages/model-utils/src/qwen3/{model,decoder_layer,
for_causal_lm}.ts, attention/gqa.ts, mlp/swiglu.ts) loads Hugging Face checkpoints of this
architecture; these vectors pin the composition in oracle/qwen3.py (layer order, pre-norms, per-head
q/k RMSNorm before RoPE, rotate_half RoPE, GQA, SwiGLU, tied lm_head, greedy decoding) at float32,
beyond the per-op checks of golden.npz.

Stored: the weights as bf16 bit patterns (every value bf16-representable, so both implementations
see identical weights), the prompt, the 3 tokens greedy decoding appends, and the float32 logits
at the last prompt position and at each appended position.

Run: python tests/golden/make_qwen3_golden.py   (CPU only; writes the .npz beside this file)
"""
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "qwen3_tiny.npz"

CFG = dict(vocab_size=97, hidden_size=64, intermediate_size=96, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-6, rope_theta=1e6, max_position_embeddings=128,
           tie_word_embeddings=True)
PROMPT = [5, 17, 3, 88, 42, 0, 61]
STEPS = 3


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main():
    from transformers import Qwen3Config, Qwen3ForCausalLM

    torch.manual_seed(4321)
    cfg = Qwen3Config(**CFG, attention_bias=False, hidden_act="silu")
    cfg._attn_implementation = "eager"
    model = Qwen3ForCausalLM(cfg).float().eval()
    weights = {}
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name == "lm_head.weight":
                continue  # tied to model.embed_tokens.weight
            v = torch.randn_like(p) * 0.1 if p.dim() == 2 else 0.5 + torch.rand_like(p)
            v = v.to(torch.bfloat16).float()
            p.copy_(v)
            weights[name] = bf16_bits(v)
        model.lm_head.weight = model.model.embed_tokens.weight
        ids = list(PROMPT)
        for _ in range(STEPS):
            logits = model(torch.tensor([ids])).logits[0, -1]
            ids.append(int(torch.argmax(logits)))
        full = model(torch.tensor([ids])).logits[0].float().numpy()
    P = len(PROMPT)
    out = {f"w:{k}": v for k, v in weights.items()}
    out["ids"] = np.array(ids, np.int32)
    out["prompt_len"] = np.array(P, np.int32)
    out["logits"] = full[P - 1:P - 1 + STEPS + 1]  # last prompt position, then each appended token
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({len(weights)} tensors, ids {ids})")


if __name__ == "__main__":
    main()
