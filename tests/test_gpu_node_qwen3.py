"""The TypeScript Qwen3 model (packages/backend-hip/src/qwen3.ts) generating from Node: a 2-layer
Qwen3 with the 0.6B's layer shapes (hidden 1024, 16/8 heads of 128, MLP 3072; vocab 4096) is written
as a bf16 safetensors checkpoint; tests/node/qwen3_generate.js reads it, runs the prefill of a
40-token prompt and 8 greedy decode steps through the backend's registry kernels and writes every
forward's logits, then generates twice more with HIP graphs: the decode step captured and replayed,
and the second time the prefill replayed from the graph captured for its prompt length.
The Python model (kandle_amd.model_utils.qwen3) on the same weights must give the same tokens and
the same logits bit for bit -- both hosts issue the same launches, eagerly or replayed -- and the
same RoPE inverse frequencies; every device byte the TS model allocated is returned."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from kandle_amd import synthetic as syn
from kandle_amd.model_utils.qwen3 import Qwen3Config, Qwen3ForCausalLM, init_qwen3_weights

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "packages", "backend-hip")
ADDON = os.path.join(PKG, "native", "kandle_hip.node")
SCRIPT = os.path.join(ROOT, "tests", "node", "qwen3_generate.js")


def _ensure_dist():
    for mod in ("index", "qwen3"):
        src = os.path.join(PKG, "src", mod + ".ts")
        dist = os.path.join(PKG, "dist", mod + ".js")
        if not os.path.exists(dist) or os.path.getmtime(dist) < os.path.getmtime(src):
            os.makedirs(os.path.dirname(dist), exist_ok=True)
            subprocess.run(["node", os.path.join(PKG, "strip-types.js"), src, dist], check=True, timeout=60)


@pytest.mark.parametrize("heads,kv_heads,head_dim", [
    (16, 8, 128),   # the 0.6B's attention shapes
    (10, 2, 128),   # GQA ratio 5
    (16, 8, 64),    # head dim 64: the decode step's attention as separate launches
])
def test_typescript_qwen3_generation_matches_python_model(hip, tmp_path, heads, kv_heads, head_dim):
    if shutil.which("node") is None or not os.path.exists(ADDON):
        pytest.skip("node or the built addon is not available")
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file

    _ensure_dist()
    cfg = Qwen3Config(vocab_size=4096, num_hidden_layers=2, num_attention_heads=heads, num_key_value_heads=kv_heads,
                      head_dim=head_dim)
    w = init_qwen3_weights(cfg, seed=13)
    for i, name in enumerate(sorted(k for k in w if k.endswith("norm.weight"))):   # norms other than 1
        w[name] = syn.bf16(syn.uniform(500 + i, w[name].shape, 0.5, 1.5))[0]
    save_file({k: torch.from_numpy(v.astype(np.int16)).view(torch.bfloat16) for k, v in w.items()},
              str(tmp_path / "model.safetensors"))
    prompt = syn.randint(14, (40,), 0, cfg.vocab_size)
    N, max_seq = 8, 64
    meta = {"cfg": {"vocabSize": cfg.vocab_size, "hiddenSize": cfg.hidden_size,
                    "intermediateSize": cfg.intermediate_size, "numHiddenLayers": cfg.num_hidden_layers,
                    "numAttentionHeads": cfg.num_attention_heads, "numKeyValueHeads": cfg.num_key_value_heads,
                    "headDim": cfg.head_dim, "rmsNormEps": cfg.rms_norm_eps, "ropeTheta": cfg.rope_theta},
            "prompt": prompt.tolist(), "n": N, "maxSeq": max_seq}
    (tmp_path / "meta.json").write_text(json.dumps(meta))
    out = subprocess.run(["node", SCRIPT, str(tmp_path)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads(out.stdout.strip().splitlines()[-1])
    assert res["liveAfter"] == res["liveBefore"], res
    ts_logits = np.fromfile(str(tmp_path / "logits.f32"), np.float32).reshape(N + 1, cfg.vocab_size)

    model = Qwen3ForCausalLM(cfg, w, max_seq_len=max_seq)
    try:
        np.testing.assert_array_equal(np.fromfile(str(tmp_path / "inv_freq.f32"), np.float32),
                                      model.rope.inv_freq_host)
        toks, logits = model.generate(prompt, N, return_logits=True, use_graph=False)
    finally:
        model.dispose()
    assert res["tokens"] == list(toks)
    assert np.all(np.isfinite(ts_logits))
    np.testing.assert_array_equal(ts_logits, np.stack(logits))
    # graph replay of the decode step, then of the prefill as well, issues the same launches:
    # identical tokens and logits
    assert res["tokensGraph"] == list(toks) and res["rowsGraph"] == N + 1
    assert res["tokensGraph2"] == list(toks) and res["rowsGraph2"] == N + 1
    assert res["prefillGraphs"] == [len(prompt)]
    for name in ("logits_graph.f32", "logits_graph2.f32"):
        np.testing.assert_array_equal(np.fromfile(str(tmp_path / name), np.float32).reshape(N + 1, cfg.vocab_size),
                                      ts_logits)
