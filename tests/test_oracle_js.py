"""The JavaScript Qwen3 forward (oracle/js/qwen3_cpu.js, the C5 CPU baseline that bench.py times in
Node) against the numpy oracle with its bf16 rounding points off (oracle/qwen3.py, exact=True), on
a 2-layer configuration small enough to run in a second: the prefill of a 10-token prompt and three
greedy decode steps must give the same tokens and logits within 1e-4 of their scale.  The numpy
oracle itself is pinned against Hugging Face transformers in tests/test_oracle.py, so a JavaScript
restatement that drops a term, swaps an operand or misplaces a RoPE half fails here."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from kandle_amd import synthetic as syn
from kandle_amd.model_utils import Qwen3Config, init_qwen3_weights
from oracle import from_bf16_bits
from oracle.qwen3 import Qwen3Oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "oracle", "js", "qwen3_cpu.js")

DRIVER = r"""
const fs = require('fs');
const path = require('path');
const { Qwen3Cpu, argmax } = require(process.argv[1]);   // node -e SCRIPT JS DIR
const dir = process.argv[2];
const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
const w = {};
for (const name of meta.names) {
  const buf = fs.readFileSync(path.join(dir, name + '.f32'));
  w[name] = new Float32Array(buf.buffer, buf.byteOffset, buf.byteLength / 4);
}
const model = new Qwen3Cpu(meta.cfg, w, meta.prompt.length + meta.steps + 1);
let logits = model.forward(meta.prompt, 0);
const rows = [Array.from(logits)];
const toks = [];
for (let i = 0; i < meta.steps; i++) {
  const t = argmax(logits);
  toks.push(t);
  logits = model.forward([t], meta.prompt.length + i);
  rows.push(Array.from(logits));
}
console.log(JSON.stringify({ tokens: toks, logits: rows }));
"""


def test_js_qwen3_matches_numpy_oracle(tmp_path):
    if shutil.which("node") is None:
        pytest.skip("node is not available")
    cfg = Qwen3Config(vocab_size=97, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16)
    w = init_qwen3_weights(cfg, seed=21)
    for i, name in enumerate(sorted(k for k in w if k.endswith("norm.weight"))):   # norms other than 1
        w[name] = syn.bf16(syn.uniform(300 + i, w[name].shape, 0.5, 1.5))[0]
    # larger projections than N(0, 0.02) so that the logits spread and the tokens are not near ties
    for name in w:
        if name.endswith("proj.weight"):
            w[name] = syn.bf16(syn.normal(400 + len(name), w[name].shape) * 0.2)[0]
    prompt = syn.randint(22, (10,), 0, cfg.vocab_size)
    steps = 3
    for name, bits in w.items():
        from_bf16_bits(bits).astype(np.float32).tofile(str(tmp_path / (name + ".f32")))
    meta = {"names": sorted(w), "prompt": [int(t) for t in prompt], "steps": steps,
            "cfg": {"vocabSize": cfg.vocab_size, "hiddenSize": cfg.hidden_size,
                    "intermediateSize": cfg.intermediate_size, "numHiddenLayers": cfg.num_hidden_layers,
                    "numAttentionHeads": cfg.num_attention_heads, "numKeyValueHeads": cfg.num_key_value_heads,
                    "headDim": cfg.head_dim, "rmsNormEps": cfg.rms_norm_eps, "ropeTheta": cfg.rope_theta}}
    (tmp_path / "meta.json").write_text(json.dumps(meta))
    out = subprocess.run(["node", "-e", DRIVER, JS, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads(out.stdout.strip().splitlines()[-1])

    ref = Qwen3Oracle(cfg, w, max_seq_len=len(prompt) + steps + 1, exact=True)
    logits = ref.forward(prompt, 0)
    want_rows, want_toks = [logits], []
    for i in range(steps):
        t = int(np.argmax(logits))
        want_toks.append(t)
        logits = ref.forward([t], len(prompt) + i)
        want_rows.append(logits)
    assert res["tokens"] == want_toks
    got = np.array(res["logits"], np.float64)
    want = np.stack(want_rows).astype(np.float64)
    scale = float(np.max(np.abs(want)))
    assert scale > 0.1
    err = float(np.max(np.abs(got - want)))
    assert err < 1e-4 * scale, (err, scale)
