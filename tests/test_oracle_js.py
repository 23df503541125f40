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


OPS = os.path.join(ROOT, "oracle", "js", "cpu_ops.js")
OPS_DRIVER = r"""
const fs = require('fs');
const path = require('path');
const ops = require(process.argv[1]);                    // node -e SCRIPT OPS DIR
const dir = process.argv[2];
const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
const rd = (n) => { const b = fs.readFileSync(path.join(dir, n)); return new Float32Array(b.buffer, b.byteOffset, b.byteLength / 4); };
const { T, H, D, N, eps, theta } = meta;
const x = rd('x'), wx = rd('wx'), q = rd('q'), wq = rd('wq');
const y = new Float32Array(T * N);
ops.rmsNorm(x, 0, wx, y, 0, T, N, eps);
const inv = ops.ropeInvFreq(D, theta);
const tab = ops.ropeTables(Int32Array.from(meta.pos), inv, D);
const qo = new Float32Array(T * H * D);
ops.qkNormRope(q, wq, qo, T, H, D, tab, eps);
fs.writeFileSync(path.join(dir, 'y'), Buffer.from(y.buffer));
fs.writeFileSync(path.join(dir, 'qo'), Buffer.from(qo.buffer));
fs.writeFileSync(path.join(dir, 'inv'), Buffer.from(inv.buffer));
console.log('ok');
"""


def test_js_cpu_ops_match_c_oracle(tmp_path):
    """oracle/js/cpu_ops.js (the C2 CPU baseline's RMSNorm and qk-norm + RoPE) at C2's head_dim 128
    and hidden 1024 against the C oracle's or_rms_norm / or_rope_inv_freq / or_qk_norm_rope on the
    same inputs: to float32 rounding (1e-5 of the output scale; positions up to 4000, so the angles
    reach thousands of radians)."""
    import oracle

    if shutil.which("node") is None:
        pytest.skip("node is not available")
    T, H, D, N, eps, theta = 9, 3, 128, 1024, 1e-6, 1e6
    x = syn.normal(31, (T, N), 3.0)
    wx = syn.uniform(32, (N,), 0.5, 1.5)
    q = syn.normal(33, (T, H, D), 2.0)
    wq = syn.uniform(34, (D,), 0.5, 1.5)
    pos = [0, 1, 2, 17, 255, 511, 1000, 2999, 4000]
    for name, arr in (("x", x), ("wx", wx), ("q", q), ("wq", wq)):
        np.ascontiguousarray(arr, np.float32).tofile(str(tmp_path / name))
    (tmp_path / "meta.json").write_text(json.dumps({"T": T, "H": H, "D": D, "N": N, "eps": eps, "theta": theta,
                                                    "pos": pos}))
    out = subprocess.run(["node", "-e", OPS_DRIVER, OPS, str(tmp_path)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr[-2000:]
    inv = np.fromfile(str(tmp_path / "inv"), np.float32)
    assert np.array_equal(inv, oracle.rope_inv_freq(D, theta))
    y = np.fromfile(str(tmp_path / "y"), np.float32).reshape(T, N)
    ry = oracle.rms_norm(x, wx, eps)
    assert float(np.max(np.abs(y - ry))) <= 1e-5 * float(np.max(np.abs(ry)))
    qo = np.fromfile(str(tmp_path / "qo"), np.float32).reshape(T, H, D)
    rq = oracle.qk_norm_rope(q, wq, np.array(pos, np.int32), inv, eps)
    assert float(np.max(np.abs(qo - rq))) <= 1e-5 * float(np.max(np.abs(rq)))
