'use strict';
/*
 * bench_cpu.js — times the JavaScript restatements of the reference math (flash_sdpa.js,
 * cpu_ops.js) on one thread: bench.py's CPU baseline, test infrastructure only.
 *
 * Usage: node bench_cpu.js OP DIR REPEAT ARGS...
 *   flash    DIR REPEAT B Hq Hkv Lq Lk D scale causal headsLimit   (q.f32, k.f32, v.f32 -> o.f32)
 *   decode   DIR REPEAT Hq Hkv D scale L_0 L_1 ...                 (q.f32 [B,Hq,D]; k_b.f32, v_b.f32
 *            [Hkv, L_b, D] per sequence b -> o.f32): one L = 1 SDPA per sequence, as the caller
 *            issues it for a one-token decode step (packages/model-utils/src/attention/gqa.ts:333-336)
 *   normrope DIR REPEAT T Hid Hq Hkv D eps theta                 (x.f32 [T,Hid], q.f32 [T,Hq,D],
 *            k.f32 [T,Hkv,D], w.f32, wq.f32, wk.f32 -> y.f32, qo.f32, ko.f32); positions 0..T-1
 *   qwen3    DIR REPEAT Hid I Hq Hkv D vocab S steps eps theta seed  (qwen3_cpu.js: ONE decoder layer
 *            of seeded weights, uniform in +-0.035 (std 0.02), norms 1): the S-token prefill of seeded
 *            ids, then `steps` greedy one-token forwards, and the lm_head row alone; REPEAT is
 *            ignored (one pass, no untimed run: a prefill layer takes seconds) and the op prints
 *            {"prefill_ms", "decode_ms" (per step), "head_ms"} instead of runs_ms
 * Runs the op once untimed, then REPEAT timed runs (performance.now from perf_hooks: Node 12 has no
 * global performance), writes the last run's outputs and prints {"runs_ms": [...]}.
 */
const fs = require('fs');
const path = require('path');
const perf = require('perf_hooks').performance;
const flash = require('./flash_sdpa.js');
const ops = require('./cpu_ops.js');
const qwen3 = require('./qwen3_cpu.js');

function readF32(dir, name) {
  const buf = fs.readFileSync(path.join(dir, name));
  return new Float32Array(buf.buffer, buf.byteOffset, buf.byteLength / 4);
}
function writeF32(dir, name, a) {
  fs.writeFileSync(path.join(dir, name), Buffer.from(a.buffer, a.byteOffset, a.byteLength));
}

function timed(repeat, fn) {
  fn();
  const runs = [];
  for (let i = 0; i < repeat; i++) {
    const t0 = perf.now();
    fn();
    runs.push(perf.now() - t0);
  }
  return runs;
}

function main() {
  const a = process.argv.slice(2);
  const op = a[0];
  const dir = a[1];
  const repeat = Number(a[2]);
  const p = a.slice(3).map(Number);
  let runs;
  if (op === 'flash') {
    const B = p[0], Hq = p[1], Hkv = p[2], Lq = p[3], Lk = p[4], D = p[5], scale = p[6], causal = p[7] === 1;
    const headsLimit = p[8];
    const q = readF32(dir, 'q.f32'), k = readF32(dir, 'k.f32'), v = readF32(dir, 'v.f32');
    const o = new Float32Array(B * Hq * Lq * D);
    runs = timed(repeat, function () { flash.flashSdpa(q, k, v, o, B, Hq, Hkv, Lq, Lk, D, scale, causal, headsLimit); });
    writeF32(dir, 'o.f32', o);
  } else if (op === 'decode') {
    const Hq = p[0], Hkv = p[1], D = p[2], scale = p[3];
    const lens = p.slice(4);
    const B = lens.length;
    const q = readF32(dir, 'q.f32');
    const ks = [], vs = [];
    for (let b = 0; b < B; b++) {
      ks.push(readF32(dir, 'k_' + b + '.f32'));
      vs.push(readF32(dir, 'v_' + b + '.f32'));
    }
    const o = new Float32Array(B * Hq * D);
    runs = timed(repeat, function () {
      for (let b = 0; b < B; b++) {
        const qb = q.subarray(b * Hq * D, (b + 1) * Hq * D);
        const ob = o.subarray(b * Hq * D, (b + 1) * Hq * D);
        flash.flashSdpa(qb, ks[b], vs[b], ob, 1, Hq, Hkv, 1, lens[b], D, scale, false, 0);
      }
    });
    writeF32(dir, 'o.f32', o);
  } else if (op === 'normrope') {
    const T = p[0], Hid = p[1], Hq = p[2], Hkv = p[3], D = p[4], eps = p[5], theta = p[6];
    const x = readF32(dir, 'x.f32'), q = readF32(dir, 'q.f32'), k = readF32(dir, 'k.f32');
    const w = readF32(dir, 'w.f32'), wq = readF32(dir, 'wq.f32'), wk = readF32(dir, 'wk.f32');
    const y = new Float32Array(T * Hid), qo = new Float32Array(T * Hq * D), ko = new Float32Array(T * Hkv * D);
    const pos = new Int32Array(T);
    for (let t = 0; t < T; t++) pos[t] = t;
    const inv = ops.ropeInvFreq(D, theta);
    runs = timed(repeat, function () {
      ops.rmsNorm(x, 0, w, y, 0, T, Hid, eps);
      const tab = ops.ropeTables(pos, inv, D);
      ops.qkNormRope(q, wq, qo, T, Hq, D, tab, eps);
      ops.qkNormRope(k, wk, ko, T, Hkv, D, tab, eps);
    });
    writeF32(dir, 'y.f32', y);
    writeF32(dir, 'qo.f32', qo);
    writeF32(dir, 'ko.f32', ko);
  } else if (op === 'qwen3') {
    const cfg = { hiddenSize: p[0], intermediateSize: p[1], numAttentionHeads: p[2], numKeyValueHeads: p[3],
                  headDim: p[4], vocabSize: p[5], numHiddenLayers: 1, rmsNormEps: p[8], ropeTheta: p[9] };
    const S = p[6], steps = p[7];
    let st = (p[10] >>> 0) || 1;
    const rnd = function () {  // xorshift32, uniform in [0, 1)
      st ^= st << 13; st >>>= 0; st ^= st >>> 17; st ^= st << 5; st >>>= 0;
      return st / 4294967296;
    };
    const fill = function (n, ones) {
      const a = new Float32Array(n);
      for (let i = 0; i < n; i++) a[i] = ones ? 1 : (rnd() * 2 - 1) * 0.035;
      return a;
    };
    const Hd = cfg.hiddenSize, I = cfg.intermediateSize, D = cfg.headDim;
    const nq = cfg.numAttentionHeads * D, nkv = cfg.numKeyValueHeads * D;
    const pre = 'model.layers.0.';
    const w = {
      'model.embed_tokens.weight': fill(cfg.vocabSize * Hd), 'model.norm.weight': fill(Hd, true),
    };
    w[pre + 'input_layernorm.weight'] = fill(Hd, true);
    w[pre + 'post_attention_layernorm.weight'] = fill(Hd, true);
    w[pre + 'self_attn.q_norm.weight'] = fill(D, true);
    w[pre + 'self_attn.k_norm.weight'] = fill(D, true);
    w[pre + 'self_attn.q_proj.weight'] = fill(nq * Hd);
    w[pre + 'self_attn.k_proj.weight'] = fill(nkv * Hd);
    w[pre + 'self_attn.v_proj.weight'] = fill(nkv * Hd);
    w[pre + 'self_attn.o_proj.weight'] = fill(Hd * nq);
    w[pre + 'mlp.gate_proj.weight'] = fill(I * Hd);
    w[pre + 'mlp.up_proj.weight'] = fill(I * Hd);
    w[pre + 'mlp.down_proj.weight'] = fill(Hd * I);
    const model = new qwen3.Qwen3Cpu(cfg, w, S + steps + 1);
    const ids = [];
    for (let i = 0; i < S; i++) ids.push(Math.floor(rnd() * cfg.vocabSize));
    let t0 = perf.now();
    let logits = model.forward(ids, 0);
    const prefillMs = perf.now() - t0;
    t0 = perf.now();
    for (let i = 0; i < steps; i++) logits = model.forward([qwen3.argmax(logits)], S + i);
    const decodeMs = (perf.now() - t0) / steps;
    const row = fill(Hd, true);
    t0 = perf.now();
    for (let i = 0; i < 3; i++) model.lmHead(row);
    const headMs = (perf.now() - t0) / 3;
    process.stdout.write(JSON.stringify({ prefill_ms: prefillMs, decode_ms: decodeMs, head_ms: headMs,
                                          last_token: qwen3.argmax(logits) }) + '\n');
    return;
  } else {
    process.stderr.write('unknown op ' + op + '\n');
    process.exit(2);
  }
  process.stdout.write(JSON.stringify({ runs_ms: runs }) + '\n');
}

main();
