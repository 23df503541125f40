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
 * Runs the op once untimed, then REPEAT timed runs (performance.now from perf_hooks: Node 12 has no
 * global performance), writes the last run's outputs and prints {"runs_ms": [...]}.
 */
const fs = require('fs');
const path = require('path');
const perf = require('perf_hooks').performance;
const flash = require('./flash_sdpa.js');
const ops = require('./cpu_ops.js');

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
  } else {
    process.stderr.write('unknown op ' + op + '\n');
    process.exit(2);
  }
  process.stdout.write(JSON.stringify({ runs_ms: runs }) + '\n');
}

main();
