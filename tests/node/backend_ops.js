'use strict';
/*
 * backend_ops.js — runs kernels through the TypeScript HipBackend (packages/backend-hip, compiled
 * by strip-types.js into dist/index.js) the way Kandle's dispatcher calls them: registry lookups by
 * name and the reference kernel signatures.  Test infrastructure: tests/test_gpu_node_backend.py
 * writes the inputs and checks the outputs against the CPU oracle.
 *
 * Usage: node backend_ops.js DIR
 *   DIR/meta.json holds the shapes; inputs are raw little-endian files (bf16 as uint16 bits, f32,
 *   int32); outputs are written back as f32 (or int32) files and a JSON summary is printed.
 */
const fs = require('fs');
const path = require('path');
const { HipBackend, HipTensorIterator } = require(path.join(__dirname, '..', '..', 'packages', 'backend-hip', 'dist',
                                                             'index.js'));

const dir = process.argv[2];
const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));

function readU16(name) {
  const b = fs.readFileSync(path.join(dir, name));
  return new Uint16Array(b.buffer, b.byteOffset, b.length / 2);
}
function readF32(name) {
  const b = fs.readFileSync(path.join(dir, name));
  return new Float32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.length));
}
function readI32(name) {
  const b = fs.readFileSync(path.join(dir, name));
  return new Int32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.length));
}
function write(name, arr) {
  fs.writeFileSync(path.join(dir, name), Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength));
}

// full(fill_value) into an existing handle: the nullary iterator of handlers/factory.ts:50-61
function fullIter(h, value) {
  const it = HipTensorIterator.nullaryOp(h.shape, h.dtype, h);
  it.setScalarArgs({ fill_value: value });
  return it;
}

async function main() {
  const backend = await HipBackend.create(0);
  const ops = backend.operators;
  const t = (shape, dtype, data) => backend.createTensorHandle({ shape, dtype, data });
  const before = backend.memoryStats();

  // flash_attention(q, k, v, out, scale, isCausal): causal GQA prefill, bf16
  const f = meta.flash;
  const q = t([f.B, f.Hq, f.S, f.D], 'bfloat16', readU16('fq'));
  const k = t([f.B, f.Hkv, f.S, f.D], 'bfloat16', readU16('fk'));
  const v = t([f.B, f.Hkv, f.S, f.D], 'bfloat16', readU16('fv'));
  const o = backend.createTensorHandle([f.B, f.Hq, f.S, f.D], 'bfloat16');
  ops.find('flash_attention')(q, k, v, o, 1 / Math.sqrt(f.D), true);
  write('fo', await o.dataAsync());

  // sdpa_masked with a [Lq, Lk] f32 additive mask broadcast over batch and heads
  const mask = t([f.S, f.S], 'float32', readF32('fmask'));
  const om = backend.createTensorHandle([f.B, f.Hq, f.S, f.D], 'bfloat16');
  ops.find('sdpa_masked')(q, k, v, mask, om, 1 / Math.sqrt(f.D));
  write('fmo', await om.dataAsync());

  // rms_norm of an fp32 residual into bf16, with weight
  const r = meta.norm;
  const x = t([r.rows, r.n], 'float32', readF32('nx'));
  const w = t([r.n], 'bfloat16', readU16('nw'));
  const y = ops.find('rms_norm')([x], { normalizedShape: [r.n], eps: r.eps, weight: w, outDtype: 'bfloat16' });
  write('ny', await y.dataAsync());

  // matmul: out = a @ b^T + 1 * c (linear with a residual), bf16 in, f32 out
  const m = meta.mm;
  const a = t([m.M, m.K], 'bfloat16', readU16('ma'));
  const b = t([m.N, m.K], 'bfloat16', readU16('mb'));
  const c = t([m.M, m.N], 'float32', readF32('mc'));
  const out = backend.createTensorHandle([m.M, m.N], 'float32');
  ops.find('matmul')({ output: out, M: m.M, K: m.K, N: m.N, batchSize: 1, transposeA: false, transposeB: true,
                       alpha: 1, beta: 1, inputC: c }, a, b);
  write('mo', await out.dataAsync());

  // silu_mul, and the iterator kernels silu / mul on a strided (transposed) view
  const g = t([m.M, m.N], 'float32', readF32('mc'));
  const u = backend.createTensorHandle({ shape: [m.M, m.N], dtype: 'float32' });
  ops.find('full')(fullIter(u, 0.5));
  const h = backend.createTensorHandle([m.M, m.N], 'float32');
  ops.find('silu_mul')(g, u, h);
  write('sm', await h.dataAsync());
  const gT = backend.createTensorHandle({ storage: g.storage, shape: [m.N, m.M], dtype: 'float32',
                                          strides: [1, m.N], offset: 0 });
  const s1 = backend.createTensorHandle([m.N, m.M], 'float32');
  ops.find('silu')({ numInputs: 1, output: () => ({ tensorHandle: s1 }), input: () => ({ tensorHandle: gT }) });
  write('st', await s1.dataAsync());
  const prod = backend.createTensorHandle([m.N, m.M], 'float32');
  ops.find('mul')({ numInputs: 2, output: () => ({ tensorHandle: prod }),
                    input: (i) => ({ tensorHandle: i === 0 ? gT : s1 }) });
  write('pt', await prod.dataAsync());

  // index_select (embedding rows) and argmax over the last axis
  const e = meta.emb;
  const table = t([e.V, e.H], 'bfloat16', readU16('et'));
  const ids = t([e.n], 'int32', readI32('ei'));
  const rows = backend.createTensorHandle([e.n, e.H], 'float32');
  ops.find('index_select')(table, ids, { dim: 0 }, rows);
  write('eo', await rows.dataAsync());
  const am = backend.createTensorHandle([m.M], 'int32');
  ops.find('argmax')(HipTensorIterator.reductionOp(c, [-1], false, am));
  write('am', await am.dataAsync());

  // neg / cos / sin (the composite RoPE's iterator kernels) and arange
  const un = {};
  for (const name of ['neg', 'cos', 'sin']) {
    un[name] = backend.createTensorHandle([m.M, m.N], 'float32');
    ops.find(name)({ numInputs: 1, output: () => ({ tensorHandle: un[name] }), input: () => ({ tensorHandle: g }) });
    write('u_' + name, await un[name].dataAsync());
  }
  const ar = backend.createTensorHandle([10], 'float32');
  const arIt = HipTensorIterator.nullaryOp([10], 'float32', ar);
  arIt.setScalarArgs({ start: 0.5, end: 20.5, step: 2 });
  ops.find('arange')(arIt);
  write('ar', await ar.dataAsync());

  // rms_norm_rope into whole KV caches at device positions (the decode-step cache write)
  const p = meta.rope;
  const rq = t([1, p.T, p.Hq, p.D], 'bfloat16', readU16('rq'));
  const rk = t([1, p.T, p.Hkv, p.D], 'bfloat16', readU16('rk'));
  const rv = t([1, p.T, p.Hkv, p.D], 'bfloat16', readU16('rv'));
  const wq = t([p.D], 'bfloat16', readU16('rwq'));
  const wk = t([p.D], 'bfloat16', readU16('rwk'));
  const inv = t([p.D / 2], 'float32', readF32('rinv'));
  const pos = t([p.T], 'int32', readI32('rpos'));
  const kc = backend.createTensorHandle([1, p.Hkv, p.L, p.D], 'bfloat16');
  const vc = backend.createTensorHandle([1, p.Hkv, p.L, p.D], 'bfloat16');
  ops.find('full')(fullIter(kc, 7));
  ops.find('full')(fullIter(vc, 7));
  const qk = ops.find('rms_norm_rope')(rq, rk, { qWeight: wq, kWeight: wk, invFreq: inv, positions: pos, eps: p.eps,
                                                 kOut: kc, v: rv, vOut: vc, cachePositions: true });
  write('rqo', await qk[0].dataAsync());
  write('rkc', await kc.dataAsync());
  write('rvc', await vc.dataAsync());

  // decode_attention: one token per sequence against ragged cache lengths read from the device
  const d = meta.decode;
  const dq = t([d.B, d.Hq, d.D], 'bfloat16', readU16('dq'));
  const dk = t([d.B, d.Hkv, d.L, d.D], 'bfloat16', readU16('dk'));
  const dv = t([d.B, d.Hkv, d.L, d.D], 'bfloat16', readU16('dv'));
  const lens = t([d.B], 'int32', new Int32Array(d.lens));
  const dout = backend.createTensorHandle([d.B, d.Hq, 1, d.D], 'bfloat16');
  ops.find('decode_attention')(dq, dk, dv, lens, dout, 1 / Math.sqrt(d.D));
  write('do', await dout.dataAsync());

  // fused decode / prefill ops, compared bit for bit with the Python binding on the same inputs
  const f2 = meta.fused;
  const gx = t([f2.gvK], 'float32', readF32('gvx'));
  const gw = t([f2.gvN, f2.gvK], 'bfloat16', readU16('gvw'));
  const gn = t([f2.gvK], 'bfloat16', readU16('gvn'));
  const go = backend.createTensorHandle([1, f2.gvN], 'bfloat16');
  ops.find('gemv_fused')('rms_norm', gx, gw, go, { normWeight: gn, eps: 1e-6 });
  write('gvo', await go.dataAsync());
  const gb = t([f2.gvK], 'bfloat16', readU16('gvb'));
  const gc = t([1, f2.gvN], 'float32', readF32('gvc'));
  ops.find('gemv_fused')('none', gb, gw, gc, { cin: gc });
  write('gvr', await gc.dataAsync());

  const gs = backend.createTensorHandle([1, f2.gvN / 2], 'bfloat16');
  ops.find('gemv_swiglu')('rms_norm', gx, gw, gs, { normWeight: gn, eps: 1e-6 });
  write('gvs', await gs.dataAsync());

  const sx = t([f2.swM, f2.swH], 'bfloat16', readU16('swx'));
  const sg = t([2 * f2.swI, f2.swH], 'bfloat16', readU16('swg'));
  const so = backend.createTensorHandle([f2.swM, f2.swI], 'bfloat16');
  ops.find('linear_swiglu')(sx, sg, so);
  write('swo', await so.dataAsync());

  const lx = t([f2.lM, f2.lK], 'bfloat16', readU16('lax'));
  const lw = t([f2.lN, f2.lK], 'bfloat16', readU16('law'));
  const lr = t([f2.lM, f2.lN], 'float32', readF32('lar'));
  const ln = t([f2.lN], 'bfloat16', readU16('lan'));
  const lo = backend.createTensorHandle([f2.lM - 1, f2.lN], 'bfloat16');
  ops.find('linear_add_rms_norm')(lx, lw, lr, ln, 1e-6, lo, [1, f2.lM]);
  write('lao', await lo.dataAsync());
  write('lar2', await lr.dataAsync());

  const d2 = meta.block;
  const bqkv = t([1, (d2.Hq + 2 * d2.Hkv) * 128], 'bfloat16', readU16('bqkv'));
  const bqn = t([128], 'bfloat16', readU16('bqn'));
  const bkn = t([128], 'bfloat16', readU16('bkn'));
  const binv = t([64], 'float32', readF32('binv'));
  const bpos = t([1], 'int32', new Int32Array([d2.pos]));
  const bkc = t([1, d2.Hkv, d2.L, 128], 'bfloat16', readU16('bkc'));
  const bvc = t([1, d2.Hkv, d2.L, 128], 'bfloat16', readU16('bvc'));
  const bwo = t([d2.hidden, d2.Hq * 128], 'bfloat16', readU16('bwo'));
  const bx = t([1, d2.hidden], 'float32', readF32('bx'));
  ops.find('decode_attention_block')(bqkv, { qNorm: bqn, kNorm: bkn, invFreq: binv, eps: 1e-6, position: bpos,
                                             kCache: bkc, vCache: bvc, wO: bwo, x: bx, scale: 1 / Math.sqrt(128) });
  write('bxo', await bx.dataAsync());
  // the prefill QKV projection with qk-norm, RoPE and the cache write (positions run past the cache)
  const qx = t([d2.qS, d2.hidden], 'bfloat16', readU16('qx'));
  const qw = t([(d2.Hq + 2 * d2.Hkv) * 128, d2.hidden], 'bfloat16', readU16('qw'));
  const qpos = t([d2.qS], 'int32', Int32Array.from({ length: d2.qS }, (_, i) => d2.qPos0 + i));
  const qkc = t([1, d2.Hkv, d2.L, 128], 'bfloat16', readU16('bkc'));
  const qvc = t([1, d2.Hkv, d2.L, 128], 'bfloat16', readU16('bvc'));
  const qq = backend.createTensorHandle([1, d2.Hq, d2.qS, 128], 'bfloat16');
  ops.find('linear_qk_norm_rope')(qx, qw, { qWeight: bqn, kWeight: bkn, invFreq: binv, positions: qpos, eps: 1e-6,
                                            qOut: qq, kOut: qkc, vOut: qvc });
  write('qqo', await qq.dataAsync());
  write('qkco', await qkc.dataAsync());
  write('qvco', await qvc.dataAsync());
  write('bkco', await bkc.dataAsync());
  write('bvco', await bvc.dataAsync());

  const lg = t([meta.sample.V], 'float32', readF32('slg'));
  const stok = backend.createTensorHandle([1], 'int32');
  ops.find('sample')(lg, { doSample: false, token: stok });
  const greedyTok = (await stok.dataAsync())[0];
  const sctr = t([1], 'int32', new Int32Array([meta.sample.counter]));
  const slp = backend.createTensorHandle([1], 'float32');
  ops.find('sample')(lg, { doSample: true, temperature: 0.8, topK: 50, topP: 0.9, seed: meta.sample.seed,
                          counter: sctr, token: stok, logprob: slp });
  const sampledTok = (await stok.dataAsync())[0];
  const sampledLp = (await slp.dataAsync())[0];

  const nt = t([1], 'int32', new Int32Array([42]));
  const ps = t([1], 'int32', new Int32Array([5]));
  const sl = t([1], 'int32', new Int32Array([0]));
  const lgg = t([10], 'int32', new Int32Array(10));
  ops.find('greedy_advance')(nt, ps, sl, lgg, 3);
  const adv = { pos: (await ps.dataAsync())[0], len: (await sl.dataAsync())[0], log: Array.from(await lgg.dataAsync()) };

  const cbuf = t([4, 8], 'float32', new Float32Array(32));
  const cview = backend.createTensorHandle({ storage: cbuf.storage, shape: [4, 3], dtype: 'float32', strides: [8, 1],
                                              offset: 2 });
  const csrc = t([4, 3], 'float32', readF32('cps'));
  ops.find('copy_')(HipTensorIterator.unaryOp(csrc, cview));
  write('cpo', await cbuf.dataAsync());
  const zt = t([10], 'float32', new Float32Array(10).fill(1));
  ops.find('zeros')(HipTensorIterator.nullaryOp(zt.shape, zt.dtype, zt));
  const zsum = Array.from(await zt.dataAsync()).reduce((p2, q2) => p2 + Math.abs(q2), 0);

  for (const hnd of [q, k, v, o, mask, om, x, w, y, a, b, c, out, g, u, h, gT, s1, prod, table, ids, rows, am,
                     un.neg, un.cos, un.sin, ar, rq, rk, rv, wq, wk, inv, pos, kc, vc, qk[0], qk[1], dq, dk, dv, lens, dout,
                     gx, gw, gn, go, gs, gb, gc, sx, sg, so, lx, lw, lr, ln, lo, bqkv, bqn, bkn, binv, bpos, bkc, bvc, bwo, bx,
                     qx, qw, qpos, qkc, qvc, qq,
                     lg, stok, sctr, slp, nt, ps, sl, lgg, cbuf, cview, csrc, zt]) {
    hnd.dispose();
  }
  backend.synchronize();
  const after = backend.memoryStats();

  // A storage dropped without dispose(): the garbage collector's finalizer returns its block.
  let gcFreed = null;
  if (typeof global.gc === 'function') {
    const base = backend.memoryStats().liveBytes;
    (() => { backend.createTensorHandle([1 << 20], 'float32'); })();   // 4 MiB, never disposed
    const held = backend.memoryStats().liveBytes - base;
    for (let i = 0; i < 5 && backend.memoryStats().liveBytes > base; ++i) {
      global.gc();
      await new Promise((resolve) => setImmediate(resolve));
    }
    gcFreed = { held, left: backend.memoryStats().liveBytes - base };
  }
  console.log(JSON.stringify({ ok: true, names: ops.names(), liveBefore: before.liveBytes, liveAfter: after.liveBytes,
                                greedyTok, sampledTok, sampledLp, adv, zsum, gcFreed }));
}

main().catch((err) => {
  console.error(err && err.stack ? err.stack : err);
  process.exit(1);
});
