'use strict';
/*
 * iterator_ops.js — the iterator kernels of the TypeScript HipBackend called the way Kandle's
 * dispatcher calls them (register.ts:9: kernel(iter)), with iterators shaped as the dispatcher
 * builds them: plain ITensorIterator objects (types/src/tensor.ts:282-569) whose operands carry
 * element strides aligned to the output shape (0 on broadcast axes, as expand / unsqueeze views
 * give), element offsets (slices), scalar arguments (alpha, fill_value, start/step) and, for a
 * reduction, the kept-axis strides plus reductionStrides.  Then Kandle's composite RoPE
 * (model-utils/src/rope.ts:159-255 forward, :546-644 applyRotaryPosEmbDirect) is run op by op
 * through the registry.  Test infrastructure: tests/test_gpu_node_iterators.py writes the inputs
 * and checks every output.
 *
 * Usage: node iterator_ops.js DIR   (DIR/meta.json holds the shapes; raw little-endian files)
 */
const fs = require('fs');
const path = require('path');
const { HipBackend } = require(path.join(__dirname, '..', '..', 'packages', 'backend-hip', 'dist', 'index.js'));

const dir = process.argv[2];
const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));

function readF32(name) {
  const b = fs.readFileSync(path.join(dir, name));
  return new Float32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.length));
}
function write(name, arr) {
  fs.writeFileSync(path.join(dir, name), Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength));
}

function contiguousStrides(shape) {
  const s = new Array(shape.length).fill(1);
  for (let i = shape.length - 2; i >= 0; --i) s[i] = s[i + 1] * shape[i + 1];
  return s;
}

// An elementwise iterator as TensorIterator.build leaves it: operands [output, ...inputs], each
// {tensorHandle, dtype, shape, strides, offset, isOutput}, strides over outputShape.
function kIter(outShape, outputs, inputs, scalars) {
  const mk = (o, isOutput) => ({ tensorHandle: o.h, dtype: o.h.dtype, shape: o.h.shape,
                                 strides: o.strides || o.h.strides, offset: o.offset === undefined ? o.h.offset : o.offset,
                                 isOutput });
  const ops = outputs.map((o) => mk(o, true)).concat(inputs.map((o) => mk(o, false)));
  const sc = Object.assign({}, scalars || {});
  return {
    inputShape: outShape, outputShape: outShape, outputNumel: outShape.reduce((a, b) => a * b, 1),
    numOutputs: outputs.length, numInputs: inputs.length, isReduction: false, reductionAxes: [],
    output: (i = 0) => ops[i], input: (i = 0) => ops[outputs.length + i], getScalarArgs: () => Object.assign({}, sc),
  };
}

// A reduction iterator as reductionOp leaves it (splitStridesForReduction): the input operand's
// strides cover the kept axes, reductionStrides the reduced ones.
function kReduction(x, axes, keepDims, out) {
  const nd = x.shape.length;
  const red = axes.map((a) => (a < 0 ? a + nd : a)).sort((p, q) => p - q);
  const kept = x.shape.map((_, i) => i).filter((i) => red.indexOf(i) < 0);
  const outShape = keepDims ? x.shape.map((e, i) => (red.indexOf(i) >= 0 ? 1 : e)) : kept.map((i) => x.shape[i]);
  const ops = [
    { tensorHandle: out, dtype: out.dtype, shape: out.shape, strides: out.strides, offset: out.offset, isOutput: true },
    { tensorHandle: x, dtype: x.dtype, shape: x.shape, strides: kept.map((i) => x.strides[i]), offset: x.offset,
      isOutput: false, reductionStrides: red.map((i) => x.strides[i]) },
  ];
  return { inputShape: x.shape, outputShape: outShape, numOutputs: 1, numInputs: 1, isReduction: true,
           reductionAxes: red, reductionShape: red.map((i) => x.shape[i]), keepDims,
           output: (i = 0) => ops[i], input: (i = 0) => ops[1 + i], getScalarArgs: () => ({}) };
}

async function main() {
  const backend = await HipBackend.create(0);
  const ops = backend.operators;
  const before = backend.memoryStats();
  const held = [];
  const t = (shape, dtype, data) => { const h = backend.createTensorHandle({ shape, dtype, data }); held.push(h); return h; };
  const view = (base, shape, strides, offset) => {
    const h = backend.createTensorHandle({ storage: base.storage, shape, dtype: base.dtype, strides, offset });
    held.push(h);
    return h;
  };
  const res = {};

  // 1. binary ops: a permuted view [2,5,4,3] of a [2,3,4,5] buffer; b a [4,1] view (offset 1,
  //    stride 2) of a [10] buffer broadcast over the rest; alpha for add / sub
  const ab = t([2, 3, 4, 5], 'float32', readF32('a'));
  const bb = t([10], 'float32', readF32('b'));
  const av = view(ab, [2, 5, 4, 3], [60, 1, 5, 20], 0);
  const bv = view(bb, [4, 1], [2, 1], 1);
  const oshape = [2, 5, 4, 3];
  for (const [name, sc] of [['add', { alpha: 2 }], ['sub', { alpha: 0.5 }], ['mul', {}], ['div', {}]]) {
    const out = t(oshape, 'float32');
    ops.find(name)(kIter(oshape, [{ h: out }], [{ h: av }, { h: bv, strides: [0, 0, 2, 0] }], sc));
    write('bin_' + name, await out.dataAsync());
  }

  // 2. copy family: casts, contiguous of a permuted view, clone, copy_ into a strided window
  const x = t([6, 10], 'float32', readF32('x'));
  for (const dt of ['bfloat16', 'int32', 'int64']) {
    const o = t([6, 10], dt);
    ops.find('cast')(kIter([6, 10], [{ h: o }], [{ h: x }]));
    const d = await o.dataAsync();
    write('cast_' + dt, dt === 'int64' ? BigInt64Array.from(d) : d);
  }
  const xT = view(x, [10, 6], [1, 10], 0);
  const oc = t([10, 6], 'float32');
  ops.find('contiguous')(kIter([10, 6], [{ h: oc }], [{ h: xT }]));
  write('contig', await oc.dataAsync());
  const ocl = t([6, 10], 'float32');
  ops.find('clone')(kIter([6, 10], [{ h: ocl }], [{ h: x }]));
  write('clone', await ocl.dataAsync());
  const buf = t([8, 16], 'float32', new Float32Array(128).fill(-7));
  const win = view(buf, [6, 10], [16, 1], 17);
  ops.find('copy_')(kIter([6, 10], [{ h: win }], [{ h: x }]));
  write('win1', await buf.dataAsync());
  const row = t([10], 'float32', Float32Array.from({ length: 10 }, (_, i) => i));
  ops.find('copy_')(kIter([6, 10], [{ h: win }], [{ h: row, strides: [0, 1] }]));
  write('win2', await buf.dataAsync());

  // 3. factories (handlers/factory.ts:50-61: fill_value or fillValue; arangeExecutor.ts:37-44)
  const fz = t([3, 5], 'float32', new Float32Array(15).fill(9));
  ops.find('zeros')(kIter([3, 5], [{ h: fz }], []));
  const fo = t([3, 5], 'float32');
  ops.find('ones')(kIter([3, 5], [{ h: fo }], []));
  const ff = t([3, 5], 'bfloat16');
  ops.find('full')(kIter([3, 5], [{ h: ff }], [], { fill_value: -2.5 }));
  const ff2 = t([3, 5], 'int32');
  ops.find('full')(kIter([3, 5], [{ h: ff2 }], [], { fillValue: 11 }));
  const fe = t([3, 5], 'float32', new Float32Array(15).fill(4));
  ops.find('empty')(kIter([3, 5], [{ h: fe }], []));
  res.factories = {
    zeros: Array.from(await fz.dataAsync()), ones: Array.from(await fo.dataAsync()),
    full: Array.from(await ff.dataAsync()), fullInt: Array.from(await ff2.dataAsync()),
  };
  const ar = t([1000], 'float32');
  ops.find('arange')(kIter([1000], [{ h: ar }], [], { start: 0.5, end: 250.5, step: 0.25 }));
  write('arange_f32', await ar.dataAsync());
  const ari = t([100], 'int32');
  ops.find('arange')(kIter([100], [{ h: ari }], [], { start: -7, end: 293, step: 3 }));
  write('arange_i32', await ari.dataAsync());

  // 4. argmax over any axes of a permuted [5, 7, 300] view of a [300, 7, 5] buffer
  const rb = t([300, 7, 5], 'float32', readF32('r'));
  const rv = view(rb, [5, 7, 300], [1, 5, 35], 0);
  for (const [tag, axes, keep, dt] of meta.argmax) {
    const nd = 3;
    const red = axes.map((a) => (a < 0 ? a + nd : a));
    const oshp = keep ? rv.shape.map((e, i) => (red.indexOf(i) >= 0 ? 1 : e)) : rv.shape.filter((_, i) => red.indexOf(i) < 0);
    const o = t(oshp, dt);
    ops.find('argmax')(kReduction(rv, axes, keep, o));
    const d = await o.dataAsync();
    write('am_' + tag, dt === 'int64' ? BigInt64Array.from(d) : d);
  }

  // 5. Kandle's composite RoPE op by op: cos/sin from arange positions and inv_freq (rope.ts:
  //    193-255), then q * cos + rotate_half(q) * sin (rope.ts:546-644) on heads-first q, a
  //    transposed view of a [1, T, H, D] buffer (q.transpose(1, 2))
  const { T, H, D } = meta.rope;
  const hd = D / 2;
  const pos = t([T], 'float32');
  ops.find('arange')(kIter([T], [{ h: pos }], [], { start: 0, end: T, step: 1 }));
  const inv = t([hd], 'float32', readF32('inv'));
  // unsqueeze(-1) + expand and unsqueeze(0) + expand: stride-0 views
  const posE = view(pos, [T, hd], [1, 0], 0);
  const invE = view(inv, [T, hd], [0, 1], 0);
  const freqs = t([T, hd], 'float32');
  ops.find('mul')(kIter([T, hd], [{ h: freqs }], [{ h: posE }, { h: invE }]));
  // emb = cat([freqs, freqs], -1): copies into the two halves
  const emb = t([T, D], 'float32');
  for (const off of [0, hd]) ops.find('copy_')(kIter([T, hd], [{ h: view(emb, [T, hd], [D, 1], off) }], [{ h: freqs }]));
  const cosT = t([T, D], 'float32');
  const sinT = t([T, D], 'float32');
  ops.find('cos')(kIter([T, D], [{ h: cosT }], [{ h: emb }]));
  ops.find('sin')(kIter([T, D], [{ h: sinT }], [{ h: emb }]));
  const xq = t([1, T, H, D], 'float32', readF32('q'));
  const q = view(xq, [1, H, T, D], [T * H * D, D, H * D, 1], 0);
  const shp = [1, H, T, D];
  const half = [1, H, T, hd];
  // rotate_half: contiguous slices, neg, cat(-x2, x1)
  const x1 = t(half, 'float32');
  const x2 = t(half, 'float32');
  ops.find('contiguous')(kIter(half, [{ h: x1 }], [{ h: view(xq, half, q.strides, 0) }]));
  ops.find('contiguous')(kIter(half, [{ h: x2 }], [{ h: view(xq, half, q.strides, hd) }]));
  const nx2 = t(half, 'float32');
  ops.find('neg')(kIter(half, [{ h: nx2 }], [{ h: x2 }]));
  const rot = t(shp, 'float32');
  const rs = contiguousStrides(shp);
  ops.find('copy_')(kIter(half, [{ h: view(rot, half, rs, 0) }], [{ h: nx2 }]));
  ops.find('copy_')(kIter(half, [{ h: view(rot, half, rs, hd) }], [{ h: x1 }]));
  // cos / sin unsqueezed twice to [1, 1, T, D] and broadcast over heads
  const cosE = view(cosT, [1, 1, T, D], [T * D, T * D, D, 1], 0);
  const sinE = view(sinT, [1, 1, T, D], [T * D, T * D, D, 1], 0);
  const qc = t(shp, 'float32');
  const rsn = t(shp, 'float32');
  const qr = t(shp, 'float32');
  ops.find('mul')(kIter(shp, [{ h: qc }], [{ h: q }, { h: cosE, strides: [0, 0, D, 1] }]));
  ops.find('mul')(kIter(shp, [{ h: rsn }], [{ h: rot }, { h: sinE, strides: [0, 0, D, 1] }]));
  ops.find('add')(kIter(shp, [{ h: qr }], [{ h: qc }, { h: rsn }]));
  write('rope_composite', await qr.dataAsync());
  // the fused kernel on the same rows (unit weights; the rows have unit RMS already)
  const ones = t([D], 'float32', new Float32Array(D).fill(1));
  const ipos = t([T], 'int32', Int32Array.from({ length: T }, (_, i) => i));
  const fused = ops.find('rms_norm_rope')(xq, xq, { qWeight: ones, kWeight: ones, invFreq: inv, positions: ipos, eps: 1e-6 });
  held.push(fused[0], fused[1]);
  write('rope_fused', await fused[0].dataAsync());

  for (const h of held) h.dispose();
  backend.synchronize();
  const after = backend.memoryStats();
  res.ok = true;
  res.liveBefore = before.liveBytes;
  res.liveAfter = after.liveBytes;
  console.log(JSON.stringify(res));
}

main().catch((err) => {
  console.error(err && err.stack ? err.stack : err);
  process.exit(1);
});
