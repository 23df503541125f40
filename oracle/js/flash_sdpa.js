'use strict';
/*
 * flash_sdpa.js — JavaScript restatement of Kandle's flash-attention kernel math, used ONLY as test
 * infrastructure: as bench.py's CPU baseline (the reference's "pure-JS CPU backend" does not exist,
 * README.md:1043,1245) and as a checker in tests/.  Node 12 compatible (no optional chaining).
 *
 * Follows packages/backend-webgpu/src/kernels/attention/builder.ts:138-329 and
 * packages/backend-webgpu/src/kernels/attention/types.ts:69-122 (D = 128 -> Br = 8, Bc = 4):
 *   per (batch, query head) and block of Br query rows, walk key blocks of Bc keys up to the end
 *   of the query block when causal (:196-203); score = (q . k) * scale (:253-256); causal
 *   key j > query i gets -1e20 (:247-249); online softmax with running max m and sum l per row
 *   (:270-311); O = acc / l (:319-329); query head h reads kv head floor(h / (Hq / Hkv)) (:143).
 * Storage is float32 (Float32Array); arithmetic is JavaScript's double precision, as a JS backend
 * computes.
 *
 * Usage: node flash_sdpa.js DIR B Hq Hkv Lq Lk D scale causal headsLimit
 *   reads DIR/q.f32, DIR/k.f32, DIR/v.f32 (contiguous [B,H,L,D]), writes DIR/o.f32 and prints
 *   {"ms": wall milliseconds of the computation, "heads": (batch, head) pairs computed}.
 */
const fs = require('fs');
const path = require('path');

function flashSdpa(q, k, v, o, B, Hq, Hkv, Lq, Lk, D, scale, causal, headsLimit) {
  const G = Hq / Hkv;
  const Br = 8;
  const Bc = 4;
  const mRow = new Float64Array(Br);
  const lRow = new Float64Array(Br);
  const acc = new Float64Array(Br * D);
  const sTile = new Float64Array(Br * Bc);
  let heads = 0;
  for (let b = 0; b < B; b++) {
    for (let h = 0; h < Hq; h++) {
      if (headsLimit > 0 && heads >= headsLimit) return heads;
      heads++;
      const hk = Math.floor(h / G);
      const qb = (b * Hq + h) * Lq * D;
      const kb = (b * Hkv + hk) * Lk * D;
      for (let i0 = 0; i0 < Lq; i0 += Br) {
        const rows = Math.min(Br, Lq - i0);
        mRow.fill(-Infinity);
        lRow.fill(0);
        acc.fill(0);
        const kvEnd = causal ? Math.min(Lk, i0 + Br) : Lk;
        for (let j0 = 0; j0 < kvEnd; j0 += Bc) {
          const cols = Math.min(Bc, Lk - j0);
          for (let r = 0; r < rows; r++) {
            const qi = qb + (i0 + r) * D;
            let mNew = mRow[r];
            for (let c = 0; c < cols; c++) {
              const kj = kb + (j0 + c) * D;
              let dot = 0;
              for (let d = 0; d < D; d++) dot += q[qi + d] * k[kj + d];
              let s = dot * scale;
              if (causal && j0 + c > i0 + r) s = -1e20;
              sTile[r * Bc + c] = s;
              if (s > mNew) mNew = s;
            }
            const alpha = Math.exp(mRow[r] - mNew);
            let lNew = lRow[r] * alpha;
            const ar = r * D;
            for (let d = 0; d < D; d++) acc[ar + d] *= alpha;
            for (let c = 0; c < cols; c++) {
              const p = Math.exp(sTile[r * Bc + c] - mNew);
              lNew += p;
              const vj = kb + (j0 + c) * D;
              for (let d = 0; d < D; d++) acc[ar + d] += p * v[vj + d];
            }
            mRow[r] = mNew;
            lRow[r] = lNew;
          }
        }
        for (let r = 0; r < rows; r++) {
          const oi = qb + (i0 + r) * D;
          for (let d = 0; d < D; d++) o[oi + d] = acc[r * D + d] / lRow[r];
        }
      }
    }
  }
  return heads;
}

function readF32(file) {
  const buf = fs.readFileSync(file);
  return new Float32Array(buf.buffer, buf.byteOffset, buf.byteLength / 4);
}

function main() {
  const a = process.argv.slice(2);
  if (a.length !== 10) {
    process.stderr.write('usage: node flash_sdpa.js DIR B Hq Hkv Lq Lk D scale causal headsLimit\n');
    process.exit(2);
  }
  const dir = a[0];
  const [B, Hq, Hkv, Lq, Lk, D] = a.slice(1, 7).map(Number);
  const scale = Number(a[7]);
  const causal = a[8] === '1';
  const headsLimit = Number(a[9]);
  const q = readF32(path.join(dir, 'q.f32'));
  const k = readF32(path.join(dir, 'k.f32'));
  const v = readF32(path.join(dir, 'v.f32'));
  const o = new Float32Array(B * Hq * Lq * D);
  const t0 = process.hrtime();
  const heads = flashSdpa(q, k, v, o, B, Hq, Hkv, Lq, Lk, D, scale, causal, headsLimit);
  const dt = process.hrtime(t0);
  fs.writeFileSync(path.join(dir, 'o.f32'), Buffer.from(o.buffer));
  process.stdout.write(JSON.stringify({ ms: dt[0] * 1e3 + dt[1] / 1e6, heads: heads }) + '\n');
}

if (require.main === module) main();
module.exports = { flashSdpa };
