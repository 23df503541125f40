'use strict';
/*
 * addon_ops.js — drives the HIP kernels from Node through packages/backend-hip/native/kandle_hip.node
 * (test infrastructure: tests/test_gpu_node_addon.py writes the inputs and checks the outputs).
 *
 * Usage: node addon_ops.js DIR
 *   DIR/meta.json {"flash": {B, Hq, Hkv, S, D, causal}, "decode": {B, Hq, Hkv, D, ML, lens}};
 *   bf16 inputs as raw uint16 files: fq, fk, fv, dq, dk, dv; writes fo, do (bf16) and prints
 *   {"ok": true, "allocs": allocStats}.
 */
const fs = require('fs');
const path = require('path');
const hip = require(path.join(__dirname, '..', '..', 'packages', 'backend-hip', 'native', 'kandle_hip.node'));

const dir = process.argv[2];
const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));

function upload(name) {
  const host = fs.readFileSync(path.join(dir, name));
  const ptr = hip.alloc(host.length);
  hip.memcpyH2D(ptr, host);
  return ptr;
}
function download(ptr, bytes, name) {
  const host = new Uint8Array(bytes);
  hip.memcpyD2H(host, ptr);
  fs.writeFileSync(path.join(dir, name), host);
}
// contiguous [b, h, l, d] element strides of (batch, head, seq)
function bhl(H, L, D) { return [H * L * D, L * D, D]; }

hip.init(0);

// flash_attention(q, k, v, out, scale, isCausal) — register.ts:102-109, shapes from the handles
const f = meta.flash;
const fq = upload('fq'), fk = upload('fk'), fv = upload('fv');
const foBytes = f.B * f.Hq * f.S * f.D * 2;
const fo = hip.alloc(foBytes);
const st = [].concat(bhl(f.Hq, f.S, f.D), bhl(f.Hkv, f.S, f.D), bhl(f.Hkv, f.S, f.D), bhl(f.Hq, f.S, f.D));
hip.flashAttention(fq, fk, fv, fo, f.B, f.Hq, f.Hkv, f.S, f.S, f.D, st, 1 / Math.sqrt(f.D), f.causal, hip.BF16);
download(fo, foBytes, 'fo');

// decode attention over [B, Hkv, ML, D] caches with per-sequence lengths
const d = meta.decode;
const dq = upload('dq'), dk = upload('dk'), dv = upload('dv');
const lens = new Int32Array(d.lens);
const dl = hip.alloc(lens.byteLength);
hip.memcpyH2D(dl, lens);
const doBytes = d.B * d.Hq * d.D * 2;
const dout = hip.alloc(doBytes);
const cst = [d.Hkv * d.ML * d.D, d.ML * d.D, d.D];
const dst = [d.Hq * d.D, d.D].concat(cst, cst, [d.Hq * d.D, d.D]);
hip.decodeAttention(dq, dk, dv, dout, dl, d.B, d.Hq, d.Hkv, d.D, d.ML, dst, 1 / Math.sqrt(d.D), hip.BF16);
download(dout, doBytes, 'do');

let threw = '';
try {
  hip.flashAttention(fq, fk, fv, fo, f.B, f.Hq, 3, f.S, f.S, f.D, st, 0.1, true, hip.BF16);
} catch (e) {
  threw = e.message;
}
for (const p of [fq, fk, fv, fo, dq, dk, dv, dl, dout]) hip.free(p);
hip.synchronize();
process.stdout.write(JSON.stringify({ ok: true, gqaError: threw, allocs: hip.allocStats() }) + '\n');
