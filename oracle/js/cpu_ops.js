'use strict';
/*
 * cpu_ops.js — JavaScript restatement of the reference's RMSNorm and rotary-embedding math, used ONLY
 * as test infrastructure: bench.py's CPU baseline for config C2 (the reference's "pure-JS CPU
 * backend" does not exist, README.md:1043,1245) and a checker in tests/.  Node 12 compatible.
 *
 * Storage is float32 (Float32Array, every op's output rounded to float32 as a tensor op stores it);
 * arithmetic is JavaScript's double precision, as a JS backend computes.
 *
 * rmsNorm follows packages/backend-webgpu/src/kernels/normalize/shaderBuilder.ts:394-411:
 *   sum_sq = sum x^2; rms = sqrt(sum_sq / N + eps); y = x * (1 / rms) * w[i].
 * qkNormRope follows packages/model-utils/src/attention/gqa.ts:279-309 (per-head q_norm / k_norm,
 * an RMSNorm over head_dim) then packages/model-utils/src/rope.ts:
 *   inv_freq[i] = f32(1 / theta^(i / (D/2)))          (:159-171)
 *   freqs = f32(position * inv_freq[i])                 (:226, a float32 mul)
 *   emb = cat(freqs, freqs); cos = f32(cos(emb)), sin = f32(sin(emb))   (:251-255)
 *   x' = x cos + rotate_half(x) sin, rotate_half(x) = cat(-x2, x1)     (:590-630)
 */

const f32 = Math.fround;

function rmsNorm(x, xOff, w, y, yOff, rows, n, eps) {
  for (let r = 0; r < rows; r++) {
    const xb = xOff + r * n;
    const yb = yOff + r * n;
    let ss = 0;
    for (let i = 0; i < n; i++) {
      const v = x[xb + i];
      ss += v * v;
    }
    const scale = 1 / Math.sqrt(ss / n + eps);
    for (let i = 0; i < n; i++) {
      const nv = f32(x[xb + i] * scale);
      y[yb + i] = w ? nv * w[i] : nv;
    }
  }
}

function ropeInvFreq(D, theta) {
  const half = D / 2;
  const inv = new Float32Array(half);
  for (let i = 0; i < half; i++) inv[i] = 1.0 / Math.pow(theta, i / half);
  return inv;
}

// cos / sin tables [T, D] of the composite (emb = cat(freqs, freqs)), float32.
function ropeTables(positions, invFreq, D) {
  const T = positions.length;
  const half = D / 2;
  const cos = new Float32Array(T * D);
  const sin = new Float32Array(T * D);
  for (let t = 0; t < T; t++) {
    for (let i = 0; i < half; i++) {
      const f = f32(positions[t] * invFreq[i]);
      const c = Math.cos(f);
      const s = Math.sin(f);
      cos[t * D + i] = c;
      cos[t * D + half + i] = c;
      sin[t * D + i] = s;
      sin[t * D + half + i] = s;
    }
  }
  return { cos: cos, sin: sin };
}

// x [T, H, D] (token-major, as the projection stores it) -> out [T, H, D]: per-head RMSNorm with
// weight w [D], then RoPE at positions[t] with the tables.
function qkNormRope(x, w, out, T, H, D, tables, eps) {
  const half = D / 2;
  const n = new Float32Array(D);
  for (let t = 0; t < T; t++) {
    const cb = t * D;
    for (let h = 0; h < H; h++) {
      const base = (t * H + h) * D;
      rmsNorm(x, base, w, n, 0, 1, D, eps);
      for (let i = 0; i < D; i++) {
        const rot = i < half ? f32(-n[i + half]) : n[i - half];
        out[base + i] = f32(n[i] * tables.cos[cb + i]) + f32(rot * tables.sin[cb + i]);
      }
    }
  }
}

module.exports = { rmsNorm: rmsNorm, ropeInvFreq: ropeInvFreq, ropeTables: ropeTables, qkNormRope: qkNormRope };
