'use strict';
/*
 * qwen3_cpu.js — JavaScript restatement of the Qwen3 causal-LM forward, used ONLY as test
 * infrastructure: bench.py's CPU baseline for config C5 (the reference's "pure-JS CPU backend" does
 * not exist, README.md:1043,1245) and, on a tiny configuration, checked against the numpy oracle
 * (oracle/qwen3.py with exact=True) in tests/test_oracle_js.py.  Node 12 compatible.
 *
 * Module order of the reference: Qwen3Model.forwardWithLayerOutputs (packages/model-utils/src/
 * qwen3/model.ts:265-347), Qwen3DecoderLayer.forward (qwen3/decoder_layer.ts:191-241),
 * GroupedQueryAttention.forward (attention/gqa.ts:246-430: q/k/v projections, per-head q_norm /
 * k_norm, RoPE, KV-cache update, SDPA with causal off for a single new token, o_proj), SwiGLUMLP
 * (mlp/swiglu.ts:119-134: silu(x) = x / (1 + exp(-clamp(x, -88, 88)))), tied lm_head
 * (qwen3/for_causal_lm.ts:121-125, 184-185).  Storage float32, arithmetic JavaScript doubles, as a
 * JS backend computes; weights are float32 arrays (bf16 checkpoints widened exactly, as the
 * reference's loader does).
 */

const flash = require('./flash_sdpa.js');
const ops = require('./cpu_ops.js');

const f32 = Math.fround;

// y[s, n] = sum_k x[s, k] w[n, k] (x [S, K], w [N, K] row-major; nn.Linear without bias), four rows
// of x at a time so that each weight row is read once per block.
function linear(x, S, K, w, N, y) {
  let s = 0;
  for (; s + 4 <= S; s += 4) {
    const x0 = s * K, x1 = x0 + K, x2 = x1 + K, x3 = x2 + K;
    for (let n = 0; n < N; n++) {
      const wb = n * K;
      let a0 = 0, a1 = 0, a2 = 0, a3 = 0;
      for (let k = 0; k < K; k++) {
        const wv = w[wb + k];
        a0 += x[x0 + k] * wv;
        a1 += x[x1 + k] * wv;
        a2 += x[x2 + k] * wv;
        a3 += x[x3 + k] * wv;
      }
      y[s * N + n] = a0;
      y[(s + 1) * N + n] = a1;
      y[(s + 2) * N + n] = a2;
      y[(s + 3) * N + n] = a3;
    }
  }
  for (; s < S; s++) {
    const xb = s * K;
    for (let n = 0; n < N; n++) {
      const wb = n * K;
      let a = 0;
      for (let k = 0; k < K; k++) a += x[xb + k] * w[wb + k];
      y[s * N + n] = a;
    }
  }
}

class Qwen3Cpu {
  // cfg: {vocabSize, hiddenSize, intermediateSize, numHiddenLayers, numAttentionHeads,
  // numKeyValueHeads, headDim, rmsNormEps, ropeTheta}; w: Hugging Face tensor name -> Float32Array.
  constructor(cfg, w, maxSeqLen) {
    this.cfg = cfg;
    this.maxSeqLen = maxSeqLen;
    const get = (n) => {
      if (w[n] === undefined) throw new Error('Qwen3Cpu: missing weight ' + n);
      return w[n];
    };
    this.embed = get('model.embed_tokens.weight');
    this.finalNorm = get('model.norm.weight');
    this.layers = [];
    const Hkv = cfg.numKeyValueHeads, D = cfg.headDim;
    for (let i = 0; i < cfg.numHiddenLayers; i++) {
      const p = 'model.layers.' + i + '.';
      this.layers.push({
        inNorm: get(p + 'input_layernorm.weight'), q: get(p + 'self_attn.q_proj.weight'),
        k: get(p + 'self_attn.k_proj.weight'), v: get(p + 'self_attn.v_proj.weight'),
        o: get(p + 'self_attn.o_proj.weight'), qNorm: get(p + 'self_attn.q_norm.weight'),
        kNorm: get(p + 'self_attn.k_norm.weight'), postNorm: get(p + 'post_attention_layernorm.weight'),
        gate: get(p + 'mlp.gate_proj.weight'), up: get(p + 'mlp.up_proj.weight'), down: get(p + 'mlp.down_proj.weight'),
        kCache: new Float32Array(Hkv * maxSeqLen * D), vCache: new Float32Array(Hkv * maxSeqLen * D),
      });
    }
    this.invFreq = ops.ropeInvFreq(D, cfg.ropeTheta);
  }

  // float32 logits [vocab] of the last position after appending ids at cache rows [pos, pos + S).
  forward(ids, pos) {
    const c = this.cfg;
    const S = ids.length, Hd = c.hiddenSize, I = c.intermediateSize, Hq = c.numAttentionHeads;
    const Hkv = c.numKeyValueHeads, D = c.headDim, eps = c.rmsNormEps, end = pos + S, M = this.maxSeqLen;
    if (end > M) throw new Error('Qwen3Cpu: ' + end + ' positions for a cache of ' + M);
    const x = new Float32Array(S * Hd);
    for (let s = 0; s < S; s++) x.set(this.embed.subarray(ids[s] * Hd, (ids[s] + 1) * Hd), s * Hd);
    const positions = new Int32Array(S);
    for (let s = 0; s < S; s++) positions[s] = pos + s;
    const tables = ops.ropeTables(positions, this.invFreq, D);
    const h = new Float32Array(S * Hd);
    const q = new Float32Array(S * Hq * D), k = new Float32Array(S * Hkv * D), v = new Float32Array(S * Hkv * D);
    const qr = new Float32Array(S * Hq * D), kr = new Float32Array(S * Hkv * D);
    const qh = new Float32Array(Hq * S * D), att = new Float32Array(Hq * S * D), o = new Float32Array(S * Hq * D);
    const kw = new Float32Array(Hkv * end * D), vw = new Float32Array(Hkv * end * D);
    const proj = new Float32Array(S * Hd);
    const g = new Float32Array(S * I), u = new Float32Array(S * I);
    for (const L of this.layers) {
      ops.rmsNorm(x, 0, L.inNorm, h, 0, S, Hd, eps);
      linear(h, S, Hd, L.q, Hq * D, q);
      linear(h, S, Hd, L.k, Hkv * D, k);
      linear(h, S, Hd, L.v, Hkv * D, v);
      ops.qkNormRope(q, L.qNorm, qr, S, Hq, D, tables, eps);
      ops.qkNormRope(k, L.kNorm, kr, S, Hkv, D, tables, eps);
      // K/V cache rows [pos, end) (StaticKVCache.update, kv-cache.ts:164-212), [Hkv, M, D]
      for (let s = 0; s < S; s++) {
        for (let hh = 0; hh < Hkv; hh++) {
          const src = (s * Hkv + hh) * D, dst = (hh * M + pos + s) * D;
          L.kCache.set(kr.subarray(src, src + D), dst);
          L.vCache.set(v.subarray(src, src + D), dst);
        }
      }
      // heads-first q [Hq, S, D] and the attended cache window [Hkv, end, D]
      for (let s = 0; s < S; s++) {
        for (let hh = 0; hh < Hq; hh++) qh.set(qr.subarray((s * Hq + hh) * D, (s * Hq + hh + 1) * D), (hh * S + s) * D);
      }
      for (let hh = 0; hh < Hkv; hh++) {
        kw.set(L.kCache.subarray(hh * M * D, (hh * M + end) * D), hh * end * D);
        vw.set(L.vCache.subarray(hh * M * D, (hh * M + end) * D), hh * end * D);
      }
      flash.flashSdpa(qh, kw, vw, att, 1, Hq, Hkv, S, end, D, 1 / Math.sqrt(D), S > 1, 0);
      for (let s = 0; s < S; s++) {
        for (let hh = 0; hh < Hq; hh++) o.set(att.subarray((hh * S + s) * D, (hh * S + s + 1) * D), (s * Hq + hh) * D);
      }
      linear(o, S, Hq * D, L.o, Hd, proj);
      for (let i = 0; i < S * Hd; i++) x[i] = x[i] + proj[i];
      ops.rmsNorm(x, 0, L.postNorm, h, 0, S, Hd, eps);
      linear(h, S, Hd, L.gate, I, g);
      linear(h, S, Hd, L.up, I, u);
      for (let i = 0; i < S * I; i++) {
        const gv = g[i];
        const cl = gv < -88 ? -88 : (gv > 88 ? 88 : gv);
        g[i] = (gv / (1 + Math.exp(-cl))) * u[i];
      }
      linear(g, S, I, L.down, Hd, proj);
      for (let i = 0; i < S * Hd; i++) x[i] = x[i] + proj[i];
    }
    const last = new Float32Array(Hd);
    ops.rmsNorm(x, (S - 1) * Hd, this.finalNorm, last, 0, 1, Hd, eps);
    return this.lmHead(last);
  }

  // logits = embed h (the tied lm_head over one normalised row)
  lmHead(row) {
    const out = new Float32Array(this.cfg.vocabSize);
    linear(row, 1, this.cfg.hiddenSize, this.embed, this.cfg.vocabSize, out);
    return out;
  }
}

function argmax(a) {
  let best = 0;
  for (let i = 1; i < a.length; i++) if (a[i] > a[best]) best = i;
  return best;
}

module.exports = { Qwen3Cpu: Qwen3Cpu, linear: linear, argmax: argmax, f32: f32 };
