// Qwen3 causal LM on the HIP backend, host side in TypeScript: the caller of the hot path, written
// against the backend's operator registry the way Kandle's model code reaches its kernels
// (packages/model-utils/src/qwen3/{model,decoder_layer,for_causal_lm}.ts, attention/gqa.ts,
// mlp/swiglu.ts).  It runs the same launches, in the same order, as the Python mirror
// (kandle_amd/model_utils/qwen3.py), so both produce the same logits bit for bit:
//
//   prefill of S tokens (pre-norm decoder layers, decoder_layer.ts:191-241)
//     x = embed[ids] (fp32 residual stream), h = rms_norm(x, input_layernorm) (activation dtype)
//     per layer: qkv = h W_qkv^T (q/k/v rows concatenated); q/k per-head RMSNorm + RoPE, q written
//       heads-first, k and v written into the KV caches at their positions (rms_norm_rope);
//       o = causal flash attention over the cache rows [0, S); x += o W_o^T and h = rms_norm(x,
//       post_attention_layernorm) (linear_add_rms_norm); a = silu(h W_gate^T) * (h W_up^T)
//       (linear_swiglu, gate/up interleaved in blocks of 8 rows); x += a W_down^T and h = the next
//       layer's input norm of x (the final norm of the last row after the last layer)
//     logits = h E^T in fp32 with the tied embedding E (for_causal_lm.ts:121-125, 184-185)
//   decode step of one token at device position p (greedy loop, for_causal_lm.ts:475-508)
//     x = embed[token]; per layer: qkv = rms_norm(x) W_qkv^T (gemv_fused); the attention block
//       (decode_attention_block: qk-norm, RoPE, K/V cache write at p, attention over rows [0, p],
//       o_proj, residual add; head_dim 128 -- other head dims run rms_norm_rope, decode_attention
//       and the o_proj gemv_fused); a = silu * mul of rms_norm(x) through the gate/up weight
//       (gemv_swiglu); x += a W_down^T (gemv_fused)
//     logits = rms_norm(x) E^T; token = argmax (lowest index); greedy_advance moves p on.
//
// Activations other than x (h, q/k/v, the K/V caches, attention output, the SwiGLU product) are
// stored in the model's activation dtype: 'float32' (the default; every op in fp32 as the
// reference computes, its bf16 checkpoint widened to float32 on load, io/safetensor/dtypes.ts:17-31:
// the weights stay bf16 and the kernels multiply fp32 activations by them) or 'bfloat16' (rounded to
// bf16 at each store: the fastest path).

const fs = require('fs');
const path = require('path');
const { performance } = require('perf_hooks');  // wall times in ms, sub-millisecond resolution
// the iterators Kandle's dispatcher builds for the factory, copy and reduction kernels
const { HipTensorIterator } = require(path.join(__dirname, 'index.js'));

export interface Qwen3Config {
  vocabSize: number;
  hiddenSize: number;
  intermediateSize: number;
  numHiddenLayers: number;
  numAttentionHeads: number;
  numKeyValueHeads: number;
  headDim: number;
  rmsNormEps: number;
  ropeTheta: number;
}

export interface SafeTensor {
  dtype: string;
  shape: number[];
  bytes: Buffer;
}

// A .safetensors file: an 8-byte little-endian header length n, n bytes of JSON mapping each tensor
// name to {dtype, shape, data_offsets: [begin, end]} (offsets into the data after the header), then
// the data (the format Kandle's io/safetensor/parser.ts reads).
export function readSafetensors(file: string): { [name: string]: SafeTensor } {
  const buf: Buffer = fs.readFileSync(file);
  if (buf.length < 8) throw new Error(`${file}: not a safetensors file (shorter than its header length)`);
  const n = Number(buf.readBigUInt64LE(0));
  if (n <= 0 || 8 + n > buf.length) throw new Error(`${file}: header length ${n} outside the file`);
  const header = JSON.parse(buf.slice(8, 8 + n).toString('utf8'));
  const out: { [name: string]: SafeTensor } = {};
  for (const name of Object.keys(header)) {
    if (name === '__metadata__') continue;
    const e = header[name];
    const b = 8 + n + e.data_offsets[0];
    const end = 8 + n + e.data_offsets[1];
    if (end > buf.length || b > end) throw new Error(`${file}: ${name} data outside the file`);
    out[name] = { dtype: e.dtype, shape: e.shape, bytes: buf.slice(b, end) };
  }
  return out;
}

// bf16 bit patterns of a BF16 tensor (copied: the file's data need not be 2-byte aligned).
function bf16Bits(t: SafeTensor, name: string): Uint16Array {
  if (t.dtype !== 'BF16') throw new Error(`${name}: BF16 expected, the file holds ${t.dtype}`);
  const ab = t.bytes.buffer.slice(t.bytes.byteOffset, t.bytes.byteOffset + t.bytes.length);
  return new Uint16Array(ab);
}

// bf16 bit patterns widened exactly to float32 (the reference's BF16 load, dtypes.ts:82-94).
function widenBf16(bits: Uint16Array): Float32Array {
  const u = new Uint32Array(bits.length);
  for (let i = 0; i < bits.length; ++i) u[i] = bits[i] << 16;
  return new Float32Array(u.buffer);
}

function concatRows(parts: Uint16Array[]): Uint16Array {
  const out = new Uint16Array(parts.reduce((s: number, p: Uint16Array) => s + p.length, 0));
  let off = 0;
  for (const p of parts) {
    out.set(p, off);
    off += p.length;
  }
  return out;
}

// The gate/up weight of the fused SwiGLU kernels: rows 16i .. 16i + 7 are gate rows 8i .. 8i + 7 and
// rows 16i + 8 .. 16i + 15 the matching up rows (gate and up [I, H], I % 8 == 0).
function interleaveGateUp(gate: Uint16Array, up: Uint16Array, I: number, H: number): Uint16Array {
  if (I % 8 !== 0) throw new Error('interleaveGateUp: the intermediate size must be a multiple of 8');
  const out = new Uint16Array(2 * I * H);
  for (let blk = 0; blk < I / 8; ++blk) {
    out.set(gate.subarray(8 * blk * H, 8 * (blk + 1) * H), 16 * blk * H);
    out.set(up.subarray(8 * blk * H, 8 * (blk + 1) * H), (16 * blk + 8) * H);
  }
  return out;
}

interface Layer {
  inNorm: any;
  wQkv: any;
  qNorm: any;
  kNorm: any;
  wO: any;
  postNorm: any;
  // the norm weights in the activation dtype, for the kernels whose weight shares the output's
  // dtype (rms_norm, linear_add_rms_norm, rms_norm_rope); the bf16 handles above with bf16 activations
  inNormA: any;
  postNormA: any;
  qNormA: any;
  kNormA: any;
  wGu: any;
  wDown: any;
  kCache: any;
  vCache: any;
}

interface PrefillGraph {
  graph: bigint;
  ids: any;        // device token ids the graph reads (uploaded before each replay)
  positions: any;  // 0 .. S-1
  logits: any;     // fp32 [1, vocab], written by each replay
}

export class Qwen3ForCausalLM {
  cfg: Qwen3Config;
  backend: any;
  ops: any;
  maxSeqLen: number;
  embed: any;
  finalNorm: any;
  finalNormA: any;
  act: string;
  flashName: string;
  // decode steps run each layer's attention block as one decode_attention_block call (head_dim
  // 128); false runs rms_norm_rope, decode_attention and the o_proj GEMV
  fusedDecode: boolean;
  invFreq: any;
  invFreqHost: Float32Array;
  layers: Layer[] = [];
  scale: number;
  // Captured prefills by prompt length (generate with useGraph), least recently used first; at most
  // maxPrefillGraphs are kept, each holding its activations and logits until dropped.
  prefillGraphs: Map<number, PrefillGraph> = new Map();
  maxPrefillGraphs: number = 4;

  // weights: Hugging Face tensor names -> bf16 bit patterns (tied embeddings: the lm_head is the
  // embedding matrix, for_causal_lm.ts:121-125).
  constructor(backend: any, cfg: Qwen3Config, weights: { [name: string]: Uint16Array }, maxSeqLen: number,
              activations?: string, f32Attention?: string) {
    this.cfg = cfg;
    this.backend = backend;
    this.ops = backend.operators;
    this.maxSeqLen = maxSeqLen;
    this.act = activations === undefined ? 'float32' : activations;
    if (this.act !== 'float32' && this.act !== 'bfloat16')
      throw new Error(`Qwen3ForCausalLM: activations must be float32 or bfloat16, not ${this.act}`);
    // float32 activations: the prefill attention in split-bf16 form ('split', the default) or on the
    // fp32 MFMA ('fp32'), as the Python model's f32_attention
    const fa = f32Attention === undefined ? 'split' : f32Attention;
    if (fa !== 'split' && fa !== 'fp32') throw new Error(`Qwen3ForCausalLM: f32Attention must be split or fp32, not ${fa}`);
    this.flashName = this.act === 'float32' && fa === 'split' ? 'flash_attention_split' : 'flash_attention';
    const H = cfg.hiddenSize, I = cfg.intermediateSize, D = cfg.headDim;
    const up = (bits: Uint16Array, shape: number[]): any => backend.createTensorHandle({ shape, dtype: 'bfloat16', data: bits });
    // a norm weight in the activation dtype (exactly widened for float32 activations)
    const upA = (bits: Uint16Array, shape: number[], bf: any): any =>
      this.act === 'float32' ? backend.createTensorHandle({ shape, dtype: 'float32', data: widenBf16(bits) }) : bf;
    const w = (name: string): Uint16Array => {
      const bits = weights[name];
      if (bits === undefined) throw new Error(`Qwen3ForCausalLM: missing weight ${name}`);
      return bits;
    };
    this.embed = up(w('model.embed_tokens.weight'), [cfg.vocabSize, H]);
    this.finalNorm = up(w('model.norm.weight'), [H]);
    this.finalNormA = upA(w('model.norm.weight'), [H], this.finalNorm);
    const nq = cfg.numAttentionHeads * D, nkv = cfg.numKeyValueHeads * D;
    for (let i = 0; i < cfg.numHiddenLayers; ++i) {
      const p = `model.layers.${i}.`;
      const cacheShape = [1, cfg.numKeyValueHeads, maxSeqLen, D];
      const inNorm = up(w(p + 'input_layernorm.weight'), [H]);
      const postNorm = up(w(p + 'post_attention_layernorm.weight'), [H]);
      const qNorm = up(w(p + 'self_attn.q_norm.weight'), [D]);
      const kNorm = up(w(p + 'self_attn.k_norm.weight'), [D]);
      this.layers.push({
        inNorm,
        wQkv: up(concatRows([w(p + 'self_attn.q_proj.weight'), w(p + 'self_attn.k_proj.weight'),
                             w(p + 'self_attn.v_proj.weight')]), [nq + 2 * nkv, H]),
        qNorm,
        kNorm,
        wO: up(w(p + 'self_attn.o_proj.weight'), [H, nq]),
        postNorm,
        inNormA: upA(w(p + 'input_layernorm.weight'), [H], inNorm),
        postNormA: upA(w(p + 'post_attention_layernorm.weight'), [H], postNorm),
        qNormA: upA(w(p + 'self_attn.q_norm.weight'), [D], qNorm),
        kNormA: upA(w(p + 'self_attn.k_norm.weight'), [D], kNorm),
        wGu: up(interleaveGateUp(w(p + 'mlp.gate_proj.weight'), w(p + 'mlp.up_proj.weight'), I, H), [2 * I, H]),
        wDown: up(w(p + 'mlp.down_proj.weight'), [H, I]),
        kCache: backend.createTensorHandle(cacheShape, this.act),
        vCache: backend.createTensorHandle(cacheShape, this.act),
      });
      // zero-filled as StaticKVCache's (kv-cache.ts:106-131): the decode block reads the row it is
      // about to write with a zero weight, which must not meet a NaN bit pattern
      const last = this.layers[this.layers.length - 1];
      for (const c of [last.kCache, last.vCache]) this.ops.find('zeros')(HipTensorIterator.nullaryOp(c.shape, c.dtype, c));
    }
    // RotaryEmbedding._computeInvFreqDirect (rope.ts:159-171): 1 / theta^(i / (D/2)) in float64,
    // stored as float32.
    const half = D / 2;
    this.invFreqHost = new Float32Array(half);
    for (let i = 0; i < half; ++i) this.invFreqHost[i] = 1 / Math.pow(cfg.ropeTheta, i / half);
    this.invFreq = backend.createTensorHandle({ shape: [half], dtype: 'float32', data: this.invFreqHost });
    this.scale = 1 / Math.sqrt(D);
    this.fusedDecode = D === 128;
  }

  static fromSafetensors(backend: any, cfg: Qwen3Config, file: string, maxSeqLen: number,
                         activations?: string, f32Attention?: string): Qwen3ForCausalLM {
    const tensors = readSafetensors(file);
    const weights: { [name: string]: Uint16Array } = {};
    for (const name of Object.keys(tensors)) weights[name] = bf16Bits(tensors[name], name);
    return new Qwen3ForCausalLM(backend, cfg, weights, maxSeqLen, activations, f32Attention);
  }

  private view(base: any, shape: number[], strides: number[], offset: number): any {
    return this.backend.createTensorHandle({ storage: base.storage, shape, dtype: base.dtype, strides, offset });
  }

  // fp32 logits [1, vocab] of the last of the S prompt tokens, written at cache rows [0, S).
  prefill(promptIds: number[]): any {
    const S = promptIds.length;
    if (S < 1 || S > this.maxSeqLen) throw new Error(`prefill: ${S} tokens for a cache of ${this.maxSeqLen}`);
    const be = this.backend;
    const ids = be.createTensorHandle({ shape: [S], dtype: 'int32', data: Int32Array.from(promptIds) });
    const positions = be.createTensorHandle({ shape: [S], dtype: 'int32', data: Int32Array.from(promptIds, (_: number, i: number) => i) });
    try {
      return this.prefillFrom(ids, positions, S);
    } finally {
      ids.dispose();
      positions.dispose();
    }
  }

  // The prefill over device-resident token ids and positions (int32 [S]): every launch reads its
  // inputs from device memory, so the same sequence can be captured as a graph and replayed.
  prefillFrom(ids: any, positions: any, S: number): any {
    const cfg = this.cfg, ops = this.ops, be = this.backend;
    const H = cfg.hiddenSize, I = cfg.intermediateSize, D = cfg.headDim;
    const Hq = cfg.numAttentionHeads, Hkv = cfg.numKeyValueHeads, eps = cfg.rmsNormEps;
    const nq = Hq * D, nkv = Hkv * D, nqkv = nq + 2 * nkv;
    const act = this.act;
    const x = be.createTensorHandle([S, H], 'float32');
    // the fused QKV projection sums over all of K, as matmul does on MFMA tiles (more than 8 rows)
    // when it does not split K
    const fuseQkv = D === 128 && S > 8 && be.gemmSplitCount(S, nqkv, H) === 1;
    ops.find('index_select')(this.embed, ids, { dim: 0 }, x);
    let h = ops.find('rms_norm')([x], { normalizedShape: [H], eps, weight: this.layers[0].inNormA, outDtype: act });
    // the RoPE angles of these positions, once for every layer's fused projection
    const ropeTab = fuseQkv ? ops.find('rope_table')(positions, this.invFreq) : undefined;
    for (let li = 0; li < this.layers.length; ++li) {
      const L = this.layers[li];
      const qh = be.createTensorHandle([1, Hq, S, D], act);
      if (fuseQkv) {
        // the projection with qk-norm, RoPE and the cache write in its epilogue: the same values as
        // the two launches below when their projection is not split over K
        ops.find('linear_qk_norm_rope')(h, L.wQkv, { qWeight: L.qNorm, kWeight: L.kNorm, invFreq: this.invFreq,
                                                     positions, eps, qOut: qh, kOut: L.kCache, vOut: L.vCache,
                                                     ropeTable: ropeTab });
        h.dispose();
      } else {
        const qkv = be.createTensorHandle([S, nqkv], act);
        ops.find('matmul')({ output: qkv, M: S, K: H, N: nqkv, batchSize: 1, transposeA: false, transposeB: true,
                             alpha: 1, beta: 0 }, h, L.wQkv);
        h.dispose();
        const heads = (col0: number, nh: number): any => this.view(qkv, [1, S, nh, D], [S * nqkv, nqkv, D, 1], col0);
        const q = heads(0, Hq), k = heads(nq, Hkv), v = heads(nq + nkv, Hkv);
        ops.find('rms_norm_rope')(q, k, { qWeight: L.qNormA, kWeight: L.kNormA, invFreq: this.invFreq, positions, eps,
                                          qOut: qh, kOut: L.kCache, v, vOut: L.vCache, cachePositions: true });
        for (const t of [q, k, v, qkv]) t.dispose();
      }
      // attention into [1, Hq, S, D] viewed over an [S, Hq D] buffer that o_proj reads as a matrix
      const attn = be.createTensorHandle([S, nq], act);
      const attnView = this.view(attn, [1, Hq, S, D], [S * nq, D, nq, 1], 0);
      const kc = this.view(L.kCache, [1, Hkv, S, D], L.kCache.strides, 0);
      const vc = this.view(L.vCache, [1, Hkv, S, D], L.vCache.strides, 0);
      ops.find(this.flashName)(qh, kc, vc, attnView, this.scale, S > 1);
      for (const t of [attnView, kc, vc, qh]) t.dispose();
      const h2 = be.createTensorHandle([S, H], act);
      ops.find('linear_add_rms_norm')(attn, L.wO, x, L.postNormA, eps, h2);
      attn.dispose();
      const a = be.createTensorHandle([S, I], act);
      ops.find('linear_swiglu')(h2, L.wGu, a);
      h2.dispose();
      if (li + 1 < this.layers.length) {
        h = be.createTensorHandle([S, H], act);
        ops.find('linear_add_rms_norm')(a, L.wDown, x, this.layers[li + 1].inNormA, eps, h);
      } else {
        h = be.createTensorHandle([1, H], act);
        ops.find('linear_add_rms_norm')(a, L.wDown, x, this.finalNormA, eps, h, [S - 1, S]);
      }
      a.dispose();
    }
    if (ropeTab !== undefined) ropeTab.dispose();
    const logits = be.createTensorHandle([1, cfg.vocabSize], 'float32');
    ops.find('matmul')({ output: logits, M: 1, K: H, N: cfg.vocabSize, batchSize: 1, transposeA: false,
                         transposeB: true, alpha: 1, beta: 0 }, h, this.embed);
    for (const t of [h, x]) t.dispose();
    return logits;
  }

  // The prompt's logits and whether the caller owns (disposes) them.  With useGraph the first
  // prompt of a given length runs eagerly and the same launches are then captured over a device ids
  // buffer; a later prompt of that length uploads its ids and replays (the logits then belong to the
  // graph), as the Python model does.
  private prefillLogits(promptIds: number[], useGraph: boolean): { logits: any; owned: boolean } {
    const S = promptIds.length, be = this.backend;
    if (!useGraph) return { logits: this.prefill(promptIds), owned: true };
    const entry = this.prefillGraphs.get(S);
    if (entry !== undefined) {
      entry.ids.upload(Int32Array.from(promptIds));
      be.graphLaunch(entry.graph);
      this.prefillGraphs.delete(S);  // most recently used last
      this.prefillGraphs.set(S, entry);
      return { logits: entry.logits, owned: false };
    }
    const logits = this.prefill(promptIds);
    if (this.maxPrefillGraphs < 1) return { logits, owned: true };
    while (this.prefillGraphs.size >= this.maxPrefillGraphs) this.dropPrefillGraph(this.prefillGraphs.keys().next().value);
    const ids = be.createTensorHandle({ shape: [S], dtype: 'int32', data: new Int32Array(S) });
    const positions = be.createTensorHandle({ shape: [S], dtype: 'int32', data: Int32Array.from(promptIds, (_: number, i: number) => i) });
    let gLogits: any = null;
    be.graphBegin();
    try {
      gLogits = this.prefillFrom(ids, positions, S);   // recorded, not run
    } catch (err) {
      try {
        be.graphDestroy(be.graphEnd());
      } catch (endErr) {
        // the capture failed as a whole; nothing left to destroy
      }
      ids.dispose();
      positions.dispose();
      throw err;
    }
    const graph = be.graphEnd();
    this.prefillGraphs.set(S, { graph, ids, positions, logits: gLogits });
    return { logits, owned: true };
  }

  private dropPrefillGraph(S: number): void {
    const e = this.prefillGraphs.get(S);
    if (e === undefined) return;
    this.prefillGraphs.delete(S);
    for (const t of [e.logits, e.ids, e.positions]) t.dispose();
    this.backend.graphDestroy(e.graph);
  }

  // One greedy step on device state: logits of token[0] at position pos[0] (its K/V row written
  // there), then token = argmax and greedy_advance (log[pos + 1 - base] = token, pos += 1).
  decodeStep(token: any, pos: any, lens: any, log: any, base: number): any {
    const cfg = this.cfg, ops = this.ops, be = this.backend;
    const H = cfg.hiddenSize, I = cfg.intermediateSize, eps = cfg.rmsNormEps, D = cfg.headDim;
    const Hq = cfg.numAttentionHeads, Hkv = cfg.numKeyValueHeads;
    const nq = Hq * D, nkv = Hkv * D, nqkv = nq + 2 * nkv;
    const act = this.act;
    const x = be.createTensorHandle([1, H], 'float32');
    ops.find('index_select')(this.embed, token, { dim: 0 }, x);
    for (const L of this.layers) {
      const qkv = be.createTensorHandle([1, nqkv], act);
      ops.find('gemv_fused')('rms_norm', x, L.wQkv, qkv, { normWeight: L.inNorm, eps, actDtype: act });
      if (this.fusedDecode) {
        ops.find('decode_attention_block')(qkv, { qNorm: L.qNorm, kNorm: L.kNorm, invFreq: this.invFreq, eps,
                                                  position: pos, kCache: L.kCache, vCache: L.vCache, wO: L.wO, x,
                                                  scale: this.scale });
      } else {
        // qk-norm + RoPE at position p with the K/V rows written into the caches there, the one
        // query against cache rows [0, p], then x += o W_o^T
        const heads = (col0: number, nh: number): any => this.view(qkv, [1, 1, nh, D], [nqkv, nqkv, D, 1], col0);
        const q = heads(0, Hq), k = heads(nq, Hkv), v = heads(nq + nkv, Hkv);
        const qh = be.createTensorHandle([1, Hq, 1, D], act);
        ops.find('rms_norm_rope')(q, k, { qWeight: L.qNormA, kWeight: L.kNormA, invFreq: this.invFreq, positions: pos,
                                          eps, qOut: qh, kOut: L.kCache, v, vOut: L.vCache, cachePositions: true });
        for (const t of [q, k, v]) t.dispose();
        const attn = be.createTensorHandle([1, nq], act);
        const attnView = this.view(attn, [1, Hq, 1, D], [nq, D, D, 1], 0);
        ops.find('decode_attention')(qh, L.kCache, L.vCache, lens, attnView, this.scale);
        ops.find('gemv_fused')('none', attn, L.wO, x, { cin: x, actDtype: act });
        for (const t of [attnView, attn, qh]) t.dispose();
      }
      qkv.dispose();
      const a = be.createTensorHandle([1, I], act);
      ops.find('gemv_swiglu')('rms_norm', x, L.wGu, a, { normWeight: L.postNorm, eps });
      ops.find('gemv_fused')('none', a, L.wDown, x, { cin: x, actDtype: act });
      a.dispose();
    }
    const logits = be.createTensorHandle([1, cfg.vocabSize], 'float32');
    ops.find('gemv_fused')('rms_norm', x, this.embed, logits, { normWeight: this.finalNorm, eps, actDtype: act });
    x.dispose();
    ops.find('argmax')(HipTensorIterator.reductionOp(logits, [-1], false, token));
    ops.find('greedy_advance')(token, pos, lens, log, base);
    return logits;
  }

  // Greedy generation (generateWithKVCache, for_causal_lm.ts:475-508): maxNewTokens token ids, each
  // the argmax of the previous logits, after maxNewTokens one-token forwards; returns the ids, the
  // fp32 logits of every forward (the prefill's last position, then each decode step) unless
  // returnLogits is false, and the wall times.  With useGraph the prefill is replayed from a graph
  // captured for its prompt length when there is one (prefillLogits), and the first decode step runs
  // eagerly, after which the step is captured once as a HIP graph and replayed (every value that
  // changes from step to step lives in device memory), as the Python model does.
  async generate(promptIds: number[], maxNewTokens: number, options?: { [key: string]: any }):
      Promise<{ tokens: number[]; logits: Float32Array[]; prefillMs: number; decodeMs: number; replayMs: number }> {
    const opt = options || {};
    const useGraph = !!opt.useGraph;
    const returnLogits = opt.returnLogits === undefined ? true : !!opt.returnLogits;
    const be = this.backend, P = promptIds.length, N = maxNewTokens;
    if (P + N > this.maxSeqLen) throw new Error(`generate: ${P} + ${N} positions for a cache of ${this.maxSeqLen}`);
    const logits: Float32Array[] = [];
    const t0 = performance.now();
    const pre = this.prefillLogits(promptIds, useGraph);
    const first = pre.logits;
    if (returnLogits) logits.push((await first.dataAsync()) as Float32Array);
    const token = be.createTensorHandle({ shape: [1], dtype: 'int32', data: new Int32Array(1) });
    const log = be.createTensorHandle({ shape: [N + 1], dtype: 'int32', data: new Int32Array(N + 1) });
    this.ops.find('argmax')(HipTensorIterator.reductionOp(first, [-1], false, token));
    if (pre.owned) first.dispose();
    const head = this.view(log, [1], [1], 0);
    this.ops.find('copy_')(HipTensorIterator.unaryOp(token, head));
    head.dispose();
    const pos = be.createTensorHandle({ shape: [1], dtype: 'int32', data: new Int32Array([P]) });
    const lens = be.createTensorHandle({ shape: [1], dtype: 'int32', data: new Int32Array([P + 1]) });
    be.synchronize();
    const t1 = performance.now();
    let t2 = t1;
    let graph: bigint | null = null;
    let gLogits: any = null;
    let tokens: number[] = [];
    try {
      for (let i = 0; i < N; ++i) {
        if (!useGraph || i === 0) {
          const lg = this.decodeStep(token, pos, lens, log, P);
          if (returnLogits) logits.push((await lg.dataAsync()) as Float32Array);
          lg.dispose();
          if (useGraph && N > 1) {
            be.graphBegin();
            try {
              gLogits = this.decodeStep(token, pos, lens, log, P);   // recorded, not run
            } finally {
              graph = be.graphEnd();
            }
            be.synchronize();
            t2 = performance.now();
          }
        } else {
          be.graphLaunch(graph as bigint);
          if (returnLogits) logits.push((await gLogits.dataAsync()) as Float32Array);
        }
      }
      tokens = Array.from((await log.dataAsync()) as Int32Array).slice(0, N);
    } finally {
      if (gLogits !== null) gLogits.dispose();
      if (graph !== null) be.graphDestroy(graph);
      for (const t of [token, log, pos, lens]) t.dispose();
    }
    const t3 = performance.now();
    return { tokens, logits, prefillMs: t1 - t0, decodeMs: t3 - t1, replayMs: useGraph && N > 1 ? t3 - t2 : 0 };
  }

  dispose(): void {
    for (const S of Array.from(this.prefillGraphs.keys())) this.dropPrefillGraph(S);
    for (const L of this.layers) {
      for (const t of [L.inNorm, L.wQkv, L.qNorm, L.kNorm, L.wO, L.postNorm, L.wGu, L.wDown, L.kCache, L.vCache]) {
        t.dispose();
      }
      if (this.act === 'float32') for (const t of [L.inNormA, L.postNormA, L.qNormA, L.kNormA]) t.dispose();
    }
    for (const t of [this.embed, this.finalNorm, this.invFreq]) t.dispose();
    if (this.finalNormA !== this.finalNorm) this.finalNormA.dispose();
    this.layers = [];
  }
}
