'use strict';
/*
 * generate.js — greedy generation with the TypeScript Qwen3 model (src/qwen3.ts, stripped into
 * dist/qwen3.js) on the HIP backend, from Node.
 *
 * Usage: node examples/generate.js CONFIG.json MODEL.safetensors PROMPT_IDS.json NEW_TOKENS [options]
 *   CONFIG.json        a Hugging Face Qwen3 config (vocab_size, hidden_size, intermediate_size,
 *                      num_hidden_layers, num_attention_heads, num_key_value_heads, head_dim,
 *                      rms_norm_eps, rope_theta); tied embeddings
 *   MODEL.safetensors  one bf16 safetensors file with the Hugging Face tensor names
 *   PROMPT_IDS.json    a JSON array of prompt token ids
 *   --eager            issue every launch from the host (default: prefill and decode step replayed
 *                      from HIP graphs)
 *   --warmup N         tokens of the untimed warm-up generation (default 8; it captures the graphs)
 *   --activations A    float32 (default: the reference's float32 arithmetic) or bfloat16
 * Prints one JSON line: the generated token ids, prefill_ms and decode tokens/s of the timed run.
 */
const fs = require('fs');
const path = require('path');
const { performance } = require('perf_hooks');
const dist = path.join(__dirname, '..', 'dist');
const { HipBackend } = require(path.join(dist, 'index.js'));
const { Qwen3ForCausalLM } = require(path.join(dist, 'qwen3.js'));

function configFrom(hf) {
  const pick = (snake, camel) => (hf[snake] !== undefined ? hf[snake] : hf[camel]);
  const cfg = {
    vocabSize: pick('vocab_size', 'vocabSize'),
    hiddenSize: pick('hidden_size', 'hiddenSize'),
    intermediateSize: pick('intermediate_size', 'intermediateSize'),
    numHiddenLayers: pick('num_hidden_layers', 'numHiddenLayers'),
    numAttentionHeads: pick('num_attention_heads', 'numAttentionHeads'),
    numKeyValueHeads: pick('num_key_value_heads', 'numKeyValueHeads'),
    headDim: pick('head_dim', 'headDim'),
    rmsNormEps: pick('rms_norm_eps', 'rmsNormEps'),
    ropeTheta: pick('rope_theta', 'ropeTheta'),
  };
  for (const k of Object.keys(cfg)) {
    if (typeof cfg[k] !== 'number') throw new Error(`generate.js: config has no ${k}`);
  }
  return cfg;
}

async function main() {
  const argv = process.argv.slice(2);
  const pos = argv.filter((a, i) => !a.startsWith('--') &&
                                    !(i > 0 && (argv[i - 1] === '--warmup' || argv[i - 1] === '--activations')));
  if (pos.length !== 4) {
    console.error('usage: node examples/generate.js CONFIG.json MODEL.safetensors PROMPT_IDS.json NEW_TOKENS ' +
                  '[--eager] [--warmup N] [--activations float32|bfloat16]');
    process.exit(2);
  }
  const [cfgPath, modelPath, idsPath, nStr] = pos;
  const useGraph = !argv.includes('--eager');
  const wi = argv.indexOf('--warmup');
  const warmup = wi >= 0 ? parseInt(argv[wi + 1], 10) : 8;
  const ai = argv.indexOf('--activations');
  const activations = ai >= 0 ? argv[ai + 1] : 'float32';
  const N = parseInt(nStr, 10);
  const cfg = configFrom(JSON.parse(fs.readFileSync(cfgPath, 'utf8')));
  const prompt = JSON.parse(fs.readFileSync(idsPath, 'utf8'));
  const backend = await HipBackend.create(0);
  const t0 = performance.now();
  const model = Qwen3ForCausalLM.fromSafetensors(backend, cfg, modelPath, prompt.length + Math.max(N, warmup),
                                                 activations);
  const loadMs = performance.now() - t0;
  try {
    let warm = null;
    if (warmup > 0) warm = await model.generate(prompt, warmup, { useGraph, returnLogits: false });
    const res = await model.generate(prompt, N, { useGraph, returnLogits: false });
    const replaySteps = useGraph ? N - 1 : N;
    const decodeWindowMs = useGraph ? res.replayMs : res.decodeMs;
    console.log(JSON.stringify({
      tokens: res.tokens,
      load_ms: loadMs,
      prefill_ms: res.prefillMs,
      prefill_eager_ms: warm !== null ? warm.prefillMs : null,
      decode_ms: res.decodeMs,
      decode_tokens_per_s: decodeWindowMs > 0 ? (replaySteps * 1000) / decodeWindowMs : null,
      decode_steps_timed: replaySteps,
      issue: useGraph ? 'hip graph replay' : 'eager',
      activations,
    }));
  } finally {
    model.dispose();
  }
}

main().catch((err) => {
  console.error(err && err.stack ? err.stack : err);
  process.exit(1);
});
