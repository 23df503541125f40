'use strict';
/*
 * qwen3_generate.js — greedy generation with the TypeScript Qwen3 model (packages/backend-hip/src/
 * qwen3.ts, stripped into dist/qwen3.js) on the HIP backend.  Test infrastructure:
 * tests/test_gpu_node_qwen3.py writes the checkpoint and compares the results with the Python model.
 *
 * Usage: node qwen3_generate.js DIR
 *   DIR/meta.json {cfg, prompt, n, maxSeq} and DIR/model.safetensors (bf16); generates eagerly, then
 *   twice with HIP graphs (decode step replayed; the second time the prefill too), writes
 *   DIR/logits.f32, DIR/logits_graph.f32 and DIR/logits_graph2.f32 ((n + 1) rows of vocab fp32
 *   logits each) and DIR/inv_freq.f32, and prints a JSON summary.
 */
const fs = require('fs');
const path = require('path');
const dist = path.join(__dirname, '..', '..', 'packages', 'backend-hip', 'dist');
const { HipBackend } = require(path.join(dist, 'index.js'));
const { Qwen3ForCausalLM } = require(path.join(dist, 'qwen3.js'));

async function main() {
  const dir = process.argv[2];
  const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
  const backend = await HipBackend.create(0);
  const before = backend.memoryStats().liveBytes;
  const model = Qwen3ForCausalLM.fromSafetensors(backend, meta.cfg, path.join(dir, 'model.safetensors'), meta.maxSeq);
  const V = meta.cfg.vocabSize;
  const save = (name, rows) => {
    const all = new Float32Array(rows.length * V);
    rows.forEach((row, i) => all.set(row, i * V));
    fs.writeFileSync(path.join(dir, name), Buffer.from(all.buffer));
  };
  const res = await model.generate(meta.prompt, meta.n);
  save('logits.f32', res.logits);
  // the same generation with the decode step captured once and replayed as a HIP graph (the prefill
  // runs eagerly and is captured for this prompt length) ...
  const resG = await model.generate(meta.prompt, meta.n, { useGraph: true });
  save('logits_graph.f32', resG.logits);
  // ... and again, now with the prefill replayed from its graph too
  const resG2 = await model.generate(meta.prompt, meta.n, { useGraph: true });
  save('logits_graph2.f32', resG2.logits);
  fs.writeFileSync(path.join(dir, 'inv_freq.f32'), Buffer.from(model.invFreqHost.buffer));
  const prefillGraphs = Array.from(model.prefillGraphs.keys());   // captured prompt lengths
  model.dispose();
  backend.synchronize();
  console.log(JSON.stringify({ tokens: res.tokens, tokensGraph: resG.tokens, tokensGraph2: resG2.tokens,
                               rows: res.logits.length, rowsGraph: resG.logits.length, rowsGraph2: resG2.logits.length,
                               prefillGraphs, replayMs: resG.replayMs,
                               liveBefore: before, liveAfter: backend.memoryStats().liveBytes }));
}

main().catch((err) => {
  console.error(err && err.stack ? err.stack : err);
  process.exit(1);
});
