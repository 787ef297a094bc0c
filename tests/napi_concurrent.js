'use strict';
// Two HybridMambaModels on one device driven at once (Promise.all), then device.destroy()
// while a generate is in flight; prints one JSON line for tests/test_napi.py.
// usage: node napi_concurrent.js <ckpt A> <cfg A.json> <ckpt B> <cfg B.json> <prompt csv> <n_new>
const fs = require('fs');
const path = require('path');
const hip = require(path.join(__dirname, '..', 'ssmjs_amd', 'napi'));

async function main() {
  const [ckA, cfgA, ckB, cfgB, promptCsv, nNew] = process.argv.slice(2);
  const prompt = promptCsv.split(',').map(Number);
  const n = Number(nNew);
  const { device } = await hip.initWebGPU({});
  const a = new hip.HybridMambaModel(device, JSON.parse(fs.readFileSync(cfgA, 'utf8')));
  const b = new hip.HybridMambaModel(device, JSON.parse(fs.readFileSync(cfgB, 'utf8')));
  await Promise.all([a.loadWeights(fs.readFileSync(ckA)), b.loadWeights(fs.readFileSync(ckB))]);
  const greedy = { temperature: 1.0, topK: 1, topP: 0.9 };
  // interleaved calls of both models: each model's calls run in order, the two models' calls
  // run on pool threads at the same time
  const [genA, genB, fwdA, fwdB, genA2] = await Promise.all([
    a.generate(prompt, n, greedy), b.generate(prompt, n, greedy),
    a.forward(Uint32Array.from(prompt), 1, prompt.length),
    b.forward(Uint32Array.from(prompt), 1, prompt.length),
    a.generate(prompt, n, greedy)]);
  // destroy the device while a long generate of model b runs
  const pending = b.generate(prompt, 400, greedy).then(
    (ids) => ({ ok: true, len: ids.length }), (e) => ({ ok: false, code: e.code }));
  await new Promise((r) => setTimeout(r, 20));
  device.destroy();
  const during = await pending;
  let after = null;
  try { await a.forward(Uint32Array.from(prompt), 1, prompt.length); } catch (e) { after = e.code; }
  process.stdout.write(JSON.stringify({
    genA, genB, genA2, fwdA: Array.from(fwdA.logits), fwdB: Array.from(fwdB.logits), during, after,
  }) + '\n');
}

main().catch((e) => {
  console.error('napi_concurrent failed:', e.code, e.message);
  process.exit(1);
});
