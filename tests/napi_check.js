'use strict';
// Drives the Node-API backend the way src/session/session.ts and streaming.ts use
// MambaCode.js, and prints the results as one JSON line for tests/test_napi.py.
// usage: node napi_check.js <checkpoint> <config.json> <prompt ids, comma separated> <n_new>
const fs = require('fs');
const path = require('path');
const hip = require(path.join(__dirname, '..', 'ssmjs_amd', 'napi'));

async function main() {
  const [ckpt, cfgPath, promptCsv, nNew] = process.argv.slice(2);
  const cfg = JSON.parse(fs.readFileSync(cfgPath, 'utf8'));
  const { device } = await hip.initWebGPU({ powerPreference: 'high-performance' });
  const model = new hip.HybridMambaModel(device, cfg);
  await model.loadWeights(fs.readFileSync(ckpt));
  const prompt = promptCsv.split(',').map(Number);
  const generated = await model.generate(prompt, Number(nNew), { temperature: 0.8, topK: 1, topP: 0.9 });
  const draws = [0.1, 0.7, 0.35, 0.9, 0.5];
  let nDraw = 0;
  const sampled = await model.generate(prompt, 8, { temperature: 1.3, topK: 5, topP: 0.9,
                                                    rng: () => draws[nDraw++ % draws.length] });
  const { logits } = await model.forward(Uint32Array.from(prompt), 1, prompt.length);
  let badCode = null;
  try { await model.loadWeights(Buffer.from('JUNK0000')); } catch (e) { badCode = e.code; }
  const exported = await model.exportWeights();
  const trainer = new hip.MambaTrainer(model, { encode: (s) => Array.from(Buffer.from(s, 'latin1')) });
  const ppl = await trainer.evaluate('hello mamba');
  await model.destroy();
  let destroyedCode = null;
  try { await model.forward(Uint32Array.of(1, 2), 1, 2); } catch (e) { destroyedCode = e.code; }
  device.destroy();
  process.stdout.write(JSON.stringify({
    generated, sampled, logits: Array.from(logits), badCode, destroyedCode,
    exportedBytes: exported.byteLength, ppl,
  }) + '\n');
}

main().catch((e) => {
  console.error('napi_check failed:', e.code, e.message);
  process.exit(1);
});
