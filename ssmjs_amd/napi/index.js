'use strict';
// MI355X backend module for ssmjs's session layer: the names and call shapes that
// src/session/session.ts imports from @seanhogg/mambacode.js (session.ts:10-18), over the
// Node-API addon ssm_napi.node (C ABI: include/ssm_hip.h).
//
//   initWebGPU({powerPreference})            session.ts:274-277  -> {adapter, device}
//   new HybridMambaModel(device, config)     session.ts:359
//     .config                                streaming.ts:24 (vocabSize, eosId)
//     .forward(ids, batch, seqLen)           streaming.ts:31-35  -> Promise<{logits}>
//     .generate(ids, n, {temperature,topK,topP}) session.ts:421-425 -> Promise<number[]>
//     .loadWeights(buf) / .exportWeights()   session.ts:394,575 / :518
//   new MambaTrainer(model, tokenizer).evaluate(text)  session.ts:504-507
//   device.destroy()                         session.ts:592
// Written for Node >= 12 (plain CommonJS, no optional chaining), so it also loads under the
// Node in this image; the reference's TypeScript passes `gpuAdapter: new HipAdapter()`
// (session.ts:260-271) or replaces its import of mambacode.js with this module.

const path = require('path');

let addon = null;
function native() {
  if (addon === null) {
    // no fallback: without the addon (or without libssm_hip.so) this throws
    addon = require(path.join(__dirname, 'ssm_napi.node'));
  }
  return addon;
}

const LAYER_CODES = { mamba1: 1, mamba2: 2, mamba3: 3, attention: 4 };
const MIN_TEMPERATURE = 1e-7;   // streaming.ts:11

// ------------------------------------------------------------------ device / adapter
class HipDevice {
  constructor(ctx) {
    this._ctx = ctx;
    this._destroyed = false;
  }
  get info() { return native().ctxInfo(this._ctx); }
  destroy() {
    if (this._destroyed) return;
    this._destroyed = true;
    native().ctxDestroy(this._ctx);
  }
}

class HipAdapter {
  constructor(ordinal) { this.ordinal = ordinal || 0; }
  requestDevice() {
    return native().ctxCreate(this.ordinal).then((ctx) => new HipDevice(ctx));
  }
}

function initWebGPU(opts) {
  void opts;   // powerPreference has no meaning for one HIP device
  const adapter = new HipAdapter(0);
  return adapter.requestDevice().then((device) => ({ adapter, device }));
}

// ------------------------------------------------------------------ sampling (streaming.ts:53-97)
function sampleToken(logits, temperature, topK, topP, rng) {
  const t = Math.max(temperature, MIN_TEMPERATURE);
  const n = logits.length;
  const scaled = new Float32Array(n);
  let maxL = -Infinity;
  for (let i = 0; i < n; i++) {
    scaled[i] = logits[i] / t;
    if (scaled[i] > maxL) maxL = scaled[i];
  }
  const exps = new Float32Array(n);
  let sum = 0;
  for (let i = 0; i < n; i++) {
    exps[i] = Math.exp(scaled[i] - maxL);
    sum += exps[i];
  }
  const order = Array.from({ length: n }, (_, i) => i);
  order.sort((a, b) => exps[b] - exps[a]);   // stable: ties keep ascending index
  const top = order.slice(0, topK);
  const nucleus = [];
  let cum = 0;
  for (const idx of top) {
    cum += exps[idx] / sum;
    nucleus.push(idx);
    if (cum >= topP) break;
  }
  let nsum = 0;
  for (const idx of nucleus) nsum += exps[idx];
  const threshold = (rng || Math.random)() * nsum;
  let acc = 0;
  for (const idx of nucleus) {
    acc += exps[idx];
    if (acc >= threshold) return idx;
  }
  return nucleus[nucleus.length - 1];
}

// ------------------------------------------------------------------ model
function nativeConfig(config) {
  const layers = config.layers || [];
  const types = new Int32Array(config.numLayers);
  for (let i = 0; i < config.numLayers; i++) {
    const t = layers[i] ? layers[i].type : 'mamba1';
    if (!(t in LAYER_CODES)) throw new Error(`unknown layer type ${t}`);
    types[i] = LAYER_CODES[t];
  }
  const c = {};
  for (const k of ['vocabSize', 'dModel', 'numLayers', 'dState', 'dConv', 'expand', 'nHeads',
    'nGroups', 'chunkLen', 'mimoGroup', 'eosId', 'dtRank', 'normEps']) {
    if (config[k] !== undefined && config[k] !== null) c[k] = config[k];
  }
  c.layerTypes = types;
  return c;
}

class HybridMambaModel {
  constructor(device, config, seed) {
    this.device = device;
    this.config = Object.assign({ eosId: -1 }, config);
    // the constructor is synchronous in the reference; creation completes in the background
    // and every method waits for it (calls on one model run one at a time, in order)
    this._h = null;
    this._queue = native().modelCreate(device._ctx, nativeConfig(this.config), seed || 0)
      .then((h) => { this._h = h; });
  }

  _run(fn) {
    const p = this._queue.then(() => fn(native(), this._h));
    this._queue = p.then(() => undefined, () => undefined);
    return p;
  }

  forward(ids, batch, seqLen) {
    const u = ids instanceof Uint32Array ? ids : Uint32Array.from(ids);
    return this._run((a, h) => a.forward(h, u, batch, seqLen)).then((logits) => ({ logits }));
  }

  generate(promptIds, maxNewTokens, sampling) {
    const s = sampling || {};
    const temperature = s.temperature !== undefined ? s.temperature : 1.0;
    const topK = s.topK !== undefined ? s.topK : 50;
    const topP = s.topP !== undefined ? s.topP : 0.9;
    const rng = s.rng;
    const ids = Array.from(promptIds, Number);
    const eos = this.config.eosId;
    if (!(maxNewTokens > 0)) return Promise.resolve(ids);
    return this._run((a, h) => {
      const st = a.stateCreate(h, 1);
      const done = (r) => { a.stateDestroy(st); return r; };
      const fail = (e) => { a.stateDestroy(st); throw e; };
      const keep = (out) => {
        for (const t of out) {
          ids.push(t);
          if (t === eos) break;
        }
        return ids;
      };
      const V = this.config.vocabSize;
      if (topK >= 1 && V <= 262144 && Math.min(topK, V) <= 1024) {
        // sampleToken on the device (ssm_generate_sample), topK 1 included: one draw per
        // step, taken up front in the order the host loop below takes them
        const draw = rng || Math.random;
        const u = new Float64Array(maxNewTokens);
        for (let k = 0; k < maxNewTokens; k++) u[k] = draw();
        return a.generateSample(h, st, Uint32Array.from(ids), ids.length, maxNewTokens,
                                temperature, topK, topP, u).then(keep).then(done, fail);
      }
      if (topK === 1) {
        // beyond the device sampler: device argmax of the logits (lowest index among equal
        // maxima)
        return a.generateGreedy(h, st, Uint32Array.from(ids), ids.length, maxNewTokens)
          .then(keep).then(done, fail);
      }
      const step = (logits, k) => {
        const nxt = sampleToken(logits, temperature, topK, topP, rng);
        ids.push(nxt);
        if (nxt === eos || k + 1 === maxNewTokens) return ids;
        return a.decodeStep(h, st, Uint32Array.of(nxt)).then((lg) => step(lg, k + 1));
      };
      return a.prefill(h, st, Uint32Array.from(ids), ids.length)
        .then((lg) => step(lg, 0)).then(done, fail);
    });
  }

  loadWeights(buf) { return this._run((a, h) => a.loadWeights(h, buf)); }

  exportWeights(f16) { return this._run((a, h) => a.exportWeights(h, !!f16)); }

  destroy() { return this._run((a, h) => a.modelDestroy(h)); }
}

// ------------------------------------------------------------------ trainer (evaluate only)
class MambaTrainer {
  constructor(model, tokenizer) {
    this.model = model;
    this.tokenizer = tokenizer;
  }

  // perplexity = exp(mean next-token cross-entropy) over the encoded text
  evaluate(text) {
    const ids = this.tokenizer.encode(text);
    if (ids.length < 2) return Promise.reject(new Error('evaluate: text must encode to >= 2 tokens'));
    const V = this.model.config.vocabSize;
    return this.model.forward(Uint32Array.from(ids), 1, ids.length).then(({ logits }) => {
      let nll = 0;
      for (let t = 0; t + 1 < ids.length; t++) {
        const row = logits.subarray(t * V, (t + 1) * V);
        let m = -Infinity;
        for (let v = 0; v < V; v++) if (row[v] > m) m = row[v];
        let s = 0;
        for (let v = 0; v < V; v++) s += Math.exp(row[v] - m);
        nll += m + Math.log(s) - row[ids[t + 1]];
      }
      return Math.exp(nll / (ids.length - 1));
    });
  }

  train() {
    return Promise.reject(new Error('training is not part of the MI355X forward-path backend'));
  }
}

module.exports = { initWebGPU, HipAdapter, HipDevice, HybridMambaModel, MambaTrainer, sampleToken,
  LAYER_CODES, native };
