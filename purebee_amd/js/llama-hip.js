/**
 * purebee_amd -- resident Llama-family model on the GPU.
 *
 * The decode-step seam of the reference: LlamaRuntime (llama.js:204-505) and
 * StreamingLlamaRuntime (llama-streaming.js:738-862) run forward / generate /
 * resetCache / rollbackCache over weights that are re-read or re-streamed on
 * every token; here the weights are uploaded once (GGUF tensor names,
 * gguf.js:378-410) and every step runs on the GPU (pbx_model_*).
 *
 *   const { HipLlamaRuntime } = require('purebee_amd/js/llama-hip');
 *   const rt = new HipLlamaRuntime({ dim, hiddenDim, nLayers, nHeads, nKvHeads,
 *                                    vocabSize, seqLen, ropeTheta,
 *                                    weightType: 'q4_0', embedType: 'q4_0' });
 *   rt.loadTensor('token_embd.weight', rawBlocks);   // per GGUF tensor
 *   const logits = rt.forward(promptTokens, 0);       // llama.js:204
 *   const out = rt.generate(promptTokens, 64, { greedy: true });
 *   const rt2 = HipLlamaRuntime.fromGGUF('model.gguf', { maxSeq: 2048 });
 *
 * HipStreamingLlamaRuntime has StreamingLlamaRuntime's surface
 * (llama-streaming.js:738-970): forward(tokenIds, startPos, { maxLayers })
 * returns { logits, layersUsed }, so SelfSpeculativeDecoder
 * (speculative.js) drives it unchanged.  HipSelfSpeculativeDecoder runs that
 * decoder's greedy mode on the GPU (draft = the first draftLayers layers);
 * HipSpeculativeDecoder drafts with a separate (smaller) model.
 */
'use strict';

const path = require('path');

const TYPES = { f32: 0, q4_0: 2, q4_1: 3, q8_0: 8 };
const TENSOR = {
  'token_embd.weight': 0, 'output.weight': 1, 'output_norm.weight': 2,
  'attn_norm.weight': 3, 'ffn_norm.weight': 4, 'attn_q.weight': 5, 'attn_k.weight': 6,
  'attn_v.weight': 7, 'attn_output.weight': 8, 'ffn_gate.weight': 9, 'ffn_up.weight': 10,
  'ffn_down.weight': 11,
};

let addon = null;
function load() {
  if (addon) return addon;
  addon = require(path.join(__dirname, '..', 'lib', 'pbx_napi.node'));
  addon.init(0);
  return addon;
}

function typeId(t) {
  if (typeof t === 'number') return t;
  if (!(t in TYPES)) throw new Error(`Unsupported weight type: ${t}`);
  return TYPES[t];
}

/**
 * Top-k / temperature sampling of llama.js:394-423 (f32: the scaled logits
 * are a Float32Array there) and llama-streaming.js:868-896 (doubles): the
 * topK largest of logits / temperature in descending order, earlier index
 * first among equal values (the stable sort of both), a softmax over them
 * and one draw of `random()` against the running sum.  The k largest are
 * kept by insertion instead of sorting the whole vocabulary.
 */
function sampleTopK(logits, topK, temperature, random, f32) {
  const k = Math.max(1, Math.min(topK, logits.length));
  const val = new Float64Array(k), idx = new Int32Array(k);
  let n = 0;
  for (let i = 0; i < logits.length; i++) {
    const v = f32 ? Math.fround(logits[i] / temperature) : logits[i] / temperature;
    if (n === k && !(v > val[k - 1])) continue;
    let j = n < k ? n++ : k - 1;
    while (j > 0 && val[j - 1] < v) { val[j] = val[j - 1]; idx[j] = idx[j - 1]; j--; }
    val[j] = v;
    idx[j] = i;
  }
  const maxV = val[0];
  const probs = new Float64Array(n);
  let sum = 0;
  for (let i = 0; i < n; i++) { probs[i] = Math.exp(val[i] - maxV); sum += probs[i]; }
  const r = random();
  let cum = 0;
  for (let i = 0; i < n; i++) {
    cum += probs[i] / sum;
    if (r <= cum) return idx[i];
  }
  return idx[0];
}

// 'blk.3.attn_q.weight' -> [5, 3]; 'token_embd.weight' -> [0, -1]
function tensorId(name) {
  const m = /^blk\.(\d+)\.(.+)$/.exec(name);
  const base = m ? m[2] : name;
  if (!(base in TENSOR)) throw new Error(`Unknown tensor name: ${name}`);
  return [TENSOR[base], m ? parseInt(m[1], 10) : -1];
}

class HipLlamaRuntime {
  /**
   * A resident model straight from a GGUF file (the build's reader; weights
   * uploaded once), configured from its metadata like loadGGUFModel /
   * parseHeader (gguf.js:778-839, streaming-loader.js:35-87).
   */
  static fromGGUF(filePath, opts = {}) {
    const r = load().modelLoadGGUF(String(filePath), opts.maxSeq || 0);
    return new HipLlamaRuntime(r.config, r.model);
  }

  constructor(config, handle) {
    const a = load();
    const c = config;
    // source of the sampling draws (Math.random in the reference)
    this.random = c.random || Math.random;
    this.config = Object.assign({}, c);
    delete this.config.random;
    this.config.headDim = c.headDim || Math.floor(c.dim / c.nHeads);
    if (handle) {
      this._model = handle;
      return;
    }
    this._model = a.modelCreate({
      dim: c.dim, hiddenDim: c.hiddenDim, nLayers: c.nLayers, nHeads: c.nHeads,
      nKvHeads: c.nKvHeads || c.nHeads, headDim: this.config.headDim, vocabSize: c.vocabSize,
      maxSeq: c.seqLen, weightType: typeId(c.weightType || 'q4_0'),
      embedType: typeId(c.embedType || 'f32'),
      outputType: c.outputType === undefined || c.outputType === null ? -1 : typeId(c.outputType),
      rmsEps: c.rmsEps || 1e-5, ropeTheta: c.ropeTheta || 10000.0,
    });
  }

  /** One GGUF tensor: raw blocks (Q4_0/Q4_1/Q8_0) or a Float32Array (F32, norms). */
  loadTensor(name, data) {
    const [tid, layer] = tensorId(name);
    addon.modelSetTensor(this._model, tid, layer, data);
  }

  /** llama.js:204: logits of the last position, KV cache written. */
  forward(tokenIds, startPos) {
    return addon.modelForward(this._model, Int32Array.from(tokenIds), startPos).logits;
  }

  /** Every position's logits in one batched pass: {logits [n*vocab], next [n]}. */
  forwardAll(tokenIds, startPos) {
    return addon.modelForwardBatch(this._model, Int32Array.from(tokenIds), startPos);
  }

  /** llama.js:432-442: the first maximum. */
  argmax(logits) {
    let maxVal = -Infinity;
    let maxIdx = 0;
    for (let i = 0; i < logits.length; i++) {
      if (logits[i] > maxVal) { maxVal = logits[i]; maxIdx = i; }
    }
    return maxIdx;
  }

  /** llama.js:394-423: top-k + temperature sampling (f32 scaled logits). */
  sample(logits, topK = 40, temperature = 0.8) {
    return sampleTopK(logits, topK, temperature, this.random, true);
  }

  resetCache() { addon.modelReset(this._model); }

  rollbackCache(pos) { addon.modelRollback(this._model, pos); }

  /** Logits of the last of tokenIds at startPos.. (the runtime's forward). */
  _logits(tokenIds, startPos) {
    return addon.modelForward(this._model, Int32Array.from(tokenIds), startPos).logits;
  }

  /**
   * llama.js:452-505.  Greedy: prefill, then the decode loop on the GPU (the
   * argmax of each step feeds the next without returning to the host, the
   * tokens checked for eosId after every graph launch of 8 steps); it stops
   * at the first eosId as the reference does, leaving no cache row past it.
   * Otherwise each step's logits come back and sample() picks the token.
   */
  generate(promptTokens, maxTokens = 50, opts = {}) {
    if (!opts.greedy) return this._generateSampled(promptTokens, maxTokens, opts);
    const eosId = opts.eosId || 2;
    this.resetCache();
    const all = [...promptTokens];
    const t0 = Date.now();
    const first = addon.modelForward(this._model, Int32Array.from(promptTokens), 0).next;
    const prefillTime = Date.now() - t0;
    all.push(first);
    if (opts.onToken) opts.onToken(first, 0);
    let generated = 1;
    const t1 = Date.now();
    if (first !== eosId && maxTokens > 1) {
      // the device loop stops at the first EOS too (no steps past it)
      const rest = addon.modelGenerate(this._model, first, promptTokens.length, maxTokens - 1,
        eosId);
      for (let i = 0; i < rest.length; i++) {
        all.push(rest[i]);
        generated++;
        if (opts.onToken) opts.onToken(rest[i], i + 1);
      }
    }
    const decodeTime = Date.now() - t1;
    const tokPerSec = Math.max(generated - 1, 1) / (Math.max(decodeTime, 1e-3) / 1000);
    return { tokens: all, generated, prefillTime, decodeTime, tokPerSec };
  }

  /** generate() with sampling: the loop of llama.js:452-505 over host logits. */
  _generateSampled(promptTokens, maxTokens, opts) {
    const temperature = opts.temperature || 0.8;
    const topK = opts.topK || 40;
    const eosId = opts.eosId || 2;
    this.resetCache();
    const all = [...promptTokens];
    const t0 = Date.now();
    const logits = this._logits(promptTokens, 0);
    const prefillTime = Date.now() - t0;
    let pos = promptTokens.length;
    let next = this.sample(logits, topK, temperature);
    all.push(next);
    if (opts.onToken) opts.onToken(next, 0);
    let generated = 1;
    const t1 = Date.now();
    for (let i = 1; i < maxTokens && next !== eosId; i++) {
      next = this.sample(this._logits([next], pos++), topK, temperature);
      all.push(next);
      generated++;
      if (opts.onToken) opts.onToken(next, i);
    }
    const decodeTime = Date.now() - t1;
    const tokPerSec = Math.max(generated - 1, 1) / (Math.max(decodeTime, 1e-3) / 1000);
    return { tokens: all, generated, prefillTime, decodeTime, tokPerSec };
  }

  free() {
    if (this._model) { addon.modelFree(this._model); this._model = null; }
  }
}

/**
 * The StreamingLlamaRuntime surface (llama-streaming.js:738-970) over the
 * same resident model: forward returns { logits, layersUsed } and takes
 * { maxLayers } (the first maxLayers layers, then the final norm and LM
 * head; later layers' caches are not written), sample scales in doubles,
 * and generate reports the reference's avgLayers / earlyExits.  Early exit
 * is not offered (the reference's path is disabled by default and cannot
 * run: llama-streaming.js:717 reads an undefined name).
 */
class HipStreamingLlamaRuntime extends HipLlamaRuntime {
  static fromGGUF(filePath, opts = {}) {
    const r = load().modelLoadGGUF(String(filePath), opts.maxSeq || 0);
    return new HipStreamingLlamaRuntime(r.config, r.model);
  }

  constructor(config, handle) {
    super(config, handle);
    this._layersUsed = 0;
    this._totalForwards = 0;
    this._earlyExits = 0;
    this._lastExitLayer = -1;
  }

  /** llama-streaming.js:738-815. */
  forward(tokenIds, startPos = 0, options = {}) {
    const r = addon.modelForward(this._model, Int32Array.from(tokenIds), startPos,
                                 options.maxLayers || 0);
    this._layersUsed += r.layersUsed;
    this._totalForwards++;
    this._lastExitLayer = r.layersUsed - 1;
    return { logits: r.logits, layersUsed: r.layersUsed };
  }

  async forwardAsync(tokenIds, startPos = 0, options = {}) {
    return this.forward(tokenIds, startPos, options);
  }

  /** llama-streaming.js:868-896 (the scaled logits stay doubles). */
  sample(logits, topK = 40, temperature = 0.8) {
    return sampleTopK(logits, topK, temperature, this.random, false);
  }

  _logits(tokenIds, startPos) { return this.forward(tokenIds, startPos).logits; }

  /** llama-streaming.js:914-970. */
  generate(promptTokens, maxTokens = 50, opts = {}) {
    this._layersUsed = 0;
    this._totalForwards = 0;
    this._earlyExits = 0;
    const nl = this.config.nLayers;
    let r;
    if (opts.greedy) {
      // the decode loop on the GPU: each of its steps runs every layer
      const onToken = opts.onToken;
      r = super.generate(promptTokens, maxTokens,
                         Object.assign({}, opts, onToken ? { onToken: (t, i) => onToken(t, i, nl) } : {}));
      this._totalForwards = r.generated;
      this._layersUsed = r.generated * nl;
    } else {
      r = this._generateSampled(promptTokens, maxTokens, opts);
    }
    r.avgLayers = this._totalForwards > 0 ? (this._layersUsed / this._totalForwards).toFixed(1) : nl;
    r.earlyExits = this._earlyExits;
    return r;
  }

  async generateAsync(promptTokens, maxTokens = 50, opts = {}) {
    return this.generate(promptTokens, maxTokens, opts);
  }

  get stats() {
    return {
      totalForwards: this._totalForwards,
      avgLayers: this._totalForwards > 0 ? (this._layersUsed / this._totalForwards).toFixed(1) : 0,
      earlyExits: this._earlyExits,
      lastExitLayer: this._lastExitLayer,
      wasmReady: false,
    };
  }

  async shutdown() { this.free(); }
}

/**
 * SelfSpeculativeDecoder (speculative.js:28-227) on the GPU: drafts with the
 * runtime's own first draftLayers layers and verifies with the full model.
 * Greedy rounds run in the C ABI (the draft chain on the device, the drafts
 * verified in one batched forward unless batchedVerify is false); with
 * sampling, each forward returns to the host for sample().
 */
class HipSelfSpeculativeDecoder {
  constructor(runtime, options = {}) {
    this.runtime = runtime;
    this.draftLayers = options.draftLayers || 4;
    this.draftCount = options.draftCount || 4;
    this.temperature = options.temperature || 0.6;
    this.topK = options.topK || 40;
    this.batchedVerify = options.batchedVerify !== false;
    this.resetStats();
  }

  resetStats() {
    this._totalRounds = 0;
    this._totalDrafted = 0;
    this._totalAccepted = 0;
  }

  get stats() {
    const d = this._totalDrafted;
    return {
      totalRounds: this._totalRounds, totalDrafted: d, totalAccepted: this._totalAccepted,
      acceptanceRate: d > 0 ? (this._totalAccepted / d * 100).toFixed(0) + '%' : 'N/A',
    };
  }

  _result(promptTokens, tokens, generated, prefillTime, decodeTime) {
    const tokPerSec = Math.max(generated - 1, 1) / (Math.max(decodeTime, 1e-3) / 1000);
    return {
      tokens: [...promptTokens, ...tokens], generated, prefillTime, decodeTime, tokPerSec,
      acceptanceRate: this.stats.acceptanceRate,
    };
  }

  generate(promptTokens, maxTokens = 50, opts = {}) {
    const eos = opts.eosIds || [2];
    if (opts.greedy) {
      const r = addon.selfSpeculative(this.runtime._model, Int32Array.from(promptTokens), maxTokens,
                                      this.draftLayers, this.draftCount, Int32Array.from(eos),
                                      this.batchedVerify);
      this._totalRounds += r.rounds;
      this._totalDrafted += r.drafted;
      this._totalAccepted += r.accepted;
      const toks = Array.from(r.tokens);
      if (opts.onToken) toks.forEach((t, i) => opts.onToken(t, i));
      return this._result(promptTokens, toks, toks.length, r.prefillMs, r.decodeMs);
    }
    return this._generateSampled(promptTokens, maxTokens, opts, eos);
  }

  // speculative.js:58-204 with sampling: draft with {maxLayers}, roll the
  // cache back, verify one forward per draft, keep the agreeing prefix.
  _generateSampled(promptTokens, maxTokens, opts, eos) {
    const rt = this.runtime;
    const temperature = opts.temperature || this.temperature;
    const topK = opts.topK || this.topK;
    const pick = (lg) => rt.sample(lg, topK, temperature);
    const isEos = (t) => eos.includes(t);
    rt.resetCache();
    const out = [];
    const emit = (t) => { out.push(t); if (opts.onToken) opts.onToken(t, out.length - 1); };
    const t0 = Date.now();
    let next = pick(rt.forward(promptTokens, 0).logits);
    const prefillTime = Date.now() - t0;
    let pos = promptTokens.length;
    emit(next);
    let done = isEos(next);
    const t1 = Date.now();
    while (out.length < maxTokens && !done) {
      const chain = [next];
      for (let d = 0; d < this.draftCount && out.length + d < maxTokens; d++) {
        const cur = chain[chain.length - 1];
        if (isEos(cur)) break;
        chain.push(pick(rt.forward([cur], pos + d, { maxLayers: this.draftLayers }).logits));
      }
      const nd = chain.length - 1;
      if (nd === 0) break;
      this._totalDrafted += nd;
      this._totalRounds++;
      rt.rollbackCache(pos);
      let accepted = 0;
      let rejected = false;
      for (let d = 0; d < nd && !done && !rejected; d++) {
        const v = pick(rt.forward([chain[d]], pos + d).logits);
        emit(v);
        if (isEos(v)) done = true;
        if (v === chain[d + 1]) {
          accepted++;
        } else {
          rejected = true;
          rt.rollbackCache(pos + d + 2);
        }
      }
      if (accepted === nd && !done) {
        const b = pick(rt.forward([chain[nd]], pos + nd).logits);
        emit(b);
        if (isEos(b)) done = true;
        pos += nd + 1;
      } else {
        pos += accepted + 1;
      }
      next = out[out.length - 1];
      this._totalAccepted += accepted;
    }
    return this._result(promptTokens, out, out.length, prefillTime, Date.now() - t1);
  }
}

/** speculative.js:58-204, greedy, draft from its own (smaller) model. */
class HipSpeculativeDecoder {
  constructor(target, draft, options = {}) {
    this.target = target;
    this.draft = draft;
    this.draftCount = options.draftCount || 4;
    this.batchedVerify = options.batchedVerify !== false;
  }

  generate(promptTokens, maxTokens = 50, opts = {}) {
    const eos = opts.eosIds || [2];
    const r = addon.speculative(this.target._model, this.draft._model, Int32Array.from(promptTokens),
                                maxTokens, this.draftCount, Int32Array.from(eos), this.batchedVerify);
    const generated = r.tokens.length;
    const tokPerSec = Math.max(generated - 1, 1) / (Math.max(r.decodeMs, 1e-3) / 1000);
    return {
      tokens: [...promptTokens, ...r.tokens],
      generated,
      prefillTime: r.prefillMs,
      decodeTime: r.decodeMs,
      tokPerSec,
      acceptanceRate: r.drafted > 0 ? (r.accepted / r.drafted * 100).toFixed(0) + '%' : 'N/A',
      rounds: r.rounds,
    };
  }
}

module.exports = { HipLlamaRuntime, HipStreamingLlamaRuntime, HipSelfSpeculativeDecoder,
                   HipSpeculativeDecoder, sampleTopK, tensorId, TYPES };
