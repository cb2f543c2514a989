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
 * HipSpeculativeDecoder follows SelfSpeculativeDecoder.generate
 * (speculative.js:58-204) in greedy mode with a separate draft model.
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
    this.config = Object.assign({}, c);
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

  resetCache() { addon.modelReset(this._model); }

  rollbackCache(pos) { addon.modelRollback(this._model, pos); }

  /**
   * llama.js:452-505 in greedy mode: prefill, then the decode loop on the GPU
   * (the argmax of each step feeds the next without returning to the host);
   * tokens after the first eosId are dropped as the reference stops there.
   */
  generate(promptTokens, maxTokens = 50, opts = {}) {
    if (!opts.greedy) throw new Error('HipLlamaRuntime.generate: only greedy decoding runs on the GPU');
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
      const rest = addon.modelGenerate(this._model, first, promptTokens.length, maxTokens - 1);
      for (let i = 0; i < rest.length; i++) {
        all.push(rest[i]);
        generated++;
        if (opts.onToken) opts.onToken(rest[i], i + 1);
        if (rest[i] === eosId) break;
      }
    }
    const decodeTime = Date.now() - t1;
    const tokPerSec = Math.max(generated - 1, 1) / (Math.max(decodeTime, 1e-3) / 1000);
    return { tokens: all, generated, prefillTime, decodeTime, tokPerSec };
  }

  free() {
    if (this._model) { addon.modelFree(this._model); this._model = null; }
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

module.exports = { HipLlamaRuntime, HipSpeculativeDecoder, tensorId, TYPES };
