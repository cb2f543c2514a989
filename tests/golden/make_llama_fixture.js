/**
 * Writes tests/golden/llama_tiny.json: prompt logits and greedy decode logits
 * of the reference's own LlamaRuntime (llama.js, JS fallback path) for a tiny
 * Llama with seeded f32 weights.  Run in a container that holds the
 * reference checkout:
 *     node tests/golden/make_llama_fixture.js [/path/to/purebee]
 * The weights come from a 32-bit LCG that tests/golden/llama_fixture.py
 * reproduces bit for bit, so the fixture holds only token ids and logits.
 */
'use strict';

const fs = require('fs');
const path = require('path');

const REF = process.argv[2] || '/root/reference';
const { LlamaRuntime, LlamaConfig } = require(path.join(REF, 'llama.js'));

// Config: head_dim 32, GQA 4 query heads over 2 KV heads.
const CFG = { dim: 128, hiddenDim: 256, nLayers: 2, nHeads: 4, nKvHeads: 2, vocabSize: 97,
              seqLen: 32, ropeTheta: 10000.0 };
const SEED = 20261201;
const PROMPT = [3, 14, 15, 92, 65, 35];
const DECODE_STEPS = 6;

function lcg(seed) {
  let s = seed >>> 0;
  return () => {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    return s;
  };
}

// n values of ((u >>> 8) / 2^24 - 0.5) * scale (+ offset), rounded to f32.
function draw(seed, n, scale, offset) {
  const g = lcg(seed);
  const out = new Float32Array(n);
  for (let i = 0; i < n; i++) out[i] = ((g() >>> 8) / 16777216 - 0.5) * scale + (offset || 0);
  return out;
}

// [N,K] (out, in) -> the reference's [K,N] LINEAR layout.
function transpose(w, N, K) {
  const t = new Float32Array(N * K);
  for (let n = 0; n < N; n++) for (let k = 0; k < K; k++) t[k * N + n] = w[n * K + k];
  return t;
}

const { dim, hiddenDim, nLayers, nHeads, nKvHeads, vocabSize } = CFG;
const headDim = dim / nHeads;
const kvDim = nKvHeads * headDim;
const weights = {};
let s = SEED;
weights.token_embedding = draw(s++, vocabSize * dim, 1.0);
weights.rms_final = draw(s++, dim, 0.4, 1.0);
for (let l = 0; l < nLayers; l++) {
  weights[`layer${l}.rms_att`] = draw(s++, dim, 0.4, 1.0);
  weights[`layer${l}.rms_ffn`] = draw(s++, dim, 0.4, 1.0);
  const shapes = [['wq', dim, dim], ['wk', kvDim, dim], ['wv', kvDim, dim], ['wo', dim, dim],
                  ['w1', hiddenDim, dim], ['w3', hiddenDim, dim], ['w2', dim, hiddenDim]];
  for (const [name, N, K] of shapes) {
    weights[`layer${l}.${name}`] = transpose(draw(s++, N * K, 0.4), N, K);
  }
}

const config = new LlamaConfig(CFG);
const log = console.log;
console.log = () => {};
const rt = new LlamaRuntime(config, { noWasm: true });
rt.loadWeights(weights, true);
const steps = [];
let logits = rt.forward(PROMPT, 0);
steps.push({ pos: 0, tokens: PROMPT, logits: Array.from(logits), argmax: rt.argmax(logits) });
let pos = PROMPT.length;
let tok = rt.argmax(logits);
for (let i = 0; i < DECODE_STEPS; i++) {
  logits = rt.forward([tok], pos);
  const next = rt.argmax(logits);
  steps.push({ pos, tokens: [tok], logits: Array.from(logits), argmax: next });
  tok = next;
  pos++;
}
console.log = log;

const out = {
  generator: 'tests/golden/make_llama_fixture.js (reference llama.js LlamaRuntime, noWasm)',
  config: CFG, seed: SEED, weight_order: ['token_embedding', 'rms_final',
    'per layer: rms_att, rms_ffn, wq, wk, wv, wo, w1, w3, w2 (each drawn as [N,K])'],
  steps,
};
fs.writeFileSync(path.join(__dirname, 'llama_tiny.json'), JSON.stringify(out));
log(`wrote ${steps.length} steps, tokens ${steps.map(x => x.argmax).join(',')}`);
