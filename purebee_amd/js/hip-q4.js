/**
 * purebee_amd -- HIP drop-in for PureBee's quantized matvec module.
 *
 * Same surface and calling convention as wasm-q4.js (exports at
 * wasm-q4.js:841-847) and the quantizedMatvec dispatch of
 * llama-streaming.js:168-177: synchronous calls, Float32Array inputs,
 * a fresh Float32Array result, inputs never mutated.
 *
 * Difference by design: the raw block bytes are NOT copied on every call
 * (the reference copies x and the whole weight slice into WASM memory each
 * time, wasm-q4.js:735-738).  The first call with a given byte range uploads
 * it once to the GPU (pinned staging, then repacked for the kernels); later
 * calls reuse the resident copy.  The cache is keyed by (ArrayBuffer,
 * byteOffset, type, N, K), so callers must not rewrite weight bytes in place
 * (call invalidate(rawBuf) if they do).  Weights are immutable in the
 * reference's loaders (streaming-loader.js:245-262).
 *
 * Written for Node >= 10 (no optional chaining / nullish coalescing).
 */
'use strict';

const path = require('path');

const GGML_TYPE = { F32: 0, Q4_0: 2, Q4_1: 3, Q8_0: 8 };
const BLOCK_BYTES = { 2: 18, 3: 20, 8: 34 };

let addon = null;
let _supported = false;
let _initError = null;

function loadAddon() {
  if (!addon) addon = require(path.join(__dirname, '..', 'lib', 'pbx_napi.node'));
  return addon;
}

/**
 * Initialise the GPU backend. Synchronous, like wasm-q4.js:647-668: the
 * addon and device, then the module's known-answer test
 * (wasm-q4.js:673-704) on the GPU; false when either fails.
 * @returns {boolean} true if the HIP kernels are available and correct
 */
function init(device) {
  if (_supported) return true;
  try {
    loadAddon().init(device || 0);
    _supported = true;
    _initError = null;
  } catch (e) {
    _supported = false;
    _initError = e;
    return false;
  }
  let ok = false;
  try {
    ok = selfTest();
  } catch (e) {
    _initError = e;
  }
  if (!ok) {
    _supported = false;
    if (!_initError) _initError = new Error('Q4_0 self-test failed');
  }
  return _supported;
}

/**
 * wasm-q4.js:673-704: two Q4_0 rows of one block against x = 1: scale 1 with
 * every code 9 gives 32, scale 2 with every code 10 gives 128.  Its bytes are
 * uploaded once and freed after the check (no resident cache entry).
 */
function selfTest() {
  const K = 32, N = 2;
  const x = new Float32Array(K).fill(1.0);
  const raw = new Uint8Array(36);
  raw[0] = 0x00; raw[1] = 0x3C;  // fp16 1.0
  for (let j = 2; j < 18; j++) raw[j] = 0x99;
  raw[18] = 0x00; raw[19] = 0x40;  // fp16 2.0
  for (let j = 20; j < 36; j++) raw[j] = 0xAA;
  const h = addon.upload(GGML_TYPE.Q4_0, N, K, raw);
  let r;
  try {
    r = addon.linear(h, x, 1, null);
  } finally {
    addon.free(h);
  }
  return Math.abs(r[0] - 32.0) < 0.1 && Math.abs(r[1] - 128.0) < 0.1;
}

function ensure() {
  if (!_supported && !init()) {
    const why = _initError ? `: ${_initError.message}` : '';
    throw new Error(`HIP Q4 not available${why}`);
  }
}

// ── resident weights ──────────────────────────────────────────────
const residency = new WeakMap();  // ArrayBuffer -> Map(key -> handle)

function asBytes(buf) {
  if (buf instanceof Uint8Array) return buf;
  return new Uint8Array(buf.buffer, buf.byteOffset, buf.byteLength);
}

function residentHandle(view, type, N, K, upload) {
  let m = residency.get(view.buffer);
  if (!m) {
    m = new Map();
    residency.set(view.buffer, m);
  }
  const key = `${type}:${view.byteOffset}:${N}:${K}`;
  let h = m.get(key);
  if (!h) {
    h = upload();
    m.set(key, h);
  }
  return h;
}

function quantHandle(rawBuf, type, N, K) {
  const u8 = asBytes(rawBuf);
  const need = N * (K >>> 5) * BLOCK_BYTES[type];
  if (u8.byteLength < need) {
    throw new Error(`raw buffer holds ${u8.byteLength} bytes, ${N}x${K} needs ${need}`);
  }
  return residentHandle(u8, type, N, K, () => addon.upload(type, N, K, u8.subarray(0, need)));
}

/** Drop the resident copies made from this buffer (all offsets). */
function invalidate(buf) {
  const ab = buf instanceof ArrayBuffer || (typeof SharedArrayBuffer !== 'undefined' && buf instanceof SharedArrayBuffer)
    ? buf : buf.buffer;
  const m = residency.get(ab);
  if (!m) return;
  for (const h of m.values()) addon.free(h);
  residency.delete(ab);
}

// ── the instruction ───────────────────────────────────────────────

/**
 * Q4_0 matvec: y[N] = W_q4[N,K] @ x[K].  Signature of wasm-q4.js:716.
 * @param {Float32Array} x
 * @param {Uint8Array|Buffer} rawBuf GGUF Q4_0 blocks, N rows x K/32 blocks x 18 B
 * @param {number} N
 * @param {number} K multiple of 32
 * @returns {Float32Array} [N]
 */
function q4_0_matvec(x, rawBuf, N, K) {
  ensure();
  return addon.linear(quantHandle(rawBuf, GGML_TYPE.Q4_0, N, K), x, 1, null);
}

/** Q8_0 matvec on GGUF Q8_0 blocks (34 B per 32 values). */
function q8_0_matvec(x, rawBuf, N, K) {
  ensure();
  return addon.linear(quantHandle(rawBuf, GGML_TYPE.Q8_0, N, K), x, 1, null);
}

/**
 * Q4_1 matvec: y[N] = W_q4_1[N,K] @ x[K].  Signature of wasm-q4.js:758;
 * 20-byte blocks (fp16 d, fp16 m, 16 nibble bytes), value = nibble*d + m.
 */
function q4_1_matvec(x, rawBuf, N, K) {
  ensure();
  return addon.linear(quantHandle(rawBuf, GGML_TYPE.Q4_1, N, K), x, 1, null);
}

/**
 * Dispatch by GGML type, as quantizedMatvec (llama-streaming.js:168-177).
 */
function matvec(x, rawBuf, type, N, K) {
  if (type === GGML_TYPE.Q4_0) return q4_0_matvec(x, rawBuf, N, K);
  if (type === GGML_TYPE.Q4_1) return q4_1_matvec(x, rawBuf, N, K);
  if (type === GGML_TYPE.Q8_0) return q8_0_matvec(x, rawBuf, N, K);
  throw new Error(`Unsupported quant type for matvec: ${type}`);
}

/**
 * f32 LM head: logits[v] = sum_d hidden[d] * emb[v*dim + d]
 * (wasm-q4.js:798-839).  The embedding is made resident on first use.
 */
function lmHead(hidden, embData, vocabSize, dim) {
  ensure();
  if (embData.length < vocabSize * dim) throw new Error('lmHead: embedding shorter than vocabSize*dim');
  const view = embData.length === vocabSize * dim ? embData : embData.subarray(0, vocabSize * dim);
  const h = residentHandle(view, GGML_TYPE.F32, vocabSize, dim,
    () => addon.upload(GGML_TYPE.F32, vocabSize, dim, view));
  return addon.linear(h, hidden, 1, null);
}

/**
 * Quantized LM head on a resident Q4_0 / Q8_0 tied embedding (the GGUF
 * token_embd bytes), numerically the f32 head on the exactly dequantised
 * embedding up to summation order (gguf.js:259-286 dequant is exact).
 */
function lmHeadQuant(hidden, rawBuf, type, vocabSize, dim) {
  return matvec(hidden, rawBuf, type, vocabSize, dim);
}

module.exports = {
  init,
  selfTest,
  q4_0_matvec,
  q4_1_matvec,
  q8_0_matvec,
  matvec,
  lmHead,
  lmHeadQuant,
  invalidate,
  GGML_TYPE,
  get supported() { return _supported; },
  get addon() { ensure(); return addon; },
};
