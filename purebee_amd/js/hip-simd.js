/**
 * purebee_amd -- HIP drop-in for PureBee's f32 matmul module.
 *
 * Same surface and calling convention as wasm-simd.js (exports at
 * wasm-simd.js:527-535), which engine.js (initWasm / cacheWeight /
 * tensorMul / tensorMulAdd, engine.js:28-42, 119-244) and the streaming
 * runtime's per-layer weight cycle (llama-streaming.js:367-392, 639, 658)
 * call directly:
 *   init()                                   -> boolean (runs the module's KAT)
 *   allocWeights(data)                       -> pointer (number)
 *   matmul_general(a, M, K, b, N, out)       out[M,N] = a[M,K] x b[K,N]
 *   matmulCached(x, M, K, ptr, N, bias, out) out[M,N] = x[M,K] x W[K,N] + bias
 *   resetWeights()                           releases every allocWeights block
 *   getStats()                               { supported, totalMemoryMB, weightsMB, scratchMB }
 * Synchronous calls, caller-owned output arrays, inputs never mutated.
 *
 * Pointers are what the reference's are, byte offsets of a bump allocator
 * past a 4 MB scratch region (wasm-simd.js:14-32, 406-414), so stats and
 * pointer arithmetic read the same; behind each one is a weight resident in
 * HBM.  allocWeights copies the data, as the reference copies it into WASM
 * memory; a block becomes resident (transposed once to the C ABI's [N,K])
 * when the first matmulCached names its shape, or at once when the shape is
 * passed (allocWeights(data, K, N), as HipEngine.cacheWeight does), and the
 * host copy is dropped then.  resetWeights frees the device copies too, so
 * a caller that re-caches every layer's weights per forward (the streaming
 * runtime's prefill) holds one layer's weights at a time, as it does in
 * WASM memory.
 *
 * Written for Node >= 10 (no optional chaining / nullish coalescing).
 */
'use strict';

const hipq = require('./hip-q4');

const F32 = 0;
const SCRATCH_SIZE = 4 * 1024 * 1024;  // wasm-simd.js:24
const MB = 1024 * 1024;

let _supported = false;
let bumpPtr = SCRATCH_SIZE;
let residentBytes = 0;
const blocks = new Map();  // pointer -> { data, length, shape, handle }

// The C ABI takes weights as [N rows][K columns] with K a multiple of 32;
// the reference's matmuls take any K.  Columns past K are zero in the
// resident copy, and activation rows are padded to match (the sums are the
// same: the padded terms are 0 * 0).
function padK(K) {
  return (K + 31) & ~31;
}

/** [K,N] row-major -> [N,Kp] row-major, Kp = K rounded up to 32. */
function transposeKN(data, K, N) {
  const Kp = padK(K);
  const out = new Float32Array(Kp * N);
  for (let k = 0; k < K; k++) {
    const row = k * N;
    for (let n = 0; n < N; n++) out[n * Kp + k] = data[row + n];
  }
  return out;
}

/** A [K,N] f32 weight made resident (a device handle). */
function uploadKN(data, K, N) {
  return hipq.addon.upload(F32, N, padK(K), transposeKN(data, K, N));
}

/** y[M,N] = x[M,K] W + bias on a handle from uploadKN. */
function linearKN(h, xData, M, K, biasData) {
  const Kp = padK(K);
  let x = xData;
  if (Kp !== K) {
    x = new Float32Array(M * Kp);
    for (let m = 0; m < M; m++) x.set(xData.subarray(m * K, m * K + K), m * Kp);
  }
  return hipq.addon.linear(h, x, M, biasData || null);
}

/**
 * wasm-simd.js:339-360: the backend, then its self-test (2x3 @ 3x5,
 * wasm-simd.js:365-385); false when either fails.
 */
function init(device) {
  if (_supported) return true;
  if (!hipq.init(device)) return false;
  _supported = true;
  let ok = false;
  try {
    ok = selfTest();
  } catch (e) {
    ok = false;
  }
  if (!ok) _supported = false;
  bumpPtr = SCRATCH_SIZE;
  return _supported;
}

function selfTest() {
  const M = 2, K = 3, N = 5;
  const A = new Float32Array([1, 2, 3, 4, 5, 6]);
  const B = new Float32Array([
    1, 0, 0, 0, 0,
    0, 1, 0, 0, 0,
    0, 0, 1, 0, 0,
  ]);
  const C = new Float32Array(M * N);
  const expected = [1, 2, 3, 0, 0, 4, 5, 6, 0, 0];
  matmul_general(A, M, K, B, N, C);
  for (let i = 0; i < C.length; i++) {
    if (Math.abs(C[i] - expected[i]) > 1e-5) return false;
  }
  return true;
}

function ensure(what) {
  if (!_supported) throw new Error(`${what}: HIP SIMD matmul not initialised (call init())`);
  return hipq.addon;
}

function makeResident(b, K, N) {
  b.handle = uploadKN(b.data, K, N);
  b.shape = `${K}:${N}`;
  b.data = null;
  residentBytes += padK(K) * N * 4;
}

/**
 * wasm-simd.js:406-414.  data: the [K,N] weight (flat Float32Array).  With
 * K and N given the block is made resident at once.
 */
function allocWeights(data, K, N) {
  ensure('allocWeights');
  const aligned = (bumpPtr + 15) & ~15;
  const b = { data: Float32Array.from(data), length: data.length, shape: null, handle: null };
  if (K && N) {
    if (K * N !== data.length) throw new Error(`allocWeights: ${data.length} values, not ${K}x${N}`);
    makeResident(b, K, N);
  }
  blocks.set(aligned, b);
  bumpPtr = aligned + data.length * 4;
  return aligned;
}

/** True when ptr is a block of the current allocation (not reset since). */
function isLive(ptr) {
  return blocks.has(ptr);
}

/** wasm-simd.js:427-454: C = A x B with both operands copied per call. */
function matmul_general(aData, M, K, bData, N, outData) {
  const addon = ensure('matmul_general');
  const h = uploadKN(bData, K, N);
  try {
    outData.set(linearKN(h, aData, M, K, null));
  } finally {
    addon.free(h);
  }
}

/**
 * wasm-simd.js:469-506: out = x x W + bias on the weight allocWeights
 * returned `wPtr` for.
 */
function matmulCached(xData, M, K, wPtr, N, biasData, outData) {
  const addon = ensure('matmulCached');
  const b = blocks.get(wPtr);
  if (!b) throw new Error(`matmulCached: ${wPtr} is not a live allocWeights pointer`);
  if (K * N > b.length) throw new Error(`matmulCached: ${K}x${N} exceeds the block's ${b.length} values`);
  const shape = `${K}:${N}`;
  if (!b.handle) {
    if (K * N !== b.length) {
      // a view of the front of the block: made resident from a copy of it
      b.data = b.data.subarray(0, K * N);
    }
    makeResident(b, K, N);
  } else if (b.shape !== shape) {
    throw new Error(`matmulCached: block made resident as ${b.shape.replace(':', 'x')}, called as ${K}x${N}`);
  }
  outData.set(linearKN(b.handle, xData, M, K, biasData));
}

/** wasm-simd.js:511-513: every block released (device memory too). */
function resetWeights() {
  if (_supported) {
    const addon = hipq.addon;
    for (const b of blocks.values()) if (b.handle) addon.free(b.handle);
  }
  blocks.clear();
  residentBytes = 0;
  bumpPtr = SCRATCH_SIZE;
}

/** wasm-simd.js:518-525, plus the bytes resident in HBM. */
function getStats() {
  return {
    supported: _supported,
    totalMemoryMB: (bumpPtr / MB).toFixed(1),
    weightsMB: ((bumpPtr - SCRATCH_SIZE) / MB).toFixed(1),
    scratchMB: (SCRATCH_SIZE / MB).toFixed(1),
    residentMB: (residentBytes / MB).toFixed(1),
  };
}

module.exports = {
  init,
  allocWeights,
  matmul_general,
  matmulCached,
  resetWeights,
  getStats,
  isLive,
  uploadKN,
  linearKN,
  get supported() { return _supported; },
};
