/**
 * purebee_amd -- HIP backend for PureBee's engine-level matmul ops.
 *
 * Drop-in for the matmul methods of ExecutionEngine (engine.js:17-494) that
 * PureBee.LINEAR / TENSOR_MUL call (purebee.js:61-88):
 *   tensorMul(A[M,K], B[K,N], outName)            engine.js:119-167
 *   tensorMulAdd(x[M,K], W[K,N], b|null, outName)  engine.js:180-244
 *   tensorMulAddQ8(x[M,K], Wq, b|null, outName)    engine.js:259-269 (matmul_q8)
 *   cacheWeight(tensor)                             engine.js:39-42
 *   initWasm()                                      engine.js:28-31
 * Weights keep the reference's [K,N] orientation at this seam; they are
 * transposed once to the C ABI's [N,K] when made resident.  Results are
 * Tensor objects built with the input tensor's own class, so the reference's
 * PureBee memory (purebee.js:81-86) stores them unchanged.
 *
 * install(purebee) swaps these methods into a PureBee instance's engine and
 * leaves every other op (softmax, rmsNorm, attention, ...) on the original.
 */
'use strict';

const hipq = require('./hip-q4');

const F32 = 0;

class PlainTensor {
  constructor(name, shape, data) {
    this.name = name;
    this.shape = shape;
    this.size = shape.reduce((a, b) => a * b, 1);
    this.data = data || new Float32Array(this.size);
  }
}

function makeTensor(like, name, shape, data) {
  const C = like && typeof like.constructor === 'function' && like.constructor !== Object
    ? like.constructor : PlainTensor;
  try {
    const t = new C(name, shape, data);
    if (t && t.data === data) return t;
  } catch (e) { /* fall through */ }
  return new PlainTensor(name, shape, data);
}

function transposeKN(data, K, N) {
  const out = new Float32Array(K * N);
  for (let k = 0; k < K; k++) {
    const row = k * N;
    for (let n = 0; n < N; n++) out[n * K + k] = data[row + n];
  }
  return out;
}

class HipEngine {
  constructor(options) {
    const opts = options || {};
    this._device = opts.device || 0;
    this._ready = false;
    this._opCount = 0;
    this._flops = 0;
  }

  /** engine.js:28-31 -- returns true when the GPU backend is usable. */
  initWasm() {
    this._ready = hipq.init(this._device);
    return this._ready;
  }

  _addon() {
    if (!this._ready && !this.initWasm()) {
      throw new Error('HIP engine not available (no GPU or addon not built)');
    }
    return hipq.addon;
  }

  /** engine.js:39-42: make a [K,N] f32 weight resident; sets tensor._hipW. */
  cacheWeight(tensor) {
    const addon = this._addon();
    if (tensor._hipW) return;
    const K = tensor.shape[0], N = tensor.shape[1];
    tensor._hipW = addon.upload(F32, N, K, transposeKN(tensor.data, K, N));
  }

  _f32Handle(W) {
    if (W._hipW) return { h: W._hipW, temp: false };
    const K = W.shape[0], N = W.shape[1];
    return { h: this._addon().upload(F32, N, K, transposeKN(W.data, K, N)), temp: true };
  }

  _run(x, h, M, N, bias, outName, like) {
    const addon = this._addon();
    const y = addon.linear(h, x.data, M, bias ? bias.data : null);
    return makeTensor(like, outName, [M, N], y);
  }

  /** engine.js:119-167 */
  tensorMul(A, B, outName) {
    const M = A.shape[0], K = A.shape[1];
    const K2 = B.shape[0], N = B.shape[1];
    if (K !== K2) throw new Error(`TENSOR_MUL: dimension mismatch A[${M},${K}] x B[${K2},${N}]`);
    const r = this._f32Handle(B);
    try {
      this._opCount++;
      this._flops += M * N * K * 2;
      return this._run(A, r.h, M, N, null, outName || 'matmul_out', A);
    } finally {
      if (r.temp) this._addon().free(r.h);
    }
  }

  /** engine.js:180-244 */
  tensorMulAdd(x, W, b, outName) {
    const M = x.shape[0], K = x.shape[1];
    const K2 = W.shape[0], N = W.shape[1];
    if (K !== K2) throw new Error('TENSOR_MUL_ADD: dimension mismatch');
    const r = this._f32Handle(W);
    try {
      this._opCount++;
      this._flops += M * N * K * 2 + (b ? M * N : 0);
      return this._run(x, r.h, M, N, b, outName || 'linear_out', x);
    } finally {
      if (r.temp) this._addon().free(r.h);
    }
  }

  /**
   * engine.js:259-269 -> matmul_q8 (quantize.js:224-266) on the reference's
   * QuantizedTensor 'q8_0' ([K,N], flat int8, f32 scale per 32 elements).
   */
  tensorMulAddQ8(x, Wq, b, outName) {
    if (Wq.type !== 'q8_0') throw new Error(`tensorMulAddQ8: unsupported QuantizedTensor type ${Wq.type}`);
    const addon = this._addon();
    const M = x.shape[0], K = x.shape[1];
    const N = Wq.shape[1];
    if (Wq.shape[0] !== K) throw new Error('TENSOR_MUL_ADD_Q8: dimension mismatch');
    if (!Wq._hipW) Wq._hipW = addon.uploadQ8Ref(K, N, Wq.data, Wq.scales);
    this._opCount++;
    this._flops += M * N * K * 2 + (b ? M * N : 0);
    return this._run(x, Wq._hipW, M, N, b, outName || 'linear_q8_out', x);
  }

  get stats() {
    return { ops: this._opCount, flops: this._flops };
  }
}

/**
 * Route a PureBee instance's matmul instructions to the GPU.
 * @param {object} purebee  a PureBee (purebee.js:27-211)
 * @returns {HipEngine}
 */
function install(purebee, options) {
  const hip = new HipEngine(options);
  if (!hip.initWasm()) throw new Error('HIP engine not available');
  const eng = purebee.engine;
  const orig = {
    tensorMul: eng.tensorMul, tensorMulAdd: eng.tensorMulAdd,
    tensorMulAddQ8: eng.tensorMulAddQ8, cacheWeight: eng.cacheWeight, initWasm: eng.initWasm,
  };
  eng.tensorMul = (A, B, n) => hip.tensorMul(A, B, n);
  eng.tensorMulAdd = (x, W, bb, n) => hip.tensorMulAdd(x, W, bb, n);
  eng.tensorMulAddQ8 = (x, Wq, bb, n) => hip.tensorMulAddQ8(x, Wq, bb, n);
  eng.cacheWeight = t => hip.cacheWeight(t);
  eng.initWasm = () => hip.initWasm();
  eng._hip = hip;
  eng._hipOriginal = orig;
  return hip;
}

module.exports = { HipEngine, install, PlainTensor };
