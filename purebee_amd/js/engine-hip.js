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
 *   wasmStats                                       engine.js:44-46
 * and resetWeights(), the release the streaming runtime gets from
 * wasmSimd.resetWeights (wasm-simd.js:511-513): cached f32 weights belong to
 * hip-simd.js, the module that replaces wasm-simd.js.
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
const hipSimd = require('./hip-simd');


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

class HipEngine {
  constructor(options) {
    const opts = options || {};
    this._device = opts.device || 0;
    this._ready = false;
    this._opCount = 0;
    this._flops = 0;
  }

  /** engine.js:28-31 -- true when the GPU backend passed its self-tests. */
  initWasm() {
    this._ready = hipSimd.init(this._device);
    return this._ready;
  }

  _addon() {
    if (!this._ready && !this.initWasm()) {
      throw new Error('HIP engine not available (no GPU or addon not built)');
    }
    return hipq.addon;
  }

  /**
   * engine.js:39-42: make a [K,N] f32 weight resident.  The block belongs to
   * the f32 matmul module (hip-simd.js): resetWeights() releases it, as the
   * streaming runtime's per-layer wasmSimd.resetWeights() does
   * (llama-streaming.js:367-380), and the next cacheWeight makes it again.
   */
  cacheWeight(tensor) {
    this._addon();
    if (tensor._hipW !== undefined && hipSimd.isLive(tensor._hipW)) return;
    tensor._hipW = hipSimd.allocWeights(tensor.data, tensor.shape[0], tensor.shape[1]);
  }

  /** wasm-simd.js:511-513 through this engine: every cached weight released. */
  resetWeights() {
    hipSimd.resetWeights();
  }

  /** engine.js:44-46 */
  get wasmStats() {
    return this._ready ? hipSimd.getStats() : null;
  }

  _cached(W) {
    return W._hipW !== undefined && hipSimd.isLive(W._hipW);
  }

  /** engine.js:119-167 */
  tensorMul(A, B, outName) {
    const M = A.shape[0], K = A.shape[1];
    const K2 = B.shape[0], N = B.shape[1];
    if (K !== K2) throw new Error(`TENSOR_MUL: dimension mismatch A[${M},${K}] x B[${K2},${N}]`);
    this._addon();
    const out = new Float32Array(M * N);
    if (this._cached(B)) hipSimd.matmulCached(A.data, M, K, B._hipW, N, null, out);
    else hipSimd.matmul_general(A.data, M, K, B.data, N, out);
    this._opCount++;
    this._flops += M * N * K * 2;
    return makeTensor(A, outName || 'matmul_out', [M, N], out);
  }

  /** engine.js:180-244 */
  tensorMulAdd(x, W, b, outName) {
    const M = x.shape[0], K = x.shape[1];
    const K2 = W.shape[0], N = W.shape[1];
    if (K !== K2) throw new Error('TENSOR_MUL_ADD: dimension mismatch');
    const addon = this._addon();
    const out = new Float32Array(M * N);
    if (this._cached(W)) {
      hipSimd.matmulCached(x.data, M, K, W._hipW, N, b ? b.data : null, out);
    } else {
      // one pass with the bias in the epilogue (the reference adds it after
      // its general matmul, engine.js:205-214: the same sums)
      const h = hipSimd.uploadKN(W.data, K, N);
      try {
        out.set(hipSimd.linearKN(h, x.data, M, K, b ? b.data : null));
      } finally {
        addon.free(h);
      }
    }
    this._opCount++;
    this._flops += M * N * K * 2 + (b ? M * N : 0);
    return makeTensor(x, outName || 'linear_out', [M, N], out);
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
    const y = addon.linear(Wq._hipW, x.data, M, b ? b.data : null);
    return makeTensor(x, outName || 'linear_q8_out', [M, N], y);
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
