/**
 * purebee_amd JS entry point.
 *   hipQ4    -- wasm-q4.js-shaped module (q4_0_matvec, lmHead, matvec, ...)
 *   hipSimd  -- wasm-simd.js-shaped module (allocWeights, matmulCached, ...)
 *   engine   -- ExecutionEngine matmul adapter (HipEngine, install)
 */
'use strict';

module.exports = {
  hipQ4: require('./hip-q4'),
  hipSimd: require('./hip-simd'),
  engine: require('./engine-hip'),
};
