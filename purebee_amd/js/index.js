/**
 * purebee_amd JS entry point.
 *   hipQ4    -- wasm-q4.js-shaped module (q4_0_matvec, lmHead, matvec, ...)
 *   engine   -- ExecutionEngine matmul adapter (HipEngine, install)
 */
'use strict';

module.exports = {
  hipQ4: require('./hip-q4'),
  engine: require('./engine-hip'),
};
