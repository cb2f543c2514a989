"""The oracle -- TEST INFRASTRUCTURE, NOT PART OF THE PRODUCT.

numpy front end of oracle/liboracle.so (built by oracle/build.py from
pb_oracle.c and cpu_baseline.c): a CPU restatement of PureBee's quantized
matvec arithmetic, with the reference file:line of each function in the C
sources.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
import this package, and only as the checker / the timed CPU baseline.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


class _PboCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("dim", "hidden", "n_layers", "n_heads", "n_kv",
                                            "head_dim", "vocab", "max_seq")] + \
               [("theta", ctypes.c_double), ("eps", ctypes.c_double)]


_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from . import build as _b
            _b.build()
        L = ctypes.CDLL(LIB_PATH)
        L.pbo_f16_to_f32.restype = ctypes.c_float
        L.pbo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.pbo_f16_to_f32_wasm.restype = ctypes.c_float
        L.pbo_f16_to_f32_wasm.argtypes = [ctypes.c_uint16]
        L.pbo_f64_to_f16.restype = ctypes.c_uint16
        L.pbo_f64_to_f16.argtypes = [ctypes.c_double]
        for name in ("pbo_dequant_q4_0", "pbo_dequant_q8_0", "pbo_dequant_q4_1", "pbo_dequant_f16",
                     "pbo_dequant_q6_k"):
            getattr(L, name).argtypes = [_u8p, _i64, _f32p]
        L.pbo_dequant_q8_ref.argtypes = [_i8p, _f32p, _i64, _f32p]
        for name in ("pbo_q4_0_matvec_js", "pbo_q4_0_matvec_wasm", "pbo_q8_0_matvec_f64",
                     "pbo_cpu_q4_0_matvec", "pbo_q4_1_matvec_js", "pbo_q4_1_matvec_wasm"):
            getattr(L, name).argtypes = [_f32p, _u8p, _i64, _i64, _f32p]
        for name in ("pbo_f32_matvec_f64", "pbo_batch_dot_wasm"):
            getattr(L, name).argtypes = [_f32p, _f32p, _i64, _i64, _f32p]
        L.pbo_matmul_f32_axpy.argtypes = [_f32p, _i64, _i64, _f32p, _i64, ctypes.c_void_p, _f32p]
        L.pbo_matmul_q8_ref.argtypes = [_f32p, _i64, _i64, _i8p, _f32p, _i64, ctypes.c_void_p, _f32p]
        L.pbo_quantize_q8_ref.argtypes = [_f32p, _i64, _i8p, _f32p]
        for name in ("pbo_quantize_q8_0", "pbo_quantize_q4_0", "pbo_quantize_q4_1",
                     "pbo_quantize_q6_k"):
            getattr(L, name).argtypes = [_f32p, _i64, _i64, _u8p]
        L.pbo_synth_normal.argtypes = [ctypes.c_uint64, _i64, ctypes.c_double, ctypes.c_double, _f32p]
        L.pbo_pool_create.restype = ctypes.c_void_p
        L.pbo_pool_create.argtypes = [ctypes.c_int]
        L.pbo_pool_destroy.argtypes = [ctypes.c_void_p]
        L.pbo_pool_q4_0_matvec.argtypes = [ctypes.c_void_p, _f32p, _u8p, _i64, _i64, _f32p]
        L.pbo_cpu_lm_head.argtypes = [_f32p, _f32p, _i64, _i64, _f32p]
        L.pbo_llama_create.restype = ctypes.c_void_p
        L.pbo_llama_create.argtypes = [ctypes.POINTER(_PboCfg)]
        L.pbo_llama_set.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _f32p]
        L.pbo_llama_forward.argtypes = [ctypes.c_void_p, np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS"),
                                        ctypes.c_int, ctypes.c_int, _f32p]
        L.pbo_llama_forward_layers.argtypes = [
            ctypes.c_void_p, np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS"),
            ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.pbo_llama_rollback.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.pbo_llama_free.argtypes = [ctypes.c_void_p]
        L.pbo_argmax.restype = ctypes.c_int
        L.pbo_argmax.argtypes = [_f32p, ctypes.c_int]
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def f16_to_f32(bits):
    return lib().pbo_f16_to_f32(int(bits))


def f16_to_f32_wasm(bits):
    return lib().pbo_f16_to_f32_wasm(int(bits))


def f64_to_f16(v):
    return lib().pbo_f64_to_f16(float(v))


def block_bytes(ggml_type):
    return {2: 18, 3: 20, 8: 34}[ggml_type]


def row_bytes(ggml_type, K):
    """Bytes of one GGUF row of K elements (gguf.js:36-49, 206-213)."""
    return {0: 4 * K, 1: 2 * K, 2: K // 32 * 18, 3: K // 32 * 20, 8: K // 32 * 34,
            14: K // 256 * 210}[ggml_type]


def dequant_q4_0(raw, n):
    out = np.empty(n, np.float32)
    lib().pbo_dequant_q4_0(_c(raw, np.uint8), n, out)
    return out


def dequant_q4_1(raw, n):
    out = np.empty(n, np.float32)
    lib().pbo_dequant_q4_1(_c(raw, np.uint8), n, out)
    return out


def dequant_f16(raw, n):
    out = np.empty(n, np.float32)
    lib().pbo_dequant_f16(_c(raw, np.uint8).view(np.uint8), n, out)
    return out


def dequant_q6_k(raw, n):
    out = np.empty(n, np.float32)
    lib().pbo_dequant_q6_k(_c(raw, np.uint8), n, out)
    return out


def dequant(ggml_type, raw, n):
    """loadTensorData (gguf.js:219-367) for the types this build handles."""
    if ggml_type == 0:
        return np.frombuffer(np.ascontiguousarray(raw).tobytes(), np.float32)[:n].copy()
    return {1: dequant_f16, 2: dequant_q4_0, 3: dequant_q4_1, 8: dequant_q8_0,
            14: dequant_q6_k}[ggml_type](raw, n)


def dequant_q8_0(raw, n):
    out = np.empty(n, np.float32)
    lib().pbo_dequant_q8_0(_c(raw, np.uint8), n, out)
    return out


def dequant_q8_ref(q, scales):
    q = _c(q, np.int8)
    out = np.empty(q.size, np.float32)
    lib().pbo_dequant_q8_ref(q, _c(scales, np.float32), q.size, out)
    return out


def _mv(fn, x, raw, N, K):
    out = np.empty(N, np.float32)
    fn(_c(x, np.float32), _c(raw, np.uint8), N, K, out)
    return out


def q4_0_matvec_js(x, raw, N, K):
    """llama-streaming.js:72-104 (double accumulation)."""
    return _mv(lib().pbo_q4_0_matvec_js, x, raw, N, K)


def q4_0_matvec_wasm(x, raw, N, K):
    """wasm-q4.js:118-267 replayed in f32, lane by lane."""
    return _mv(lib().pbo_q4_0_matvec_wasm, x, raw, N, K)


def q4_1_matvec_js(x, raw, N, K):
    """llama-streaming.js:115-151 (double accumulation)."""
    return _mv(lib().pbo_q4_1_matvec_js, x, raw, N, K)


def q4_1_matvec_wasm(x, raw, N, K):
    """wasm-q4.js:275-435 replayed in f32, lane by lane."""
    return _mv(lib().pbo_q4_1_matvec_wasm, x, raw, N, K)


def q4_0_matvec_cpu_sse(x, raw, N, K):
    """The SSE restatement used as the timed CPU baseline."""
    return _mv(lib().pbo_cpu_q4_0_matvec, x, raw, N, K)


def q8_0_matvec(x, raw, N, K):
    return _mv(lib().pbo_q8_0_matvec_f64, x, raw, N, K)


def f32_matvec(x, W):
    W = _c(W, np.float32)
    N, K = W.shape
    out = np.empty(N, np.float32)
    lib().pbo_f32_matvec_f64(_c(x, np.float32), W, N, K, out)
    return out


def batch_dot_wasm(x, W):
    W = _c(W, np.float32)
    N, K = W.shape
    out = np.empty(N, np.float32)
    lib().pbo_batch_dot_wasm(_c(x, np.float32), W, N, K, out)
    return out


def matvec(ggml_type, x, raw, N, K):
    """Oracle for one quantized matvec on GGUF bytes (type 2 = Q4_0,
    3 = Q4_1, 8 = Q8_0)."""
    if ggml_type == 2:
        return q4_0_matvec_js(x, raw, N, K)
    if ggml_type == 3:
        return q4_1_matvec_js(x, raw, N, K)
    if ggml_type == 8:
        return q8_0_matvec(x, raw, N, K)
    if ggml_type == 0:
        return f32_matvec(x, np.asarray(raw, np.float32).reshape(N, K))
    if ggml_type in (1, 14):
        # the reference dequantises F16 / Q6_K tensors to f32 (gguf.js:231-237,
        # 317-364) and runs the f32 matvec
        return f32_matvec(x, dequant(ggml_type, raw, N * K).reshape(N, K))
    raise ValueError(f"no oracle for type {ggml_type}")


def matmul_f32_axpy(A, B, bias=None):
    """wasm-simd.js matmul via matmulCached: C = bias + A[M,K] @ B[K,N], f32."""
    A = _c(A, np.float32)
    B = _c(B, np.float32)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    C = np.empty((M, N), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().pbo_matmul_f32_axpy(A, M, K, B, N, None if b is None else b.ctypes.data, C)
    return C


def matmul_q8_ref(A, q, scales, N, bias=None):
    """quantize.js:224-266 matmul_q8 on a QuantizedTensor [K,N]."""
    A = _c(A, np.float32)
    M, K = A.shape
    out = np.empty((M, N), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().pbo_matmul_q8_ref(A, M, K, _c(q, np.int8), _c(scales, np.float32), N,
                            None if b is None else b.ctypes.data, out)
    return out


def quantize_q8_ref(w):
    w = _c(w, np.float32).ravel()
    q = np.empty(w.size, np.int8)
    s = np.empty((w.size + 31) // 32, np.float32)
    lib().pbo_quantize_q8_ref(w, w.size, q, s)
    return q, s


def quantize_q8_0(w):
    w = _c(w, np.float32)
    N, K = w.shape
    out = np.empty(N * K // 32 * 34, np.uint8)
    lib().pbo_quantize_q8_0(w, N, K, out)
    return out


def quantize_q4_0(w):
    w = _c(w, np.float32)
    N, K = w.shape
    out = np.empty(N * K // 32 * 18, np.uint8)
    lib().pbo_quantize_q4_0(w, N, K, out)
    return out


def quantize_q6_k(w):
    w = _c(w, np.float32)
    N, K = w.shape
    out = np.empty(N * K // 256 * 210, np.uint8)
    lib().pbo_quantize_q6_k(w, N, K, out)
    return out


def quantize_q4_1(w):
    w = _c(w, np.float32)
    N, K = w.shape
    out = np.empty(N * K // 32 * 20, np.uint8)
    lib().pbo_quantize_q4_1(w, N, K, out)
    return out


def synth_normal(seed, n, mean=0.0, std=1.0):
    out = np.empty(n, np.float32)
    lib().pbo_synth_normal(seed, n, mean, std, out)
    return out


class CpuPool:
    """thread-pool.js restated: T threads (T-1 workers + the caller)."""

    def __init__(self, nthreads):
        self.nthreads = nthreads
        self._p = lib().pbo_pool_create(nthreads)

    def q4_0_matvec(self, x, raw, N, K, out=None):
        if out is None:
            out = np.empty(N, np.float32)
        lib().pbo_pool_q4_0_matvec(self._p, x, raw, N, K, out)
        return out

    def close(self):
        if self._p:
            lib().pbo_pool_destroy(self._p)
            self._p = None

    def __del__(self):
        self.close()


def cpu_lm_head(hidden, emb, vocab, dim, out=None):
    if out is None:
        out = np.empty(vocab, np.float32)
    lib().pbo_cpu_lm_head(_c(hidden, np.float32), emb, vocab, dim, out)
    return out


def argmax(v):
    """llama.js:432-442: first index of the maximum."""
    return lib().pbo_argmax(_c(v, np.float32), len(v))


class LlamaRef:
    """llama.js forward restated (llama_ref.c) on fp32 weights in GGUF
    orientation; tensor ids as the product's PBX_T_* constants."""

    def __init__(self, dim, hidden, n_layers, n_heads, n_kv, head_dim, vocab, max_seq,
                 theta=10000.0, eps=1e-5):
        self.cfg = _PboCfg(dim, hidden, n_layers, n_heads, n_kv, head_dim, vocab, max_seq,
                           theta, eps)
        self.vocab = vocab
        self._p = lib().pbo_llama_create(ctypes.byref(self.cfg))

    def set(self, tensor, layer, data):
        lib().pbo_llama_set(self._p, tensor, layer, _c(data, np.float32).ravel())

    def forward(self, tokens, start_pos, max_layers=0):
        """Logits of the last position; max_layers as StreamingLlamaRuntime's
        {maxLayers} (0: every layer)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.vocab, np.float32)
        lib().pbo_llama_forward_layers(self._p, toks, len(toks), start_pos, max_layers, out)
        return out

    def rollback(self, pos):
        lib().pbo_llama_rollback(self._p, pos)

    def close(self):
        if self._p:
            lib().pbo_llama_free(self._p)
            self._p = None

    def __del__(self):
        self.close()
