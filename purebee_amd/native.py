"""ctypes binding of the C ABI in include/pbx.h (lib/libpbhip.so).

Raises PbxError (with the library's own message) for every non-zero status;
there is no fallback path: without the built library nothing here works.
"""
import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG, "lib")

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q4_0 = 2
TYPE_Q4_1 = 3
TYPE_Q8_0 = 8
TYPE_Q6_K = 14
TYPE_Q8_REF = 100

STATUS = {0: "PBX_OK", -1: "PBX_EINVAL", -2: "PBX_ENODEV", -3: "PBX_ENOMEM",
          -4: "PBX_EHIP", -5: "PBX_ENOTSUP", -6: "PBX_ELOAD", -7: "PBX_EIO",
          -8: "PBX_ETIMEOUT"}
ETIMEOUT = -8
NOALLOC_WORKSPACE_BYTES = 64 << 20  # PBX_NOALLOC_WORKSPACE_BYTES

# Every entry point declared in include/pbx.h.
EXPORTS = (
    "pbx_init", "pbx_shutdown", "pbx_last_error", "pbx_device_info",
    "pbx_weight_upload", "pbx_weight_upload_q8ref", "pbx_weight_free", "pbx_weight_info",
    "pbx_linear", "pbx_linear_dev", "pbx_linear_dev_noalloc", "pbx_workspace_info",
    "pbx_ctx_stream", "pbx_dequant", "pbx_dequant_dev",
    "pbx_quantize_q8_0", "pbx_quantize_q4_0", "pbx_quantize_q4_1", "pbx_quantize_q6_k",
    "pbx_quantize_q8_ref",
    "pbx_synth_normal",
    "pbx_dev_alloc", "pbx_dev_free", "pbx_memcpy_h2d", "pbx_memcpy_d2h", "pbx_memset_dev",
    "pbx_dev_copy", "pbx_sync", "pbx_timer_start", "pbx_timer_stop", "pbx_bench_linear",
    "pbx_bench_linear_graph",
    "pbx_model_create", "pbx_model_free", "pbx_model_set_tensor", "pbx_model_forward",
    "pbx_model_forward_batch", "pbx_model_generate", "pbx_model_generate_eos", "pbx_model_reset_cache", "pbx_model_rollback", "pbx_model_info",
    "pbx_model_profile", "pbx_model_op_name", "pbx_model_bench_role", "pbx_model_test_handoff",
    "pbx_speculative_generate", "pbx_model_forward_layers", "pbx_self_speculative_generate",
    "pbx_gguf_open", "pbx_gguf_close", "pbx_gguf_info", "pbx_gguf_tensor_info",
    "pbx_gguf_find_tensor", "pbx_gguf_get_int", "pbx_gguf_get_float", "pbx_gguf_get_string",
    "pbx_gguf_get_array", "pbx_gguf_model_config", "pbx_model_load_gguf",
)

# Tensor ids of pbx_model_set_tensor (GGUF tensor names, gguf.js:378-410).
T_TOKEN_EMBD, T_OUTPUT, T_OUTPUT_NORM, T_ATTN_NORM, T_FFN_NORM = 0, 1, 2, 3, 4
T_ATTN_Q, T_ATTN_K, T_ATTN_V, T_ATTN_OUTPUT = 5, 6, 7, 8
T_FFN_GATE, T_FFN_UP, T_FFN_DOWN = 9, 10, 11


class ModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab_size",
        "max_seq", "weight_type", "embed_type", "output_type")] + \
        [("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_double)]


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("dims", ctypes.c_int64 * 4), ("offset", ctypes.c_uint64),
                ("nbytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]


class SpecStats(ctypes.Structure):
    _fields_ = [("rounds", ctypes.c_int32), ("drafted", ctypes.c_int32),
                ("accepted", ctypes.c_int32), ("prefill_ms", ctypes.c_double),
                ("decode_ms", ctypes.c_double)]


class PbxError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code


def library_path():
    return os.path.join(LIB_DIR, "libpbhip.so")


_lib = None
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")


def load_library():
    """Load lib/libpbhip.so; raises if it was not built (no silent fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not os.path.exists(path):
        raise PbxError(-6, f"{path} not built: run `python -m purebee_amd.build`")
    L = ctypes.CDLL(path)
    sig = {
        "pbx_init": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_vp)]),
        "pbx_shutdown": (None, [_vp]),
        "pbx_last_error": (ctypes.c_char_p, [_vp]),
        "pbx_device_info": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_size_t,
                                           ctypes.POINTER(ctypes.c_int)]),
        "pbx_weight_upload": (ctypes.c_int, [_vp, ctypes.c_int, _i64, _i64, _vp,
                                             ctypes.c_size_t, ctypes.POINTER(_vp)]),
        "pbx_weight_upload_q8ref": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _i64,
                                                   ctypes.POINTER(_vp)]),
        "pbx_weight_free": (ctypes.c_int, [_vp, _vp]),
        "pbx_weight_info": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int),
                                           ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                                           ctypes.POINTER(ctypes.c_size_t)]),
        "pbx_linear": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _vp]),
        "pbx_linear_dev": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _vp]),
        "pbx_linear_dev_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _vp]),
        "pbx_workspace_info": (ctypes.c_int, [_vp, _vp, _vp]),
        "pbx_ctx_stream": (_vp, [_vp]),
        "pbx_dequant": (ctypes.c_int, [_vp, _vp, _vp]),
        "pbx_dequant_dev": (ctypes.c_int, [_vp, _vp, _vp]),
        "pbx_quantize_q8_0": (ctypes.c_int, [_f32p, _i64, _i64, _u8p]),
        "pbx_quantize_q4_0": (ctypes.c_int, [_f32p, _i64, _i64, _u8p]),
        "pbx_quantize_q4_1": (ctypes.c_int, [_f32p, _i64, _i64, _u8p]),
        "pbx_quantize_q6_k": (ctypes.c_int, [_f32p, _i64, _i64, _u8p]),
        "pbx_quantize_q8_ref": (ctypes.c_int, [_f32p, _i64, _i8p, _f32p]),
        "pbx_synth_normal": (ctypes.c_int, [ctypes.c_uint64, _i64, ctypes.c_double,
                                            ctypes.c_double, _f32p]),
        "pbx_dev_alloc": (ctypes.c_int, [_vp, ctypes.c_size_t, ctypes.POINTER(_vp)]),
        "pbx_dev_free": (ctypes.c_int, [_vp, _vp]),
        "pbx_memcpy_h2d": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_size_t]),
        "pbx_memcpy_d2h": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_size_t]),
        "pbx_memset_dev": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_size_t]),
        "pbx_dev_copy": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_size_t]),
        "pbx_sync": (ctypes.c_int, [_vp]),
        "pbx_timer_start": (ctypes.c_int, [_vp]),
        "pbx_timer_stop": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_double)]),
        "pbx_bench_linear": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.POINTER(_vp),
                                            ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i64,
                                            ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
        "pbx_bench_linear_graph": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.POINTER(_vp),
                                            ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i64,
                                            ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
        "pbx_model_create": (ctypes.c_int, [_vp, ctypes.POINTER(ModelConfig), ctypes.POINTER(_vp)]),
        "pbx_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
        "pbx_gguf_close": (None, [_vp]),
        "pbx_gguf_info": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_i64),
                                         ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_uint64)]),
        "pbx_gguf_tensor_info": (ctypes.c_int, [_vp, _i64, ctypes.POINTER(GgufTensor)]),
        "pbx_gguf_find_tensor": (_i64, [_vp, ctypes.c_char_p]),
        "pbx_gguf_get_int": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_i64)]),
        "pbx_gguf_get_float": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
        "pbx_gguf_get_string": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                               ctypes.POINTER(ctypes.c_uint64)]),
        "pbx_gguf_get_array": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32),
                                              ctypes.POINTER(ctypes.c_uint64)]),
        "pbx_gguf_model_config": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.POINTER(ModelConfig)]),
        "pbx_model_load_gguf": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(_vp)]),
        "pbx_model_free": (ctypes.c_int, [_vp]),
        "pbx_model_set_tensor": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_size_t]),
        "pbx_model_forward": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, _vp, _vp]),
        "pbx_model_forward_batch": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, _vp, _vp]),
        "pbx_model_forward_layers": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int,
                                                    ctypes.c_int, _vp, _vp,
                                                    ctypes.POINTER(ctypes.c_int)]),
        "pbx_self_speculative_generate": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int,
                                                         ctypes.c_int, ctypes.c_int, _vp,
                                                         ctypes.c_int, ctypes.c_int, _vp,
                                                         ctypes.POINTER(ctypes.c_int),
                                                         ctypes.POINTER(SpecStats)]),
        "pbx_model_generate": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.c_int, ctypes.c_int, _vp, _vp]),
        "pbx_model_generate_eos": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.c_int, ctypes.c_int,
                                                  _vp, ctypes.c_int, _vp, _vp]),
        "pbx_model_reset_cache": (ctypes.c_int, [_vp]),
        "pbx_model_rollback": (ctypes.c_int, [_vp, ctypes.c_int]),
        "pbx_model_test_handoff": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
        "pbx_model_info": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_size_t),
                                          ctypes.POINTER(ctypes.c_int)]),
        "pbx_model_profile": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.c_int, ctypes.c_int,
                                             _vp, _vp, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
        "pbx_model_op_name": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]),
        "pbx_model_bench_role": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int,
                                                ctypes.POINTER(ctypes.c_double),
                                                ctypes.POINTER(ctypes.c_double),
                                                ctypes.POINTER(ctypes.c_int)]),
        "pbx_speculative_generate": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int,
                                                    ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int,
                                                    _vp, ctypes.POINTER(ctypes.c_int),
                                                    ctypes.POINTER(SpecStats)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _check(rc, ctx_ptr=None):
    if rc != 0:
        msg = load_library().pbx_last_error(ctx_ptr)
        raise PbxError(rc, msg.decode() if msg else "")


def block_bytes(t):
    """Bytes per 32 elements (Q6_K: per 256, see row_bytes)."""
    return {TYPE_Q4_0: 18, TYPE_Q4_1: 20, TYPE_Q8_0: 34, TYPE_F32: 128, TYPE_F16: 64}[t]


def row_bytes(t, K):
    """Bytes of one GGUF row of K elements."""
    return K // 256 * 210 if t == TYPE_Q6_K else K // 32 * block_bytes(t)


def quantize_q8_0(w):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    out = np.empty(N * (K // 32) * 34, np.uint8)
    _check(load_library().pbx_quantize_q8_0(w, N, K, out))
    return out


def quantize_q4_0(w):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    out = np.empty(N * (K // 32) * 18, np.uint8)
    _check(load_library().pbx_quantize_q4_0(w, N, K, out))
    return out


def quantize_q4_1(w):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    out = np.empty(N * (K // 32) * 20, np.uint8)
    _check(load_library().pbx_quantize_q4_1(w, N, K, out))
    return out


def quantize_q6_k(w):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    out = np.empty(N * (K // 256) * 210, np.uint8)
    _check(load_library().pbx_quantize_q6_k(w, N, K, out))
    return out


def to_f16_bytes(w):
    """GGUF F16 bytes of w (round to nearest even)."""
    return np.ascontiguousarray(w, np.float32).astype(np.float16).view(np.uint8).ravel()


def quantize_q8_ref(w):
    w = np.ascontiguousarray(w, np.float32).ravel()
    q = np.empty(w.size, np.int8)
    s = np.empty((w.size + 31) // 32, np.float32)
    _check(load_library().pbx_quantize_q8_ref(w, w.size, q, s))
    return q, s


def synth_normal(seed, n, mean=0.0, std=1.0):
    out = np.empty(n, np.float32)
    _check(load_library().pbx_synth_normal(seed, n, mean, std, out))
    return out


class DeviceBuffer:
    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = nbytes
        p = _vp()
        ctx._call("pbx_dev_alloc", ctx._p, nbytes, ctypes.byref(p))
        self.ptr = p.value

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        self.ctx._call("pbx_memcpy_h2d", self.ctx._p, self.ptr, arr.ctypes.data, arr.nbytes)
        return self

    def download(self, dtype, count):
        out = np.empty(count, dtype)
        assert out.nbytes <= self.nbytes
        self.ctx._call("pbx_memcpy_d2h", self.ctx._p, out.ctypes.data, self.ptr, out.nbytes)
        return out

    def free(self):
        if self.ptr:
            self.ctx._call("pbx_dev_free", self.ctx._p, self.ptr)
            self.ptr = None


class Weight:
    def __init__(self, ctx, ptr, type_, N, K):
        self.ctx, self.ptr, self.type, self.N, self.K = ctx, ptr, type_, N, K

    @property
    def device_bytes(self):
        t, n, k, b = ctypes.c_int(), _i64(), _i64(), ctypes.c_size_t()
        _check(load_library().pbx_weight_info(self.ptr, ctypes.byref(t), ctypes.byref(n),
                                              ctypes.byref(k), ctypes.byref(b)))
        return b.value

    def free(self):
        if self.ptr:
            self.ctx._call("pbx_weight_free", self.ctx._p, self.ptr)
            self.ptr = None


class Context:
    """One pbx_ctx: a device, its stream and the loaded code objects."""

    def __init__(self, device=0):
        L = load_library()
        p = _vp()
        _check(L.pbx_init(device, ctypes.byref(p)))
        self._p = p.value
        self.L = L

    def _call(self, name, *args):
        rc = getattr(self.L, name)(*args)
        if rc != 0:
            msg = self.L.pbx_last_error(self._p)
            raise PbxError(rc, msg.decode() if msg else "")

    def close(self):
        if self._p:
            self.L.pbx_shutdown(self._p)
            self._p = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def device_info(self):
        buf = ctypes.create_string_buffer(256)
        cu = ctypes.c_int()
        self._call("pbx_device_info", self._p, buf, 256, ctypes.byref(cu))
        return buf.value.decode(), cu.value

    def upload(self, type_, N, K, data):
        data = np.ascontiguousarray(data)
        w = _vp()
        self._call("pbx_weight_upload", self._p, type_, N, K, data.ctypes.data, data.nbytes,
                   ctypes.byref(w))
        return Weight(self, w.value, type_, N, K)

    def upload_q8ref(self, K, N, q, scales):
        q = np.ascontiguousarray(q, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        w = _vp()
        self._call("pbx_weight_upload_q8ref", self._p, K, N, q.ctypes.data, scales.ctypes.data,
                   scales.size, ctypes.byref(w))
        return Weight(self, w.value, TYPE_Q8_REF, N, K)

    def linear(self, w, X, bias=None):
        X = np.ascontiguousarray(X, np.float32)
        M = 1 if X.ndim == 1 else X.shape[0]
        assert X.size == M * w.K, (X.shape, w.K)
        Y = np.empty((M, w.N), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self._call("pbx_linear", self._p, w.ptr, X.ctypes.data, M,
                   None if b is None else b.ctypes.data, Y.ctypes.data)
        return Y[0] if X.ndim == 1 else Y

    def linear_dev(self, w, dX, M, dY, dBias=None):
        self._call("pbx_linear_dev", self._p, w.ptr, dX, M, dBias, dY)

    def linear_dev_noalloc(self, w, dX, M, dY, dBias=None):
        """pbx_linear_dev_noalloc: the same result, no device allocation."""
        self._call("pbx_linear_dev_noalloc", self._p, w.ptr, dX, M, dBias, dY)

    def workspace_info(self):
        """(bytes of workspace the allocating entry points grew, bytes of the
        static no-allocation workspace)."""
        g, st = ctypes.c_size_t(), ctypes.c_size_t()
        self._call("pbx_workspace_info", self._p, ctypes.byref(g), ctypes.byref(st))
        return g.value, st.value

    def stream(self):
        """The context's hipStream_t, as an integer handle."""
        return self.L.pbx_ctx_stream(self._p)

    def dequant(self, w):
        shape = (w.K, w.N) if w.type == TYPE_Q8_REF else (w.N, w.K)
        out = np.empty(shape, np.float32)
        self._call("pbx_dequant", self._p, w.ptr, out.ctypes.data)
        return out

    def alloc(self, nbytes):
        return DeviceBuffer(self, nbytes)

    def sync(self):
        self._call("pbx_sync", self._p)

    def dev_copy(self, dst, src, nbytes):
        self._call("pbx_dev_copy", self._p, dst, src, nbytes)

    def timer_start(self):
        self._call("pbx_timer_start", self._p)

    def timer_stop(self):
        ms = ctypes.c_double()
        self._call("pbx_timer_stop", self._p, ctypes.byref(ms))
        return ms.value

    def bench_linear(self, weights, dXs, dYs, M, reps, graph=False):
        """ms for `reps` passes over the linears, launched one by one or (graph)
        as one captured HIP graph replayed `reps` times."""
        n = len(weights)
        W = (_vp * n)(*[w.ptr for w in weights])
        X = (_vp * n)(*dXs)
        Y = (_vp * n)(*dYs)
        ms = ctypes.c_double()
        self._call("pbx_bench_linear_graph" if graph else "pbx_bench_linear", self._p, n, W, X, Y,
                   M, reps, ctypes.byref(ms))
        return ms.value


class GGUF:
    """A GGUF file opened with the build's reader (pbx_gguf_*; no GPU use)."""

    def __init__(self, path):
        self.L = load_library()
        self._g = None
        p = _vp()
        _check(self.L.pbx_gguf_open(os.fsencode(path), ctypes.byref(p)))
        self._g = p.value
        v, nt, nk, ds = ctypes.c_uint32(), _i64(), _i64(), ctypes.c_uint64()
        _check(self.L.pbx_gguf_info(self._g, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nk),
                                    ctypes.byref(ds)))
        self.version, self.n_tensors, self.n_kv, self.data_start = v.value, nt.value, nk.value, ds.value

    def tensor(self, i):
        t = GgufTensor()
        _check(self.L.pbx_gguf_tensor_info(self._g, i, ctypes.byref(t)))
        return {"name": t.name.decode(), "type": t.type, "dims": list(t.dims[:t.n_dims]),
                "offset": t.offset, "nbytes": t.nbytes, "data": t.data}

    def tensors(self):
        return [self.tensor(i) for i in range(self.n_tensors)]

    def tensor_bytes(self, i):
        t = self.tensor(i)
        return np.ctypeslib.as_array((ctypes.c_uint8 * t["nbytes"]).from_address(t["data"])).copy()

    def find(self, name):
        return self.L.pbx_gguf_find_tensor(self._g, name.encode())

    def get_int(self, key):
        v = _i64()
        _check(self.L.pbx_gguf_get_int(self._g, key.encode(), ctypes.byref(v)))
        return v.value

    def get_float(self, key):
        v = ctypes.c_double()
        _check(self.L.pbx_gguf_get_float(self._g, key.encode(), ctypes.byref(v)))
        return v.value

    def get_string(self, key):
        s, n = ctypes.c_void_p(), ctypes.c_uint64()
        _check(self.L.pbx_gguf_get_string(self._g, key.encode(), ctypes.byref(s), ctypes.byref(n)))
        return ctypes.string_at(s.value, n.value).decode() if n.value else ""

    def get_array(self, key):
        t, n = ctypes.c_uint32(), ctypes.c_uint64()
        _check(self.L.pbx_gguf_get_array(self._g, key.encode(), ctypes.byref(t), ctypes.byref(n)))
        return t.value, n.value

    def model_config(self, max_seq=0):
        cfg = ModelConfig()
        _check(self.L.pbx_gguf_model_config(self._g, max_seq, ctypes.byref(cfg)))
        return {f: getattr(cfg, f) for f, _ in ModelConfig._fields_}

    def close(self):
        if getattr(self, "_g", None):
            self.L.pbx_gguf_close(self._g)
            self._g = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()


class Model:
    """A resident Llama-family model with the on-GPU decode step (pbx_model_*)."""

    @classmethod
    def from_gguf(cls, ctx, path, max_seq=0):
        """pbx_model_load_gguf: configure from the file's metadata and upload
        every tensor once."""
        p = _vp()
        ctx._call("pbx_model_load_gguf", ctx._p, os.fsencode(path), max_seq, ctypes.byref(p))
        self = cls.__new__(cls)
        self.ctx = ctx
        self._m = p.value
        cfg = ModelConfig()
        self.cfg = cfg
        with GGUF(path) as g:
            c = g.model_config(max_seq)
        for f, _ in ModelConfig._fields_:
            setattr(cfg, f, c[f])
        self.vocab = cfg.vocab_size
        return self

    def __init__(self, ctx, dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, max_seq,
                 weight_type, embed_type, output_type=-1, head_dim=None, rms_eps=1e-5,
                 rope_theta=10000.0):
        self.ctx = ctx
        hd = head_dim or dim // n_heads
        self.cfg = ModelConfig(dim, hidden_dim, n_layers, n_heads, n_kv_heads, hd, vocab_size,
                               max_seq, weight_type, embed_type, output_type, rms_eps, rope_theta)
        p = _vp()
        ctx._call("pbx_model_create", ctx._p, ctypes.byref(self.cfg), ctypes.byref(p))
        self._m = p.value
        self.vocab = vocab_size

    def _mcall(self, name, *args):
        rc = getattr(self.ctx.L, name)(self._m, *args)
        if rc != 0:
            msg = self.ctx.L.pbx_last_error(self.ctx._p)
            raise PbxError(rc, msg.decode() if msg else "")

    def set_tensor(self, tensor, layer, data):
        data = np.ascontiguousarray(data)
        self._mcall("pbx_model_set_tensor", tensor, layer, data.ctypes.data, data.nbytes)

    def forward(self, tokens, start_pos, want_logits=True, max_layers=0):
        """(logits of the last position or None, their argmax); max_layers as
        StreamingLlamaRuntime.forward's {maxLayers} (0: every layer)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.vocab, np.float32) if want_logits else None
        nxt = ctypes.c_int32()
        used = ctypes.c_int()
        self._mcall("pbx_model_forward_layers", toks.ctypes.data, len(toks), start_pos,
                    int(max_layers), None if logits is None else logits.ctypes.data,
                    ctypes.byref(nxt), ctypes.byref(used))
        self.layers_used = used.value
        return logits, nxt.value

    def forward_batch(self, tokens, start_pos, want_logits=True):
        """One batched forward over all tokens: (logits [n, vocab] or None, argmax [n])."""
        toks = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty((len(toks), self.vocab), np.float32) if want_logits else None
        nxt = np.empty(len(toks), np.int32)
        self._mcall("pbx_model_forward_batch", toks.ctypes.data, len(toks), start_pos,
                    None if logits is None else logits.ctypes.data, nxt.ctypes.data)
        return logits, nxt

    def generate(self, token, start_pos, n_steps, want_logits=False):
        out = np.empty(n_steps, np.int32)
        logits = np.empty(self.vocab, np.float32) if want_logits else None
        self._mcall("pbx_model_generate", int(token), start_pos, n_steps, out.ctypes.data,
                    None if logits is None else logits.ctypes.data)
        return (out, logits) if want_logits else out

    def generate_until(self, token, start_pos, max_steps, eos_ids):
        """pbx_model_generate_eos: greedy steps stopping at the first token in
        eos_ids (returned last)."""
        eos = np.ascontiguousarray(eos_ids, np.int32)
        out = np.empty(max_steps, np.int32)
        n = ctypes.c_int()
        self._mcall("pbx_model_generate_eos", int(token), start_pos, max_steps,
                    eos.ctypes.data if len(eos) else None, len(eos), out.ctypes.data,
                    ctypes.byref(n))
        return out[:n.value]

    def reset_cache(self):
        self._mcall("pbx_model_reset_cache")

    def rollback(self, pos):
        self._mcall("pbx_model_rollback", pos)

    def test_handoff(self, layer, skew, spin=0):
        """Test hook: the joined q|k|v + attention launch of `layer` waits
        for cells that never arrive (tag offset `skew`), giving up after
        `spin` polls; layer < 0 restores the normal launch."""
        self._mcall("pbx_model_test_handoff", layer, skew, spin)

    def info(self):
        b, g = ctypes.c_size_t(), ctypes.c_int()
        self._mcall("pbx_model_info", ctypes.byref(b), ctypes.byref(g))
        return {"device_bytes": b.value, "graph": bool(g.value)}

    def profile(self, token, start_pos, n_steps):
        """[(role, kernel, mean us, mean algorithmic bytes)] per kernel of a step."""
        cap = 4096
        us = np.zeros(cap, np.float64)
        by = np.zeros(cap, np.float64)
        n = ctypes.c_int()
        self._mcall("pbx_model_profile", int(token), start_pos, n_steps, us.ctypes.data,
                    by.ctypes.data, cap, ctypes.byref(n))
        out = []
        buf = ctypes.create_string_buffer(256)
        for i in range(min(n.value, cap)):
            self._mcall("pbx_model_op_name", i, buf, 256)
            role, kern = buf.value.decode().split(":", 1)
            out.append((role, kern, float(us[i]), float(by[i])))
        return out

    def bench_role(self, role, reps):
        """(us per launch, algorithmic bytes per launch, launches per pass)."""
        us, by, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int()
        self._mcall("pbx_model_bench_role", role.encode(), reps, ctypes.byref(us),
                    ctypes.byref(by), ctypes.byref(n))
        return us.value, by.value, n.value

    def free(self):
        if self._m:
            self._mcall("pbx_model_free")
            self._m = None


def speculative_generate(target, draft, prompt, max_tokens, draft_count=4, eos_ids=(2,),
                         batched_verify=True):
    """Greedy speculative decoding (speculative.js:58-204) with `draft` proposing
    and `target` verifying.  Returns (generated tokens, stats dict)."""
    ctx = target.ctx
    p = np.ascontiguousarray(prompt, np.int32)
    eos = np.ascontiguousarray(list(eos_ids), np.int32)
    out = np.empty(max_tokens + 1, np.int32)
    n = ctypes.c_int()
    st = SpecStats()
    rc = ctx.L.pbx_speculative_generate(target._m, draft._m, p.ctypes.data, len(p), max_tokens,
                                        draft_count, eos.ctypes.data if len(eos) else None,
                                        len(eos), 1 if batched_verify else 0, out.ctypes.data,
                                        ctypes.byref(n), ctypes.byref(st))
    if rc != 0:
        msg = ctx.L.pbx_last_error(ctx._p)
        raise PbxError(rc, msg.decode() if msg else "")
    stats = {k: getattr(st, k) for k, _ in SpecStats._fields_}
    return out[:n.value].copy(), stats


def self_speculative_generate(model, prompt, max_tokens, draft_layers=4, draft_count=4,
                              eos_ids=(2,), batched_verify=True):
    """SelfSpeculativeDecoder.generate (speculative.js:58-204), greedy, drafting
    with the model's own first draft_layers layers.  Returns (generated
    tokens, stats dict)."""
    ctx = model.ctx
    p = np.ascontiguousarray(prompt, np.int32)
    eos = np.ascontiguousarray(list(eos_ids), np.int32)
    out = np.empty(max_tokens + 1, np.int32)
    n = ctypes.c_int()
    st = SpecStats()
    rc = ctx.L.pbx_self_speculative_generate(model._m, p.ctypes.data, len(p), max_tokens,
                                             draft_layers, draft_count,
                                             eos.ctypes.data if len(eos) else None, len(eos),
                                             1 if batched_verify else 0, out.ctypes.data,
                                             ctypes.byref(n), ctypes.byref(st))
    if rc != 0:
        msg = ctx.L.pbx_last_error(ctx._p)
        raise PbxError(rc, msg.decode() if msg else "")
    stats = {k: getattr(st, k) for k, _ in SpecStats._fields_}
    return out[:n.value].copy(), stats
