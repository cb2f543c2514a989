// pbx_napi.cc -- N-API addon exposing the C ABI (include/pbx.h) to Node.js.
//
// Thin on purpose: typed-array backing stores are handed to the C ABI
// directly (no copies on the JS side), every non-zero status becomes a thrown
// Error carrying pbx_last_error(), and results come back as fresh
// Float32Arrays, the synchronous convention of wasm-q4.js:744-746.
// N-API is ABI-stable, so the same binary loads in any Node >= 10.
#include <node_api.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "pbx.h"

namespace {

pbx_ctx *g_ctx = nullptr;

struct WeightRef {
  pbx_weight *w;
  int type;
  int64_t N, K;
};

napi_value throw_pbx(napi_env env, int rc, const char *who) {
  char msg[1200];
  snprintf(msg, sizeof msg, "%s: %s (status %d)", who, pbx_last_error(g_ctx), rc);
  napi_throw_error(env, nullptr, msg);
  return nullptr;
}

napi_value throw_msg(napi_env env, const char *msg) {
  napi_throw_error(env, nullptr, msg);
  return nullptr;
}

bool get_args(napi_env env, napi_callback_info info, size_t want, napi_value *argv,
              size_t *got = nullptr) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok) return false;
  for (size_t i = argc; i < want; ++i) napi_get_undefined(env, &argv[i]);
  if (got) *got = argc;
  return true;
}

bool is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  return t == napi_undefined || t == napi_null;
}

bool get_i64(napi_env env, napi_value v, int64_t *out) {
  return napi_get_value_int64(env, v, out) == napi_ok;
}

// Any typed array (or Buffer): returns data pointer and byte length.
bool typed_bytes(napi_env env, napi_value v, void **data, size_t *bytes,
                 napi_typedarray_type *ty = nullptr) {
  bool is = false;
  napi_is_typedarray(env, v, &is);
  if (!is) return false;
  napi_typedarray_type t;
  size_t len = 0, off = 0;
  napi_value ab;
  if (napi_get_typedarray_info(env, v, &t, &len, data, &ab, &off) != napi_ok) return false;
  size_t el = 1;
  switch (t) {
    case napi_int16_array: case napi_uint16_array: el = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
    case napi_float64_array: el = 8; break;
    default: el = 1;
  }
  *bytes = len * el;
  if (ty) *ty = t;
  return true;
}

bool get_f32(napi_env env, napi_value v, float **data, size_t *count) {
  void *p;
  size_t b;
  napi_typedarray_type t;
  if (!typed_bytes(env, v, &p, &b, &t) || t != napi_float32_array) return false;
  *data = (float *)p;
  *count = b / 4;
  return true;
}

napi_value new_f32(napi_env env, size_t count, float **data) {
  napi_value ab, arr;
  void *p = nullptr;
  if (napi_create_arraybuffer(env, count * 4, &p, &ab) != napi_ok) return nullptr;
  if (napi_create_typedarray(env, napi_float32_array, count, ab, 0, &arr) != napi_ok) return nullptr;
  *data = (float *)p;
  return arr;
}

void finalize_weight(napi_env env, void *data, void *hint) {
  WeightRef *r = (WeightRef *)data;
  if (r->w && g_ctx) pbx_weight_free(g_ctx, r->w);
  delete r;
}

WeightRef *get_weight(napi_env env, napi_value v) {
  void *p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) return nullptr;
  return (WeightRef *)p;
}

bool need_ctx(napi_env env) {
  if (g_ctx) return true;
  throw_msg(env, "purebee_amd: call init() first");
  return false;
}

// init(device = 0) -> true
napi_value Init(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  int64_t dev = 0;
  if (!is_nullish(env, argv[0]) && !get_i64(env, argv[0], &dev))
    return throw_msg(env, "init: device must be a number");
  if (!g_ctx) {
    int rc = pbx_init((int)dev, &g_ctx);
    if (rc) {
      g_ctx = nullptr;
      return throw_pbx(env, rc, "init");
    }
  }
  napi_value t;
  napi_get_boolean(env, true, &t);
  return t;
}

napi_value DeviceInfo(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  char name[256];
  int cus = 0;
  int rc = pbx_device_info(g_ctx, name, sizeof name, &cus);
  if (rc) return throw_pbx(env, rc, "deviceInfo");
  napi_value o, n, c;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &n);
  napi_create_int32(env, cus, &c);
  napi_set_named_property(env, o, "name", n);
  napi_set_named_property(env, o, "computeUnits", c);
  return o;
}

napi_value make_handle(napi_env env, pbx_weight *w, int type, int64_t N, int64_t K) {
  WeightRef *r = new WeightRef{w, type, N, K};
  napi_value h;
  if (napi_create_external(env, r, finalize_weight, nullptr, &h) != napi_ok) {
    pbx_weight_free(g_ctx, w);
    delete r;
    return throw_msg(env, "upload: could not create handle");
  }
  return h;
}

// upload(type, N, K, bytes: TypedArray) -> handle
napi_value Upload(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[4];
  get_args(env, info, 4, argv);
  int64_t type, N, K;
  if (!get_i64(env, argv[0], &type) || !get_i64(env, argv[1], &N) || !get_i64(env, argv[2], &K))
    return throw_msg(env, "upload(type, N, K, data): type, N and K must be numbers");
  void *data;
  size_t bytes;
  if (!typed_bytes(env, argv[3], &data, &bytes))
    return throw_msg(env, "upload(type, N, K, data): data must be a TypedArray or Buffer");
  pbx_weight *w = nullptr;
  int rc = pbx_weight_upload(g_ctx, (int)type, N, K, data, bytes, &w);
  if (rc) return throw_pbx(env, rc, "upload");
  return make_handle(env, w, (int)type, N, K);
}

// uploadQ8Ref(K, N, q: Int8Array, scales: Float32Array) -> handle
napi_value UploadQ8Ref(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[4];
  get_args(env, info, 4, argv);
  int64_t K, N;
  if (!get_i64(env, argv[0], &K) || !get_i64(env, argv[1], &N))
    return throw_msg(env, "uploadQ8Ref(K, N, q, scales): K and N must be numbers");
  void *q;
  size_t qb;
  float *s;
  size_t ns;
  if (!typed_bytes(env, argv[2], &q, &qb) || !get_f32(env, argv[3], &s, &ns))
    return throw_msg(env, "uploadQ8Ref: q must be an Int8Array and scales a Float32Array");
  if ((int64_t)qb < K * N) return throw_msg(env, "uploadQ8Ref: q shorter than K*N");
  pbx_weight *w = nullptr;
  int rc = pbx_weight_upload_q8ref(g_ctx, K, N, (const int8_t *)q, s, (int64_t)ns, &w);
  if (rc) return throw_pbx(env, rc, "uploadQ8Ref");
  return make_handle(env, w, PBX_TYPE_Q8_REF, N, K);
}

napi_value Free(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[1];
  get_args(env, info, 1, argv);
  WeightRef *r = get_weight(env, argv[0]);
  if (!r) return throw_msg(env, "free: not a weight handle");
  if (r->w) {
    int rc = pbx_weight_free(g_ctx, r->w);
    r->w = nullptr;
    if (rc) return throw_pbx(env, rc, "free");
  }
  return nullptr;
}

// linear(handle, x: Float32Array [M*K], M = 1, bias: Float32Array|null) -> Float32Array [M*N]
napi_value Linear(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[4];
  get_args(env, info, 4, argv);
  WeightRef *r = get_weight(env, argv[0]);
  if (!r || !r->w) return throw_msg(env, "linear: not a live weight handle");
  float *x;
  size_t nx;
  if (!get_f32(env, argv[1], &x, &nx)) return throw_msg(env, "linear: x must be a Float32Array");
  int64_t M = 1;
  if (!is_nullish(env, argv[2]) && !get_i64(env, argv[2], &M))
    return throw_msg(env, "linear: M must be a number");
  if (M <= 0 || (int64_t)nx < M * r->K) {
    char msg[200];
    snprintf(msg, sizeof msg, "linear: x holds %zu values, M=%lld x K=%lld needed", nx,
             (long long)M, (long long)r->K);
    return throw_msg(env, msg);
  }
  float *bias = nullptr;
  size_t nb = 0;
  if (!is_nullish(env, argv[3])) {
    if (!get_f32(env, argv[3], &bias, &nb) || (int64_t)nb < r->N)
      return throw_msg(env, "linear: bias must be a Float32Array of length N");
  }
  float *y;
  napi_value out = new_f32(env, (size_t)(M * r->N), &y);
  if (!out) return throw_msg(env, "linear: out of memory");
  int rc = pbx_linear(g_ctx, r->w, x, M, bias, y);
  if (rc) return throw_pbx(env, rc, "linear");
  return out;
}

napi_value Dequant(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[1];
  get_args(env, info, 1, argv);
  WeightRef *r = get_weight(env, argv[0]);
  if (!r || !r->w) return throw_msg(env, "dequant: not a live weight handle");
  float *y;
  napi_value out = new_f32(env, (size_t)(r->N * r->K), &y);
  if (!out) return throw_msg(env, "dequant: out of memory");
  int rc = pbx_dequant(g_ctx, r->w, y);
  if (rc) return throw_pbx(env, rc, "dequant");
  return out;
}

napi_value Info(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  get_args(env, info, 1, argv);
  WeightRef *r = get_weight(env, argv[0]);
  if (!r) return throw_msg(env, "info: not a weight handle");
  napi_value o, v;
  napi_create_object(env, &o);
  napi_create_int32(env, r->type, &v);
  napi_set_named_property(env, o, "type", v);
  napi_create_int64(env, r->N, &v);
  napi_set_named_property(env, o, "N", v);
  napi_create_int64(env, r->K, &v);
  napi_set_named_property(env, o, "K", v);
  napi_get_boolean(env, r->w != nullptr, &v);
  napi_set_named_property(env, o, "live", v);
  return o;
}

// ---- resident model (pbx_model_*) ----------------------------------------

struct ModelRef {
  pbx_model *m;
  int vocab, max_seq;
};

void finalize_model(napi_env env, void *data, void *hint) {
  ModelRef *r = (ModelRef *)data;
  if (r->m && g_ctx) pbx_model_free(r->m);
  delete r;
}

ModelRef *get_model(napi_env env, napi_value v) {
  void *p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) return nullptr;
  ModelRef *r = (ModelRef *)p;
  return r->m ? r : nullptr;
}

bool prop_num(napi_env env, napi_value o, const char *k, double *out, bool required) {
  bool has = false;
  napi_has_named_property(env, o, k, &has);
  if (!has) return !required;
  napi_value v;
  napi_get_named_property(env, o, k, &v);
  return napi_get_value_double(env, v, out) == napi_ok;
}

// Int32Array, or an Array of numbers, copied into `out`.
bool get_tokens(napi_env env, napi_value v, std::vector<int32_t> *out) {
  void *p;
  size_t b;
  napi_typedarray_type t;
  if (typed_bytes(env, v, &p, &b, &t)) {
    if (t != napi_int32_array) return false;
    out->assign((int32_t *)p, (int32_t *)p + b / 4);
    return true;
  }
  bool arr = false;
  napi_is_array(env, v, &arr);
  if (!arr) return false;
  uint32_t n = 0;
  napi_get_array_length(env, v, &n);
  out->resize(n);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    int32_t x;
    napi_get_element(env, v, i, &e);
    if (napi_get_value_int32(env, e, &x) != napi_ok) return false;
    (*out)[i] = x;
  }
  return true;
}

napi_value new_i32(napi_env env, size_t count, int32_t **data) {
  napi_value ab, arr;
  void *p = nullptr;
  if (napi_create_arraybuffer(env, count * 4, &p, &ab) != napi_ok) return nullptr;
  if (napi_create_typedarray(env, napi_int32_array, count, ab, 0, &arr) != napi_ok) return nullptr;
  *data = (int32_t *)p;
  return arr;
}

// modelCreate({dim, hiddenDim, nLayers, nHeads, nKvHeads, headDim?, vocabSize, maxSeq,
//              weightType, embedType, outputType = -1, rmsEps = 1e-5, ropeTheta = 10000})
napi_value ModelCreate(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[1];
  get_args(env, info, 1, argv);
  double dim, hid, nl, nh, nkv, voc, ms, wt, et, hd = 0, ot = -1, eps = 1e-5, theta = 10000;
  napi_value o = argv[0];
  if (!prop_num(env, o, "dim", &dim, true) || !prop_num(env, o, "hiddenDim", &hid, true) ||
      !prop_num(env, o, "nLayers", &nl, true) || !prop_num(env, o, "nHeads", &nh, true) ||
      !prop_num(env, o, "nKvHeads", &nkv, true) || !prop_num(env, o, "vocabSize", &voc, true) ||
      !prop_num(env, o, "maxSeq", &ms, true) || !prop_num(env, o, "weightType", &wt, true) ||
      !prop_num(env, o, "embedType", &et, true) || !prop_num(env, o, "headDim", &hd, false) ||
      !prop_num(env, o, "outputType", &ot, false) || !prop_num(env, o, "rmsEps", &eps, false) ||
      !prop_num(env, o, "ropeTheta", &theta, false))
    return throw_msg(env, "modelCreate: config needs dim, hiddenDim, nLayers, nHeads, nKvHeads, "
                          "vocabSize, maxSeq, weightType, embedType (numbers)");
  pbx_model_config c;
  c.dim = (int32_t)dim;
  c.hidden_dim = (int32_t)hid;
  c.n_layers = (int32_t)nl;
  c.n_heads = (int32_t)nh;
  c.n_kv_heads = (int32_t)nkv;
  c.head_dim = hd > 0 ? (int32_t)hd : (nh > 0 ? (int32_t)(dim / nh) : 0);
  c.vocab_size = (int32_t)voc;
  c.max_seq = (int32_t)ms;
  c.weight_type = (int32_t)wt;
  c.embed_type = (int32_t)et;
  c.output_type = (int32_t)ot;
  c.rms_eps = (float)eps;
  c.rope_theta = theta;
  pbx_model *m = nullptr;
  int rc = pbx_model_create(g_ctx, &c, &m);
  if (rc) return throw_pbx(env, rc, "modelCreate");
  ModelRef *r = new ModelRef{m, c.vocab_size, c.max_seq};
  napi_value h;
  if (napi_create_external(env, r, finalize_model, nullptr, &h) != napi_ok) {
    pbx_model_free(m);
    delete r;
    return throw_msg(env, "modelCreate: could not create handle");
  }
  return h;
}

// modelLoadGGUF(path: string, maxSeq = 0) -> {model, config}: the GGUF file
// through pbx_model_load_gguf; config in extractConfig's field names
// (gguf.js:429-450) plus the tensor types.
napi_value ModelLoadGGUF(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[2];
  size_t argc = 0;
  get_args(env, info, 2, argv, &argc);
  char path[4096];
  size_t len = 0;
  if (argc < 1 ||
      napi_get_value_string_utf8(env, argv[0], path, sizeof path, &len) != napi_ok ||
      len + 1 >= sizeof path)
    return throw_msg(env, "modelLoadGGUF(path, maxSeq): path must be a string");
  int64_t max_seq = 0;
  if (argc >= 2 && !get_i64(env, argv[1], &max_seq))
    return throw_msg(env, "modelLoadGGUF(path, maxSeq): maxSeq must be a number");
  pbx_gguf *g = nullptr;
  pbx_model_config c;
  int rc = pbx_gguf_open(path, &g);
  if (!rc) rc = pbx_gguf_model_config(g, (int)max_seq, &c);
  if (g) pbx_gguf_close(g);
  if (rc) {  // the reader reports without a context
    char msg[1200];
    snprintf(msg, sizeof msg, "modelLoadGGUF: %s (status %d)", pbx_last_error(nullptr), rc);
    return throw_msg(env, msg);
  }
  pbx_model *m = nullptr;
  rc = pbx_model_load_gguf(g_ctx, path, (int)max_seq, &m);
  if (rc) return throw_pbx(env, rc, "modelLoadGGUF");
  ModelRef *r = new ModelRef{m, c.vocab_size, c.max_seq};
  napi_value h, out, cfg;
  if (napi_create_external(env, r, finalize_model, nullptr, &h) != napi_ok) {
    pbx_model_free(m);
    delete r;
    return throw_msg(env, "modelLoadGGUF: could not create handle");
  }
  napi_create_object(env, &out);
  napi_create_object(env, &cfg);
  const struct { const char *k; double v; } fields[] = {
      {"dim", (double)c.dim}, {"hiddenDim", (double)c.hidden_dim}, {"nLayers", (double)c.n_layers},
      {"nHeads", (double)c.n_heads}, {"nKvHeads", (double)c.n_kv_heads},
      {"headDim", (double)c.head_dim}, {"vocabSize", (double)c.vocab_size},
      {"seqLen", (double)c.max_seq}, {"rmsNormEps", (double)c.rms_eps},
      {"ropeTheta", c.rope_theta}, {"weightType", (double)c.weight_type},
      {"embedType", (double)c.embed_type}, {"outputType", (double)c.output_type}};
  for (const auto &f : fields) {
    napi_value v;
    napi_create_double(env, f.v, &v);
    napi_set_named_property(env, cfg, f.k, v);
  }
  napi_set_named_property(env, out, "model", h);
  napi_set_named_property(env, out, "config", cfg);
  return out;
}

// modelSetTensor(model, tensorId, layer, data: TypedArray)
napi_value ModelSetTensor(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[4];
  get_args(env, info, 4, argv);
  ModelRef *r = get_model(env, argv[0]);
  int64_t tid, layer;
  void *data;
  size_t bytes;
  if (!r || !get_i64(env, argv[1], &tid) || !get_i64(env, argv[2], &layer) ||
      !typed_bytes(env, argv[3], &data, &bytes))
    return throw_msg(env, "modelSetTensor(model, tensorId, layer, data): bad arguments");
  int rc = pbx_model_set_tensor(r->m, (int)tid, (int)layer, data, bytes);
  if (rc) return throw_pbx(env, rc, "modelSetTensor");
  return nullptr;
}

// modelForward(model, tokens, startPos, maxLayers = 0)
//   -> {logits: Float32Array [vocab], next, layersUsed}
napi_value ModelForward(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[4];
  get_args(env, info, 4, argv);
  ModelRef *r = get_model(env, argv[0]);
  std::vector<int32_t> toks;
  int64_t start, max_layers = 0;
  if (!r || !get_tokens(env, argv[1], &toks) || !get_i64(env, argv[2], &start) ||
      (!is_nullish(env, argv[3]) && !get_i64(env, argv[3], &max_layers)))
    return throw_msg(env, "modelForward(model, tokens, startPos, maxLayers): bad arguments");
  float *lg;
  napi_value logits = new_f32(env, (size_t)r->vocab, &lg);
  if (!logits) return throw_msg(env, "modelForward: out of memory");
  int32_t next = 0;
  int used = 0;
  int rc = pbx_model_forward_layers(r->m, toks.data(), (int)toks.size(), (int)start,
                                    (int)max_layers, lg, &next, &used);
  if (rc) return throw_pbx(env, rc, "modelForward");
  napi_value o, nv;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "logits", logits);
  napi_create_int32(env, next, &nv);
  napi_set_named_property(env, o, "next", nv);
  napi_create_int32(env, used, &nv);
  napi_set_named_property(env, o, "layersUsed", nv);
  return o;
}

// modelForwardBatch(model, tokens, startPos) -> {logits: Float32Array [n*vocab], next: Int32Array}
napi_value ModelForwardBatch(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[3];
  get_args(env, info, 3, argv);
  ModelRef *r = get_model(env, argv[0]);
  std::vector<int32_t> toks;
  int64_t start;
  if (!r || !get_tokens(env, argv[1], &toks) || !get_i64(env, argv[2], &start) || toks.empty())
    return throw_msg(env, "modelForwardBatch(model, tokens, startPos): bad arguments");
  float *lg;
  int32_t *nx;
  napi_value logits = new_f32(env, toks.size() * (size_t)r->vocab, &lg);
  napi_value next = new_i32(env, toks.size(), &nx);
  if (!logits || !next) return throw_msg(env, "modelForwardBatch: out of memory");
  int rc = pbx_model_forward_batch(r->m, toks.data(), (int)toks.size(), (int)start, lg, nx);
  if (rc) return throw_pbx(env, rc, "modelForwardBatch");
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "logits", logits);
  napi_set_named_property(env, o, "next", next);
  return o;
}

// modelGenerate(model, token, startPos, nSteps[, eosId]) -> Int32Array:
// nSteps tokens, or with eosId the tokens up to and including the first EOS
napi_value ModelGenerate(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[5];
  get_args(env, info, 5, argv);
  ModelRef *r = get_model(env, argv[0]);
  int64_t tok, start, n, eos = -1;
  if (!r || !get_i64(env, argv[1], &tok) || !get_i64(env, argv[2], &start) ||
      !get_i64(env, argv[3], &n) || n <= 0 || n > r->max_seq ||
      (!is_nullish(env, argv[4]) && !get_i64(env, argv[4], &eos)))
    return throw_msg(env, "modelGenerate(model, token, startPos, nSteps[, eosId]): bad arguments");
  if (eos < 0) {
    int32_t *out;
    napi_value arr = new_i32(env, (size_t)n, &out);
    if (!arr) return throw_msg(env, "modelGenerate: out of memory");
    int rc = pbx_model_generate(r->m, (int32_t)tok, (int)start, (int)n, out, nullptr);
    if (rc) return throw_pbx(env, rc, "modelGenerate");
    return arr;
  }
  std::vector<int32_t> buf((size_t)n);
  const int32_t e = (int32_t)eos;
  int got = 0;
  int rc = pbx_model_generate_eos(r->m, (int32_t)tok, (int)start, (int)n, &e, 1, buf.data(), &got);
  if (rc) return throw_pbx(env, rc, "modelGenerate");
  int32_t *out;
  napi_value arr = new_i32(env, (size_t)got, &out);
  if (!arr) return throw_msg(env, "modelGenerate: out of memory");
  for (int i = 0; i < got; ++i) out[i] = buf[i];
  return arr;
}

// modelRollback(model, pos) / modelReset(model) / modelFree(model)
napi_value ModelRollback(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[2];
  get_args(env, info, 2, argv);
  ModelRef *r = get_model(env, argv[0]);
  int64_t pos;
  if (!r || !get_i64(env, argv[1], &pos)) return throw_msg(env, "modelRollback(model, pos): bad arguments");
  int rc = pbx_model_rollback(r->m, (int)pos);
  if (rc) return throw_pbx(env, rc, "modelRollback");
  return nullptr;
}

napi_value ModelReset(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[1];
  get_args(env, info, 1, argv);
  ModelRef *r = get_model(env, argv[0]);
  if (!r) return throw_msg(env, "modelReset(model): not a live model");
  int rc = pbx_model_reset_cache(r->m);
  if (rc) return throw_pbx(env, rc, "modelReset");
  return nullptr;
}

napi_value ModelFree(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[1];
  get_args(env, info, 1, argv);
  void *p = nullptr;
  if (napi_get_value_external(env, argv[0], &p) != napi_ok || !p)
    return throw_msg(env, "modelFree(model): not a model handle");
  ModelRef *r = (ModelRef *)p;
  if (r->m) {
    int rc = pbx_model_free(r->m);
    r->m = nullptr;
    if (rc) return throw_pbx(env, rc, "modelFree");
  }
  return nullptr;
}

// speculative(target, draft, prompt, maxTokens, draftCount = 4, eosIds = [2], batched = true)
//   -> {tokens: Int32Array, rounds, drafted, accepted, prefillMs, decodeMs}
napi_value Speculative(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[7];
  get_args(env, info, 7, argv);
  ModelRef *t = get_model(env, argv[0]), *d = get_model(env, argv[1]);
  std::vector<int32_t> prompt, eos = {2};
  int64_t maxTok, dc = 4;
  if (!t || !d || !get_tokens(env, argv[2], &prompt) || !get_i64(env, argv[3], &maxTok) ||
      maxTok <= 0 || (!is_nullish(env, argv[4]) && !get_i64(env, argv[4], &dc)) ||
      (!is_nullish(env, argv[5]) && !get_tokens(env, argv[5], &eos)))
    return throw_msg(env, "speculative(target, draft, prompt, maxTokens, draftCount, eosIds, "
                          "batched): bad arguments");
  bool batched = true;
  if (!is_nullish(env, argv[6])) napi_get_value_bool(env, argv[6], &batched);
  std::vector<int32_t> out((size_t)maxTok + 1);
  int n = 0;
  pbx_spec_stats st;
  int rc = pbx_speculative_generate(t->m, d->m, prompt.data(), (int)prompt.size(), (int)maxTok,
                                    (int)dc, eos.empty() ? nullptr : eos.data(), (int)eos.size(),
                                    batched ? 1 : 0, out.data(), &n, &st);
  if (rc) return throw_pbx(env, rc, "speculative");
  int32_t *tk;
  napi_value toks = new_i32(env, (size_t)n, &tk);
  if (!toks) return throw_msg(env, "speculative: out of memory");
  memcpy(tk, out.data(), (size_t)n * 4);
  napi_value o, v;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "tokens", toks);
  napi_create_int32(env, st.rounds, &v);
  napi_set_named_property(env, o, "rounds", v);
  napi_create_int32(env, st.drafted, &v);
  napi_set_named_property(env, o, "drafted", v);
  napi_create_int32(env, st.accepted, &v);
  napi_set_named_property(env, o, "accepted", v);
  napi_create_double(env, st.prefill_ms, &v);
  napi_set_named_property(env, o, "prefillMs", v);
  napi_create_double(env, st.decode_ms, &v);
  napi_set_named_property(env, o, "decodeMs", v);
  return o;
}

// selfSpeculative(model, prompt, maxTokens, draftLayers = 4, draftCount = 4, eosIds = [2],
//                 batched = true)
//   -> {tokens: Int32Array, rounds, drafted, accepted, prefillMs, decodeMs}
napi_value SelfSpeculative(napi_env env, napi_callback_info info) {
  if (!need_ctx(env)) return nullptr;
  napi_value argv[7];
  get_args(env, info, 7, argv);
  ModelRef *r = get_model(env, argv[0]);
  std::vector<int32_t> prompt, eos = {2};
  int64_t maxTok, dl = 4, dc = 4;
  if (!r || !get_tokens(env, argv[1], &prompt) || !get_i64(env, argv[2], &maxTok) ||
      maxTok <= 0 || (!is_nullish(env, argv[3]) && !get_i64(env, argv[3], &dl)) ||
      (!is_nullish(env, argv[4]) && !get_i64(env, argv[4], &dc)) ||
      (!is_nullish(env, argv[5]) && !get_tokens(env, argv[5], &eos)))
    return throw_msg(env, "selfSpeculative(model, prompt, maxTokens, draftLayers, draftCount, "
                          "eosIds, batched): bad arguments");
  bool batched = true;
  if (!is_nullish(env, argv[6])) napi_get_value_bool(env, argv[6], &batched);
  std::vector<int32_t> out((size_t)maxTok + 1);
  int n = 0;
  pbx_spec_stats st;
  int rc = pbx_self_speculative_generate(r->m, prompt.data(), (int)prompt.size(), (int)maxTok,
                                         (int)dl, (int)dc, eos.empty() ? nullptr : eos.data(),
                                         (int)eos.size(), batched ? 1 : 0, out.data(), &n, &st);
  if (rc) return throw_pbx(env, rc, "selfSpeculative");
  int32_t *tk;
  napi_value toks = new_i32(env, (size_t)n, &tk);
  if (!toks) return throw_msg(env, "selfSpeculative: out of memory");
  memcpy(tk, out.data(), (size_t)n * 4);
  napi_value o, v;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "tokens", toks);
  napi_create_int32(env, st.rounds, &v);
  napi_set_named_property(env, o, "rounds", v);
  napi_create_int32(env, st.drafted, &v);
  napi_set_named_property(env, o, "drafted", v);
  napi_create_int32(env, st.accepted, &v);
  napi_set_named_property(env, o, "accepted", v);
  napi_create_double(env, st.prefill_ms, &v);
  napi_set_named_property(env, o, "prefillMs", v);
  napi_create_double(env, st.decode_ms, &v);
  napi_set_named_property(env, o, "decodeMs", v);
  return o;
}

napi_value ModuleInit(napi_env env, napi_value exports) {
  struct {
    const char *name;
    napi_callback cb;
  } fns[] = {{"init", Init},
             {"deviceInfo", DeviceInfo},
             {"upload", Upload},
             {"uploadQ8Ref", UploadQ8Ref},
             {"free", Free},
             {"linear", Linear},
             {"dequant", Dequant},
             {"info", Info},
             {"modelCreate", ModelCreate},
             {"modelLoadGGUF", ModelLoadGGUF},
             {"modelSetTensor", ModelSetTensor},
             {"modelForward", ModelForward},
             {"modelForwardBatch", ModelForwardBatch},
             {"modelGenerate", ModelGenerate},
             {"modelRollback", ModelRollback},
             {"modelReset", ModelReset},
             {"modelFree", ModelFree},
             {"speculative", Speculative},
             {"selfSpeculative", SelfSpeculative}};
  for (auto &f : fns) {
    napi_value fn;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn);
    napi_set_named_property(env, exports, f.name, fn);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, ModuleInit)
