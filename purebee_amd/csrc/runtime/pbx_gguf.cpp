// pbx_gguf.cpp -- GGUF reader and the file -> resident model path.
//
// The file is mapped read-only once; the header, metadata and tensor table
// are parsed with bounds checks on every read (a truncated or corrupt file
// is an error, never an out-of-range read), and tensor data is handed to
// pbx_model_set_tensor straight from the mapping, so each weight byte is
// copied to the device once through the pinned staging buffers.
//
// Format (little-endian), as the reference parses it (gguf.js:76-194,
// streaming-loader.js:35-87):
//   u32 magic "GGUF", u32 version (2 or 3), u64 tensor count, u64 kv count
//   kv:     string key, u32 value type, value
//   tensor: string name, u32 n_dims, u64 dims[n_dims], u32 ggml type,
//           u64 offset (relative to the data section)
//   data section: starts at the end of the tensor table rounded up to
//   general.alignment (default 32)
// where a string is u64 length + bytes and an array is u32 element type +
// u64 count + elements.

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <vector>

#include "pbx_internal.h"

#define PBX_GGUF_MAGIC 0x46554747u  // "GGUF"

namespace {

// GGUF metadata value types (gguf.js:24-27).
enum : uint32_t {
  V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
  V_STR = 8, V_ARR = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12,
};

struct KV {
  std::string key;
  uint32_t type = 0;
  int64_t i = 0;           // integer / bool values
  double f = 0.0;          // float values (and integers, converted)
  const char *s = nullptr; // string values: view into the mapping
  uint64_t slen = 0;
  uint32_t arr_type = 0;   // arrays
  uint64_t arr_count = 0;
};

struct TensorInfo {
  std::string name;
  int32_t type = 0;
  int32_t n_dims = 0;
  int64_t dims[4] = {1, 1, 1, 1};
  uint64_t rel_offset = 0, offset = 0, nbytes = 0;
};

// Block size and bytes per block of the tensor types the reference can size
// (GGML_TYPE_SIZE, gguf.js:36-49).
bool type_size(int32_t t, int64_t *block, int64_t *bytes) {
  switch (t) {
    case 0: *block = 1; *bytes = 4; return true;      // F32
    case 1: *block = 1; *bytes = 2; return true;      // F16
    case 2: *block = 32; *bytes = 18; return true;    // Q4_0
    case 3: *block = 32; *bytes = 20; return true;    // Q4_1
    case 8: *block = 32; *bytes = 34; return true;    // Q8_0
    case 9: *block = 32; *bytes = 36; return true;    // Q8_1
    case 10: *block = 256; *bytes = 84; return true;  // Q2_K
    case 11: *block = 256; *bytes = 110; return true; // Q3_K
    case 12: *block = 256; *bytes = 144; return true; // Q4_K
    case 13: *block = 256; *bytes = 176; return true; // Q5_K
    case 14: *block = 256; *bytes = 210; return true; // Q6_K
    case 15: *block = 256; *bytes = 292; return true; // Q8_K
    default: return false;
  }
}

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
  const uint8_t *p;
  uint64_t size, pos = 0;
  bool ok = true;
  bool need(uint64_t n) {
    if (!ok || n > size - pos) ok = false;
    return ok;
  }
  template <typename T>
  T get() {
    T v{};
    if (need(sizeof(T))) {
      memcpy(&v, p + pos, sizeof(T));
      pos += sizeof(T);
    }
    return v;
  }
  bool str(const char **s, uint64_t *len) {
    const uint64_t n = get<uint64_t>();
    if (!need(n)) return false;
    *s = (const char *)(p + pos);
    *len = n;
    pos += n;
    return true;
  }
};

// Reads one value of `type` into kv (scalars and strings) or skips it
// (array elements).  depth bounds nested arrays.
bool read_value(Cursor &c, uint32_t type, KV *kv, int depth) {
  switch (type) {
    case V_U8: { uint8_t v = c.get<uint8_t>(); if (kv) kv->i = v, kv->f = v; break; }
    case V_I8: { int8_t v = c.get<int8_t>(); if (kv) kv->i = v, kv->f = v; break; }
    case V_U16: { uint16_t v = c.get<uint16_t>(); if (kv) kv->i = v, kv->f = v; break; }
    case V_I16: { int16_t v = c.get<int16_t>(); if (kv) kv->i = v, kv->f = v; break; }
    case V_U32: { uint32_t v = c.get<uint32_t>(); if (kv) kv->i = v, kv->f = v; break; }
    case V_I32: { int32_t v = c.get<int32_t>(); if (kv) kv->i = v, kv->f = v; break; }
    case V_F32: { float v = c.get<float>(); if (kv) kv->f = v, kv->i = (int64_t)v; break; }
    case V_BOOL: { uint8_t v = c.get<uint8_t>(); if (kv) kv->i = v != 0, kv->f = v != 0; break; }
    case V_U64: {
      uint64_t v = c.get<uint64_t>();
      if (kv) kv->i = (int64_t)v, kv->f = (double)v;
      break;
    }
    case V_I64: { int64_t v = c.get<int64_t>(); if (kv) kv->i = v, kv->f = (double)v; break; }
    case V_F64: { double v = c.get<double>(); if (kv) kv->f = v, kv->i = (int64_t)v; break; }
    case V_STR: {
      const char *s;
      uint64_t n;
      if (!c.str(&s, &n)) return false;
      if (kv) kv->s = s, kv->slen = n;
      break;
    }
    case V_ARR: {
      if (depth > 4) return false;
      const uint32_t et = c.get<uint32_t>();
      const uint64_t n = c.get<uint64_t>();
      if (!c.ok) return false;
      if (kv) kv->arr_type = et, kv->arr_count = n;
      // fixed-size elements are skipped in one step (bounded by the file)
      static const uint64_t kSize[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
      if (et <= V_F64 && kSize[et]) {
        if (n > (c.size - c.pos) / kSize[et]) return c.ok = false;
        c.pos += n * kSize[et];
      } else {
        for (uint64_t k = 0; k < n && c.ok; ++k)
          if (!read_value(c, et, nullptr, depth + 1)) return false;
      }
      break;
    }
    default: return false;
  }
  return c.ok;
}

}  // namespace

struct pbx_gguf {
  uint32_t magic = 0x50424747u;  // "PBGG"
  int fd = -1;
  const uint8_t *map = nullptr;
  uint64_t size = 0;
  uint32_t version = 0;
  uint64_t alignment = 32, data_start = 0;
  std::vector<KV> kv;
  std::vector<TensorInfo> tensors;
};

static bool gguf_ok(const pbx_gguf *g) { return g && g->magic == 0x50424747u; }

static void gguf_release(pbx_gguf *g) {
  if (!g) return;
  if (g->map) munmap((void *)g->map, g->size);
  if (g->fd >= 0) close(g->fd);
  g->magic = 0;
  delete g;
}

static const KV *find_kv(const pbx_gguf *g, const char *key) {
  for (const KV &e : g->kv)
    if (e.key == key) return &e;
  return nullptr;
}

static bool is_int_type(uint32_t t) {
  return t <= V_I32 || t == V_BOOL || t == V_U64 || t == V_I64;
}

extern "C" int pbx_gguf_open(const char *path, pbx_gguf **out) {
  if (!path || !out) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_open: NULL argument");
  *out = nullptr;
  pbx_gguf *g = new pbx_gguf();
  g->fd = open(path, O_RDONLY | O_CLOEXEC);
  struct stat st;
  if (g->fd < 0 || fstat(g->fd, &st) != 0) {
    const int e = errno;
    gguf_release(g);
    return pbx_fail(nullptr, PBX_EIO, "pbx_gguf_open: cannot open %s: %s", path, strerror(e));
  }
  g->size = (uint64_t)st.st_size;
  if (g->size < 24) {
    const unsigned long long n = g->size;
    gguf_release(g);
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_open: %s: %llu bytes is too short for GGUF",
                    path, n);
  }
  void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
  if (m == MAP_FAILED) {
    const int e = errno;
    gguf_release(g);
    return pbx_fail(nullptr, PBX_EIO, "pbx_gguf_open: mmap of %s failed: %s", path, strerror(e));
  }
  g->map = (const uint8_t *)m;
  Cursor c{g->map, g->size};
  auto bad = [&](const char *what) {
    const uint64_t at = c.pos;
    gguf_release(g);
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_open: %s: %s (at byte %llu)", path, what,
                    (unsigned long long)at);
  };
  // readHeader (gguf.js:144-155)
  const uint32_t magic = c.get<uint32_t>();
  if (magic != PBX_GGUF_MAGIC) {
    gguf_release(g);
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_open: %s: not a GGUF file (magic 0x%x)",
                    path, magic);
  }
  g->version = c.get<uint32_t>();
  if (g->version < 2 || g->version > 3) {
    const uint32_t v = g->version;
    gguf_release(g);
    return pbx_fail(nullptr, PBX_ENOTSUP, "pbx_gguf_open: %s: GGUF version %u (supports 2-3)",
                    path, v);
  }
  const uint64_t n_tensors = c.get<uint64_t>();
  const uint64_t n_kv = c.get<uint64_t>();
  // every kv takes >= 13 bytes and every tensor >= 24: counts beyond that
  // cannot be honest
  if (n_kv > g->size / 13 || n_tensors > g->size / 24) return bad("implausible counts");
  // readMetadata (gguf.js:157-166)
  g->kv.reserve(n_kv);
  for (uint64_t i = 0; i < n_kv; ++i) {
    KV e;
    const char *k;
    uint64_t kl;
    if (!c.str(&k, &kl)) return bad("truncated metadata key");
    e.key.assign(k, kl);
    e.type = c.get<uint32_t>();
    if (!c.ok) return bad("truncated metadata");
    if (!read_value(c, e.type, &e, 0)) return bad("bad or truncated metadata value");
    g->kv.push_back(std::move(e));
  }
  if (const KV *a = find_kv(g, "general.alignment")) {
    if (!is_int_type(a->type) || a->i <= 0 || a->i > (1 << 20)) return bad("bad general.alignment");
    g->alignment = (uint64_t)a->i;
  }
  // readTensorInfos (gguf.js:168-183)
  g->tensors.reserve(n_tensors);
  for (uint64_t i = 0; i < n_tensors; ++i) {
    TensorInfo t;
    const char *s;
    uint64_t sl;
    if (!c.str(&s, &sl)) return bad("truncated tensor name");
    t.name.assign(s, sl);
    const uint32_t nd = c.get<uint32_t>();
    if (!c.ok || nd == 0 || nd > 4) return bad("bad tensor dimension count");
    t.n_dims = (int32_t)nd;
    for (uint32_t d = 0; d < nd; ++d) {
      const uint64_t v = c.get<uint64_t>();
      if (v == 0 || v > (1ull << 40)) return bad("bad tensor dimension");
      t.dims[d] = (int64_t)v;
    }
    t.type = (int32_t)c.get<uint32_t>();
    t.rel_offset = c.get<uint64_t>();
    if (!c.ok) return bad("truncated tensor table");
    g->tensors.push_back(std::move(t));
  }
  // data section (streaming-loader.js:62-63)
  g->data_start = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
  for (TensorInfo &t : g->tensors) {
    int64_t block, bytes;
    if (!type_size(t.type, &block, &bytes)) {
      char msg[160];
      snprintf(msg, sizeof msg, "tensor %s: unsupported tensor type %d", t.name.c_str(), t.type);
      return bad(msg);
    }
    // tensorByteSize (gguf.js:206-213)
    uint64_t n = 1;
    for (int d = 0; d < t.n_dims; ++d) {
      if ((uint64_t)t.dims[d] > (1ull << 62) / n) return bad("tensor too large");
      n *= (uint64_t)t.dims[d];
    }
    const uint64_t blocks = (n + block - 1) / block;
    if (blocks > g->size / (uint64_t)bytes) {  // cannot fit, and the product could wrap
      char msg[200];
      snprintf(msg, sizeof msg, "tensor %s: %llu elements do not fit in the file", t.name.c_str(),
               (unsigned long long)n);
      return bad(msg);
    }
    t.nbytes = blocks * bytes;
    t.offset = g->data_start + t.rel_offset;
    if (t.rel_offset > g->size || t.offset > g->size || t.nbytes > g->size - t.offset) {
      char msg[200];
      snprintf(msg, sizeof msg, "tensor %s: data [%llu, +%llu) past the end of the file",
               t.name.c_str(), (unsigned long long)t.offset, (unsigned long long)t.nbytes);
      return bad(msg);
    }
  }
  *out = g;
  return PBX_OK;
}

extern "C" void pbx_gguf_close(pbx_gguf *g) {
  if (gguf_ok(g)) gguf_release(g);
}

extern "C" int pbx_gguf_info(const pbx_gguf *g, uint32_t *version, int64_t *n_tensors,
                             int64_t *n_kv, uint64_t *data_start) {
  if (!gguf_ok(g)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_info: not an open GGUF file");
  if (version) *version = g->version;
  if (n_tensors) *n_tensors = (int64_t)g->tensors.size();
  if (n_kv) *n_kv = (int64_t)g->kv.size();
  if (data_start) *data_start = g->data_start;
  return PBX_OK;
}

extern "C" int pbx_gguf_tensor_info(const pbx_gguf *g, int64_t i, pbx_gguf_tensor *out) {
  if (!gguf_ok(g) || !out) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_tensor_info: bad argument");
  if (i < 0 || i >= (int64_t)g->tensors.size())
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_tensor_info: index %lld out of range",
                    (long long)i);
  const TensorInfo &t = g->tensors[(size_t)i];
  out->name = t.name.c_str();
  out->type = t.type;
  out->n_dims = t.n_dims;
  for (int d = 0; d < 4; ++d) out->dims[d] = t.dims[d];
  out->offset = t.offset;
  out->nbytes = t.nbytes;
  out->data = g->map + t.offset;
  return PBX_OK;
}

extern "C" int64_t pbx_gguf_find_tensor(const pbx_gguf *g, const char *name) {
  if (!gguf_ok(g) || !name) return -1;
  for (size_t i = 0; i < g->tensors.size(); ++i)
    if (g->tensors[i].name == name) return (int64_t)i;
  return -1;
}

extern "C" int pbx_gguf_get_int(const pbx_gguf *g, const char *key, int64_t *out) {
  if (!gguf_ok(g) || !key || !out) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_int: bad argument");
  const KV *e = find_kv(g, key);
  if (!e) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_int: no key %s", key);
  if (!is_int_type(e->type))
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_int: %s has value type %u", key, e->type);
  *out = e->i;
  return PBX_OK;
}

extern "C" int pbx_gguf_get_float(const pbx_gguf *g, const char *key, double *out) {
  if (!gguf_ok(g) || !key || !out) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_float: bad argument");
  const KV *e = find_kv(g, key);
  if (!e) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_float: no key %s", key);
  if (e->type != V_F32 && e->type != V_F64 && !is_int_type(e->type))
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_float: %s has value type %u", key, e->type);
  *out = e->f;
  return PBX_OK;
}

extern "C" int pbx_gguf_get_string(const pbx_gguf *g, const char *key, const char **str,
                                   uint64_t *len) {
  if (!gguf_ok(g) || !key || !str || !len)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_string: bad argument");
  const KV *e = find_kv(g, key);
  if (!e) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_string: no key %s", key);
  if (e->type != V_STR)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_string: %s has value type %u", key, e->type);
  *str = e->s;
  *len = e->slen;
  return PBX_OK;
}

extern "C" int pbx_gguf_get_array(const pbx_gguf *g, const char *key, uint32_t *elem_type,
                                  uint64_t *count) {
  if (!gguf_ok(g) || !key || !elem_type || !count)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_array: bad argument");
  const KV *e = find_kv(g, key);
  if (!e) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_array: no key %s", key);
  if (e->type != V_ARR)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_get_array: %s has value type %u", key, e->type);
  *elem_type = e->arr_type;
  *count = e->arr_count;
  return PBX_OK;
}

// ---------------------------------------------------------------------------
// Model config and loading.
// ---------------------------------------------------------------------------

// extractConfig (gguf.js:429-450) keyed by general.architecture, with the
// reference's defaults; the vocabulary is the tokenizer's token count
// (streaming-loader.js:57) where it is present, else token_embd's rows.
extern "C" int pbx_gguf_model_config(const pbx_gguf *g, int max_seq, pbx_model_config *cfg) {
  if (!gguf_ok(g) || !cfg)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_model_config: bad argument");
  std::string arch = "llama";
  if (const KV *a = find_kv(g, "general.architecture"))
    if (a->type == V_STR) arch.assign(a->s, a->slen);
  auto geti = [&](const char *suffix, int64_t dflt, int64_t *v) -> bool {
    const KV *e = find_kv(g, (arch + "." + suffix).c_str());
    if (!e || !is_int_type(e->type) || e->i == 0) {
      *v = dflt;
      return dflt > 0;
    }
    *v = e->i;
    return true;
  };
  auto getf = [&](const char *suffix, double dflt) -> double {
    const KV *e = find_kv(g, (arch + "." + suffix).c_str());
    if (!e || (e->type != V_F32 && e->type != V_F64 && !is_int_type(e->type)) || e->f == 0)
      return dflt;
    return e->f;
  };
  int64_t dim, hidden, layers, heads, kv_heads, ctx_len;
  if (!geti("embedding_length", 0, &dim) || !geti("feed_forward_length", 0, &hidden) ||
      !geti("block_count", 0, &layers) || !geti("attention.head_count", 0, &heads))
    return pbx_fail(nullptr, PBX_EINVAL,
                    "pbx_gguf_model_config: missing %s.embedding_length / feed_forward_length / "
                    "block_count / attention.head_count",
                    arch.c_str());
  geti("attention.head_count_kv", heads, &kv_heads);
  geti("context_length", 2048, &ctx_len);
  const int64_t ie = pbx_gguf_find_tensor(g, "token_embd.weight");
  if (ie < 0) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_model_config: no token_embd.weight");
  const TensorInfo &te = g->tensors[(size_t)ie];
  int64_t vocab = te.n_dims >= 2 ? te.dims[1] : 0;
  uint32_t et;
  uint64_t n_tok;
  const KV *tok = find_kv(g, "tokenizer.ggml.tokens");
  if (tok && tok->type == V_ARR) {
    et = tok->arr_type;
    n_tok = tok->arr_count;
    if (et == V_STR && n_tok > 0 && (int64_t)n_tok <= vocab) vocab = (int64_t)n_tok;
  }
  const int64_t iq = pbx_gguf_find_tensor(g, "blk.0.attn_q.weight");
  if (iq < 0) return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_model_config: no blk.0.attn_q.weight");
  const int64_t io = pbx_gguf_find_tensor(g, "output.weight");
  memset(cfg, 0, sizeof *cfg);
  cfg->dim = (int32_t)dim;
  cfg->hidden_dim = (int32_t)hidden;
  cfg->n_layers = (int32_t)layers;
  cfg->n_heads = (int32_t)heads;
  cfg->n_kv_heads = (int32_t)kv_heads;
  cfg->head_dim = (int32_t)(dim / heads);  // gguf.js:447
  cfg->vocab_size = (int32_t)vocab;
  cfg->max_seq = max_seq > 0 ? max_seq : (int32_t)std::min<int64_t>(ctx_len, 8192);
  cfg->weight_type = g->tensors[(size_t)iq].type;
  cfg->embed_type = te.type;
  cfg->output_type = io >= 0 ? g->tensors[(size_t)io].type : -1;
  cfg->rms_eps = (float)getf("attention.layer_norm_rms_epsilon", 1e-5);
  cfg->rope_theta = getf("rope.freq_base", 10000.0);
  if (dim > INT32_MAX || hidden > INT32_MAX || layers > 4096 || heads <= 0 || kv_heads <= 0 ||
      vocab <= 0 || vocab > INT32_MAX)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_gguf_model_config: implausible model sizes");
  return PBX_OK;
}

// mapTensorName (gguf.js:378-410) onto the PBX_T_* ids; -1 for tensors the
// model does not take.
static int tensor_id(const std::string &name, int *layer) {
  *layer = -1;
  if (name == "token_embd.weight") return PBX_T_TOKEN_EMBD;
  if (name == "output.weight") return PBX_T_OUTPUT;
  if (name == "output_norm.weight") return PBX_T_OUTPUT_NORM;
  if (name.compare(0, 4, "blk.") != 0) return -1;
  size_t p = 4;
  int l = 0;
  while (p < name.size() && name[p] >= '0' && name[p] <= '9' && l < (1 << 20))
    l = l * 10 + (name[p++] - '0');
  if (p == 4 || p >= name.size() || name[p] != '.') return -1;
  const std::string suffix = name.substr(p + 1);
  static const struct { const char *s; int id; } kMap[] = {
      {"attn_norm.weight", PBX_T_ATTN_NORM}, {"ffn_norm.weight", PBX_T_FFN_NORM},
      {"attn_q.weight", PBX_T_ATTN_Q},       {"attn_k.weight", PBX_T_ATTN_K},
      {"attn_v.weight", PBX_T_ATTN_V},       {"attn_output.weight", PBX_T_ATTN_OUTPUT},
      {"ffn_gate.weight", PBX_T_FFN_GATE},   {"ffn_up.weight", PBX_T_FFN_UP},
      {"ffn_down.weight", PBX_T_FFN_DOWN},
  };
  for (const auto &e : kMap)
    if (suffix == e.s) {
      *layer = l;
      return e.id;
    }
  return -1;
}

// [N rows][K] each tensor id must have under cfg (norms: one row of dim).
static void expected_shape(int id, const pbx_model_config &g, int64_t *N, int64_t *K) {
  const int64_t kv = (int64_t)g.n_kv_heads * g.head_dim;
  switch (id) {
    case PBX_T_ATTN_Q: case PBX_T_ATTN_OUTPUT: *N = g.dim; *K = g.dim; break;
    case PBX_T_ATTN_K: case PBX_T_ATTN_V: *N = kv; *K = g.dim; break;
    case PBX_T_FFN_GATE: case PBX_T_FFN_UP: *N = g.hidden_dim; *K = g.dim; break;
    case PBX_T_FFN_DOWN: *N = g.dim; *K = g.hidden_dim; break;
    default: *N = 1; *K = g.dim; break;  // norms
  }
}

extern "C" int pbx_model_load_gguf(pbx_ctx *c, const char *path, int max_seq, pbx_model **out) {
  if (!c || !path || !out) return pbx_fail(c, PBX_EINVAL, "pbx_model_load_gguf: NULL argument");
  *out = nullptr;
  pbx_gguf *g = nullptr;
  int rc = pbx_gguf_open(path, &g);
  if (rc) return pbx_fail(c, rc, "%s", pbx_last_error(nullptr));
  pbx_model_config cfg;
  rc = pbx_gguf_model_config(g, max_seq, &cfg);
  if (rc) {
    pbx_gguf_close(g);
    return pbx_fail(c, rc, "%s", pbx_last_error(nullptr));
  }
  // Attention / FFN biases and other extra tensors of non-Llama families are
  // not part of the model: refuse rather than drop them silently.
  for (const TensorInfo &t : g->tensors) {
    int layer;
    const int id = tensor_id(t.name, &layer);
    const bool known_extra = t.name == "rope_freqs.weight";
    if (id < 0 && !known_extra) {
      rc = pbx_fail(c, PBX_ENOTSUP, "pbx_model_load_gguf: tensor %s is not part of a Llama model",
                    t.name.c_str());
      pbx_gguf_close(g);  // t is gone after this
      return rc;
    }
    if (id >= PBX_T_ATTN_Q && t.type != cfg.weight_type) {
      rc = pbx_fail(c, PBX_ENOTSUP,
                    "pbx_model_load_gguf: %s has type %d, blk.0.attn_q.weight has %d (one type "
                    "for every layer matrix)",
                    t.name.c_str(), t.type, cfg.weight_type);
      pbx_gguf_close(g);
      return rc;
    }
  }
  pbx_model *m = nullptr;
  rc = pbx_model_create(c, &cfg, &m);
  if (rc) {
    pbx_gguf_close(g);
    return rc;
  }
  for (const TensorInfo &t : g->tensors) {
    int layer;
    const int id = tensor_id(t.name, &layer);
    if (id < 0) continue;
    // GGUF dims[0] is the row length (K), dims[1] the row count (N).
    const int64_t K = t.dims[0], N = t.n_dims >= 2 ? t.dims[1] : 1;
    const bool norm = id == PBX_T_OUTPUT_NORM || id == PBX_T_ATTN_NORM || id == PBX_T_FFN_NORM;
    if (norm && t.type != 0) {
      rc = pbx_fail(c, PBX_ENOTSUP, "pbx_model_load_gguf: norm %s has type %d (F32 expected)",
                    t.name.c_str(), t.type);
      break;
    }
    size_t bytes = (size_t)t.nbytes;
    if (id != PBX_T_TOKEN_EMBD && id != PBX_T_OUTPUT) {
      int64_t eN, eK;
      expected_shape(id, cfg, &eN, &eK);
      if (K != eK || N != eN || t.n_dims > 2) {
        rc = pbx_fail(c, PBX_EINVAL, "pbx_model_load_gguf: %s is [%lld, %lld], expected [%lld, %lld]",
                      t.name.c_str(), (long long)K, (long long)N, (long long)eK, (long long)eN);
        break;
      }
    } else {
      // rows past the tokenizer's vocabulary are never produced or looked up
      if (K != cfg.dim || N < cfg.vocab_size) {
        rc = pbx_fail(c, PBX_EINVAL, "pbx_model_load_gguf: %s is [%lld, %lld], expected [%d, >= %d]",
                      t.name.c_str(), (long long)K, (long long)N, cfg.dim, cfg.vocab_size);
        break;
      }
      bytes = (size_t)cfg.vocab_size * pbx_type_row_bytes(t.type, K);
    }
    rc = pbx_model_set_tensor(m, id, layer, g->map + t.offset, bytes);
    if (rc) break;
  }
  pbx_gguf_close(g);
  if (rc) {
    pbx_model_free(m);
    return rc;
  }
  *out = m;
  return PBX_OK;
}
