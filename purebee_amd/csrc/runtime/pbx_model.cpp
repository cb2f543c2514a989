// pbx_model.cpp -- resident Llama-family model and its on-GPU decode step.
//
// The reference's decode layer (_runLayerQ4, llama-streaming.js:505-606; the
// same math as LlamaRuntime.forward, llama.js:204-371) runs here as 5 kernels
// per layer plus embedding, LM head and argmax (see pbx_decode.hip).  One
// step is captured once into a HIP graph and replayed: the token and the
// position live in device memory, the argmax kernel writes the next token and
// advances the position, so greedy decoding never returns to the host between
// tokens.  Weights are uploaded once; q|k|v and gate|up are stored as one
// matrix each so a single GEMV reads them.

#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "pbx_internal.h"

#define PBX_MODEL_MAGIC 0x5042584Du  // "PBXM"

namespace {

using GemvArgsHost = pbx_gemv_args;

struct AttnArgsHost {  // AttnArgs in pbx_decode.hip
  const float *qkv;
  float *kcache, *vcache;
  const float *rope;
  float *out;
  const int *state;
  int n_heads, n_kv_heads, head_dim;
  float scale;
  int max_seq;
  // pbx_attention_o_*: o projection planes, pending update, residual row
  const void *oqs = nullptr;
  const void *odsc = nullptr;
  long long *oacc = nullptr;
  float *ox = nullptr;
  // pbx_qkvr_attn_o_*: the GEMV's published rows and their epoch at [cell_n]
  const unsigned long long *cells = nullptr;
  int cell_n = 0, qdim = 0;
  // the status word a bounded wait marks when it gives up, the poll limit
  // (0: the kernel's default) and the test-only tag offset
  int *status = nullptr;
  int spin = 0, skew = 0;
  // the small-model step: the tag's epoch and the published head outputs
  const unsigned long long *epoch = nullptr;
  unsigned long long *ocells = nullptr;
};

struct AttnSplitArgsHost {  // AttnSplitArgs in pbx_decode.hip
  const float *qkv;
  float *kcache, *vcache;
  const float *rope;
  float *out;
  const int *state;
  float *part;
  int n_heads, n_kv_heads, head_dim, S;
  float scale;
};

struct CombineArgsHost {  // pbx_attention_combine's parameters
  const float *part;
  float *out;
  int head_dim, S;
};

struct EmbedArgsHost {  // EmbedArgs in pbx_decode.hip
  const void *qs;
  const void *dsc;
  float *x;
  const int *state;
  int type;
  int dim, vocab;
  const void *msc;
};

struct ArgmaxArgsHost {  // ArgmaxArgs in pbx_decode.hip
  const uint64_t *partials;
  int *state;
  int *hist;
  int n_partials;
  int hist_cap;
  EmbedArgsHost emb;
  long long *clr = nullptr;
  int clr_n = 0;
};

struct FfnArgsHost {  // FfnArgs in pbx_decode.hip
  const void *qs = nullptr;
  const void *dsc = nullptr;
  const float *x = nullptr;
  const long long *acc = nullptr;
  unsigned long long *cell = nullptr;
  float *xout = nullptr;
  unsigned long long *qepoch = nullptr;
  int *status = nullptr;
  int spin = 0;
};

struct SmallLayerHost {  // SmallLayer in pbx_decode.hip
  const void *qkv_qs, *o_qs, *gu_qs, *d_qs;
  const void *qkv_d, *o_d, *gu_d, *d_d;
  const float *attn_norm, *ffn_norm;
};

struct SmallArgsHost {  // SmallArgs in pbx_decode.hip
  const SmallLayerHost *layers = nullptr;
  AttnArgsHost at{};
  long long layer_kv = 0;
  unsigned long long *cells = nullptr;
  long long cell_stride = 0;
  unsigned long long *epoch = nullptr;
  unsigned *done = nullptr;
  float *x = nullptr;
  int n_layers = 0, dim = 0, hidden = 0, qkv_rows = 0;
  float eps = 0.f;
  int rq = 0, ro = 0, rg = 0, rd = 0;
  int test_layer = -1, skew = 0;
};

enum ArgKind {
  ARG_GEMV, ARG_ATTN, ARG_ATTN_SPLIT, ARG_COMBINE, ARG_EMBED, ARG_ARGMAX, ARG_FUSED, ARG_FFN,
  ARG_SMALL
};
enum AttnMode { ATTN_HEAD, ATTN_SPLIT, ATTN_DECODE };

struct Op {
  hipFunction_t f = nullptr;
  std::string name;
  std::string role;      // embed / qkv / attn / o / gate_up / down / lm_head / argmax
  double bytes = 0;      // algorithmic bytes per launch (attention: per cached position)
  double fixed_bytes = 0;  // attention: bytes per launch on top (the fused o projection)
  dim3 grid, block;
  ArgKind kind;
  GemvArgsHost gemv;
  AttnArgsHost attn;
  AttnSplitArgsHost split;
  CombineArgsHost comb;
  EmbedArgsHost embed;
  ArgmaxArgsHost amax;
  FfnArgsHost ffn;  // ARG_FFN: the down projection's arguments (gemv: gate|up)
  SmallArgsHost small;  // ARG_SMALL: every layer of the step in one launch
  int np = 0;  // ARG_FUSED: GEMV workgroups before the attention's
};

struct Layer {
  pbx_weight *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wd = nullptr;
  float *attn_norm = nullptr, *ffn_norm = nullptr;
  unsigned set_mask = 0;
};

const char *type_tag(int t) {
  switch (t) {
    case PBX_TYPE_Q4_0: return "q4";
    case PBX_TYPE_Q4_1: return "q41";
    case PBX_TYPE_Q8_0: return "q8";
    case PBX_TYPE_F16: return "f16";
    case PBX_TYPE_Q6_K: return "q6k";
    default: return "f32";
  }
}

// PBX_Q4 / PBX_Q8 / PBX_F32 / PBX_Q41 / PBX_F16 / PBX_Q6K of pbx_gemv_impl.h
int kernel_type(int t) {
  switch (t) {
    case PBX_TYPE_Q4_0: return 0;
    case PBX_TYPE_Q8_0: return 1;
    case PBX_TYPE_Q4_1: return 3;
    case PBX_TYPE_F16: return 4;
    case PBX_TYPE_Q6_K: return 5;
    default: return 2;
  }
}

}  // namespace

struct pbx_model {
  uint32_t magic = 0;
  pbx_ctx *c = nullptr;
  pbx_model_config cfg;
  int kvdim = 0, qkv_rows = 0;
  std::vector<Layer> layers;
  pbx_weight *embd = nullptr, *output = nullptr;
  // lane-packed copy of a Q6_K LM head for the integer-limb kernel (26 bytes
  // per 32-block; its d stays in the head's scale plane)
  void *head_lanes = nullptr;
  float *out_norm = nullptr;
  unsigned global_mask = 0;
  float *kcache = nullptr, *vcache = nullptr, *rope = nullptr;
  float *x = nullptr, *qkv = nullptr, *attn = nullptr, *gu = nullptr, *logits = nullptr;
  // the residual's pending update [dim] (2^-32 fixed point) between the
  // fused attention + o projection and the down GEMV of a layer; zero
  // outside that span.  With the joined FFN launch: [2][dim], layer l
  // accumulating into [l % 2] while the launch of layer l clears the other
  // (and the step's argmax both)
  long long *xacc = nullptr;
  // joined FFN launch (dim 2048, hidden 8192, Q4_0; PBX_FFN=0 at creation:
  // separate gate|up and down): the residual rows alternate between x
  // (even layers' input) and x2, the down slices meet in ffn_cell [dim]
  // (zero between launches), and each layer publishes its SwiGLU outputs
  // in h_cells [n_layers][hidden + 64] (their epoch at [hidden])
  bool ffn_join = true, ffn_joined = false;
  float *x2 = nullptr;
  unsigned long long *ffn_cell = nullptr, *h_cells = nullptr;
  // small models (pbx_small_step_q8; PBX_SMALL_STEP=0 at creation: a launch
  // per GEMV and attention): ops[0] runs every layer of the step; its layer
  // table, per-layer cells, the step epoch and the finished-workgroup count
  bool small_ok = true, small_step = false;
  SmallLayerHost *small_layers = nullptr;
  unsigned long long *small_cells = nullptr, *small_sync = nullptr;
  uint64_t *partials = nullptr;
  int n_partials_cap = 0;
  bool gemv_int = true;  // integer-limb GEMV kernels where they apply
  // split-position attention: S splits per KV head and their partials
  int attn_splits = 0;
  float *attn_part = nullptr;
  int attn_mode = 0;  // AttnMode
  // rows of the o projection per workgroup / 256 in the fused attention +
  // o projection (0: a separate o GEMV); PBX_ATTN_O=0|1|2|4 at creation,
  // default (-1) 2 where the q|k|v GEMV joins the launch, else 1
  int attn_o_ipt = -1;
  // q|k|v GEMV and attention + o projection in one launch (PBX_QKV_ATTN=0 at
  // creation: two launches); per layer, the GEMV's published rows and the
  // layer's epoch ((qkv_rows + 64) cells, allocated with the first step)
  bool qkv_attn = true;
  unsigned long long *qa_cells = nullptr;
  // state[0] position, [1] token, [2] step, [3] status word (bits set by
  // device-side waits that gave up; read and cleared by the host calls)
  int *state = nullptr;
  // pbx_model_test_handoff: the fused launch of layer test_layer waits for
  // tags offset by test_skew, with at most test_spin polls (0: default)
  int test_layer = -1, test_skew = 0, test_spin = 0;
  int *hist = nullptr;
  int hist_cap = 0;
  std::vector<Op> ops;
  // ops[layer_op[l]] is the first kernel of layer l; layer_op[n_layers] is
  // the LM head's (then the argmax)
  std::vector<size_t> layer_op;
  Op embed_op;  // the embedding of a token set by the host (steps embed their own)
  bool ops_ready = false;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  bool graph_tried = false, graph_ok = false;
  // pbx_model_generate: graph_steps whole steps captured back to back in one
  // graph (the steps chain through the device state), which saves the gap
  // between graph launches, and a 4-step graph for shorter remainders (a
  // speculative draft of 4); PBX_GRAPH_STEPS at creation (<= 1: off)
  int graph_steps = 8;
  hipGraph_t graph_k = nullptr, graph_k4 = nullptr;
  hipGraphExec_t exec_k = nullptr, exec_k4 = nullptr;
  bool graph_k_tried = false, graph_k_ok = false, graph_k4_tried = false, graph_k4_ok = false;
  // steps that stop after the first L < n_layers layers (forward with
  // maxLayers), one captured graph per L, made on first use
  struct PartGraph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool tried = false, ok = false;
  };
  std::vector<PartGraph> part;
  size_t bytes = 0;
  // Row-batched forward (prefill / verify): activations of up to batch_cap
  // rows, grown on demand; logits of every row up to logits_cap rows.
  int batch_cap = 0, logits_cap = 0;
  float *bx = nullptr, *bxn = nullptr, *bqkv = nullptr, *battn = nullptr, *bgu = nullptr,
        *bh = nullptr, *btmp = nullptr, *blogits = nullptr;
  int *bnext = nullptr;
  // the rows' tokens and next tokens in coherent pinned host memory
  // (batch_cap each), which the kernels read and write directly through
  // their device addresses d_tok / d_next: a verify then needs no copy
  // operation; tok_ev marks the last kernel that reads h_tok
  int32_t *h_tok = nullptr, *h_next = nullptr;
  int32_t *d_tok = nullptr, *d_next = nullptr;
  hipEvent_t tok_ev = nullptr;
  // [logits_cap][64]: per row, the running maximum key and the count of
  // pbx_argmax_rows (zero between launches)
  uint64_t *bkeys = nullptr;
  // rows GEMV with the K blocks split over workgroups (the down projection):
  // a 64-bit cell per output element [MR_MAX][dim] (zero between launches)
  unsigned long long *mr_cell = nullptr;
  // fused batched layers: the fp16 activation pair of the next GEMM and the
  // split-K partials of the last one
  void *g16 = nullptr, *g16lo = nullptr;
  float *ginv = nullptr, *gpart = nullptr;
  size_t g16_cap = 0, gpart_cap = 0;
};

static bool model_ok(const pbx_model *m) { return m && m->magic == PBX_MODEL_MAGIC; }

// Integer-limb GEMV kernels (K = 2048..8192): the gate|up GEMV for Q4_0 and
// Q8_0, 16 waves x 4 rows per workgroup (Q4_0, K <= 2048) when that still
// gives >= 256 workgroups, else 8 x 4; the other Q4_0 decode GEMVs with 4
// waves (qkv 4 rows, o / down 2, lm head 8 rows a wave in a tile loop at
// K = 2048, else 16).  PBX_GEMV_INT=0 at model creation selects the
// float-unpack kernels instead.
static bool int_gemv_disabled() {
  const char *e = getenv("PBX_GEMV_INT");
  return e && e[0] == '0';
}

// Integer-limb kernel shape: WV row waves x RT rows, IB blocks a lane, BW
// builder waves, PRE rows requested before the limb barrier (0: all), tile
// loop.  Kernel name part: i<WV>x<RT>b<IB>[w<BW>][p<PRE>][l].
struct IntShape {
  int wv = 4, rt = 1, ib = 1, bw = 0, pre = 0;
  bool loop = false;
};

// PBX_GEMV_INT_SHAPES="role=WVxRT[wBW][pPRE][l],..." (roles qkv, o, gate_up,
// down, lm_head; lm_head_q6k for a Q6_K head), read when the step is
// planned: the integer-limb kernel with WV row waves x RT rows (BW builder
// waves, PRE rows requested before the barrier) for the listed roles (Q4_0 /
// Q8_0, K = 2048..8192; a Q6_K head at K = 2048; a trailing l selects the
// lm head's tile loop), for tuning.  A shape that was not compiled fails
// the plan.
static bool int_override(const char *role, IntShape *sh) {
  const char *e = getenv("PBX_GEMV_INT_SHAPES");
  if (!e || !role) return false;
  const std::string s(e), key = std::string(role) + "=";
  size_t p = 0;
  while (p < s.size()) {
    size_t q = s.find(',', p);
    if (q == std::string::npos) q = s.size();
    const std::string item = s.substr(p, q - p);
    int wv, rt, n = 0;
    if (item.compare(0, key.size(), key) == 0 &&
        sscanf(item.c_str() + key.size(), "%dx%d%n", &wv, &rt, &n) == 2) {
      sh->wv = wv;
      sh->rt = rt;
      sh->bw = sh->pre = 0;
      const char *t = item.c_str() + key.size() + n;
      if (*t == 'w') sh->bw = (int)strtol(t + 1, (char **)&t, 10);
      if (*t == 'p') sh->pre = (int)strtol(t + 1, (char **)&t, 10);
      sh->loop = *t == 'l';
      return true;
    }
    p = q + 1;
  }
  return false;
}

static bool int_shape(bool enabled, const char *mode, const char *role, int type, int N, int B,
                      IntShape *sh) {
  if (!enabled || B < 64 || B > 256) return false;
  *sh = IntShape();
  sh->ib = (B + 63) / 64;
  if (type == PBX_TYPE_Q6_K) {  // the lm head at K = 2048: 4 waves x 4 rows, tile loop
    if (strcmp(mode, "lmh") != 0 || B != 64) return false;
    if (int_override("lm_head_q6k", sh)) return true;
    sh->wv = 4;
    sh->rt = 4;
    sh->loop = true;
    return true;
  }
  if (type != PBX_TYPE_Q4_0 && type != PBX_TYPE_Q8_0) return false;
  if (int_override(role, sh)) return sh->bw > 0 || sh->ib <= sh->wv;
  if (strcmp(mode, "gu") == 0 || strcmp(mode, "gua") == 0) {
    if (B > 128) return false;
    sh->rt = 4;
    if (type == PBX_TYPE_Q4_0 && sh->ib == 1 && N / 64 >= 256) {
      if (mode[2] == 'a') {
        // input x + pending update: 8 builder waves beside 8 row waves of 8
        // rows, whose first four are requested before the limb barrier
        sh->wv = 8;
        sh->rt = 8;
        sh->bw = 8;
        sh->pre = 4;
      } else {
        // 16 waves only for Q4_0 with one block per lane (register budget);
        // their first two rows requested before the limb barrier
        sh->wv = 16;
        sh->pre = 2;
      }
    } else {
      sh->wv = 8;
    }
    return true;
  }
  if (type != PBX_TYPE_Q4_0) return false;
  sh->wv = 4;
  if (strcmp(mode, "qkv") == 0) {
    sh->rt = 4;
    return sh->ib <= 2;
  }
  if (strcmp(mode, "add") == 0) {
    sh->rt = 2;
    if (sh->ib == 4) sh->bw = 4;  // K = 8192 (down): 4 builder waves (8: +0.4 us a token)
    return sh->ib != 3;
  }
  if (strcmp(mode, "lmh") == 0) {  // K = 2048: 8-row waves with the tile loop
    sh->rt = sh->ib == 1 ? 8 : 16;
    sh->loop = sh->ib == 1;
    return sh->ib <= 2;
  }
  return false;
}

// Kernel shape for a GEMV of N rows x B blocks (the same rules as the plain
// instruction): the integer-limb kernel for the gate|up GEMV where it
// applies; else the small-K kernel for B <= 32, otherwise ceil(B/64) waves
// per workgroup and the largest row tile that keeps >= 4 workgroups per CU.
static void plan_gemv(pbx_ctx *c, bool int_ok, const char *mode, const char *role, int type,
                      int N, int B, std::string *shape, dim3 *grid, dim3 *block, int *n_tiles) {
  IntShape sh;
  if (int_shape(int_ok, mode, role, type, N, B, &sh)) {
    const int wv = sh.wv, rt = sh.rt;
    const bool loop = sh.loop;
    *shape = "i" + std::to_string(wv) + "x" + std::to_string(rt) + "b" + std::to_string(sh.ib) +
             (sh.bw ? "w" + std::to_string(sh.bw) : "") +
             (sh.pre ? "p" + std::to_string(sh.pre) : "") + (loop ? "l" : "");
    const int tiles = (N + wv * rt - 1) / (wv * rt);
    // tile loop: two workgroups per CU (four for 4-row waves), each taking
    // every G-th tile
    // (Q6_K: two, its tile buffers are 64-byte lane blocks)
    const int per_cu = type == PBX_TYPE_Q6_K ? 2 : rt <= 4 ? 4 : 2;
    *grid = dim3(loop ? std::min(tiles, per_cu * c->cu_count) : tiles);
    *block = dim3(64 * (wv + sh.bw));
    *n_tiles = (int)grid->x;
    return;
  }
  const bool q4 = type == PBX_TYPE_Q4_0 || type == PBX_TYPE_Q4_1;
  if (strcmp(mode, "lmh") == 0 &&
      ((type == PBX_TYPE_F32 && (B == 8 || B == 9 || B == 12 || B == 16)) ||
       (type == PBX_TYPE_Q8_0 && (B == 8 || B == 9 || B == 12 || B == 16 || B == 18 || B == 24)))) {
    // f32 / Q8_0 heads with small K (stories15M, SmolLM2-135M): 8 lanes a
    // row, 64 rows a workgroup
    *shape = "t" + std::to_string(B);
    *grid = dim3((N + 63) / 64);
    *block = dim3(256);
    *n_tiles = (int)grid->x * 4;
    return;
  }
  if (B <= 32) {
    const int P = q4 ? 8 : type == PBX_TYPE_F32 ? 2 : 4;
    const int T = P * (64 / B);
    const int gx = (N + 4 * T - 1) / (4 * T);
    *shape = "s";
    *grid = dim3(gx);
    *block = dim3(256);
    *n_tiles = gx * 4;
    return;
  }
  const int W = (B + 63) / 64;
  const int target = std::max(4 * c->cu_count, 256);
  int R;
  if (q4)
    R = (N / 16 >= target) ? 16 : (N / 8 >= target) ? 8 : 4;
  else if (type == PBX_TYPE_Q8_0 || type == PBX_TYPE_F16 || type == PBX_TYPE_Q6_K)
    R = (N / 8 >= target) ? 8 : 4;
  else
    R = (N / 4 >= target) ? 4 : 2;
  *shape = "w" + std::to_string(R);
  *grid = dim3((N + R - 1) / R);
  *block = dim3(64 * W);
  *n_tiles = (int)grid->x;
}

static int add_gemv(pbx_model *m, const pbx_weight *w, const char *mode, const char *role,
                    const float *X, const float *X2, const float *normw, float *Y,
                    int *n_tiles_out) {
  pbx_ctx *c = m->c;
  Op op;
  op.kind = ARG_GEMV;
  std::string shape;
  int n_tiles = 0;
  // qkvr (RoPE + cache append epilogue) is planned as qkv, adda (folds the
  // pending update in) as add; gua (input x + pending update) has its own
  const char *plan_mode = strcmp(mode, "qkvr") == 0 ? "qkv"
                          : strcmp(mode, "adda") == 0 ? "add"
                                                      : mode;
  plan_gemv(c, m->gemv_int, plan_mode, role, w->type, (int)w->N, (int)w->B, &shape, &op.grid,
            &op.block, &n_tiles);
  if (w->B > 32 && (w->B + 63) / 64 > 8)
    return pbx_fail(c, PBX_ENOTSUP, "model: K=%lld exceeds the GEMV limit of 16384",
                    (long long)w->K);
  op.name = std::string("pbx_dk_") + type_tag(w->type) + "_" + shape + "_" + mode;
  op.f = pbx_kernel_by_name(c, op.name);
  if (!op.f) return pbx_fail(c, PBX_ELOAD, "model: kernel %s not found", op.name.c_str());
  op.gemv = GemvArgsHost{w->qs, w->d, X, X2, normw, nullptr, Y, m->partials, (int)w->N,
                         (int)w->B, m->cfg.rms_eps, w->m};
  op.role = role;
  // weights + activation reads (+ up for SwiGLU, + norm weight) + output
  // (read and written for the residual epilogue)
  // (+ the pending update: read by gua, read and cleared by adda)
  op.bytes = (double)w->N * pbx_type_row_bytes(w->type, w->K) + 4.0 * w->K * (X2 ? 2 : 1) +
             (normw ? 4.0 * w->K : 0.0) +
             (strcmp(plan_mode, "add") == 0                                  ? 8.0 * w->N
              : strcmp(plan_mode, "gu") == 0 || strcmp(plan_mode, "gua") == 0 ? 2.0 * w->N
                                                                              : 4.0 * w->N) +
             (strcmp(mode, "gua") == 0 ? 8.0 * w->K : strcmp(mode, "adda") == 0 ? 16.0 * w->N : 0.0);
  if (n_tiles_out) *n_tiles_out = n_tiles;
  m->ops.push_back(op);
  return PBX_OK;
}

static int dalloc(pbx_model *m, void **p, size_t bytes);

// Fills m->head_lanes from the resident Q6_K LM head (pbx_pack_q6_k_lanes).
static int pack_head_lanes(pbx_model *m) {
  const pbx_weight *head = m->output ? m->output : m->embd;
  hipFunction_t f = pbx_kernel_by_name(m->c, "pbx_pack_q6_k_lanes");
  if (!f) return pbx_fail(m->c, PBX_ELOAD, "model: kernel pbx_pack_q6_k_lanes not found");
  const void *qs = head->qs;
  void *dst = m->head_lanes;
  int N = (int)head->N, B = (int)head->B;
  void *args[] = {&qs, &dst, &N, &B};
  const int64_t total = (int64_t)N * B;
  return pbx_launch_fn(m->c, f, "pbx_pack_q6_k_lanes", dim3((unsigned)((total + 255) / 256)),
                       dim3(256), args, m->c->stream);
}

// Small models (pbx_small_step_q8: Q8_0 layers, dim <= 1024, hidden <=
// 4096, head_dim <= 64): the per-layer ops give way to one op that runs
// every layer of the step in G workgroups (ops[0]); the LM head and the
// argmax follow as before.  G starts at dim / 6 rounded up to a multiple of
// 8, at least 32 (measured: stories15M's dim 288 ran 109-110 us a token at
// 32-64 workgroups, SmolLM2's dim 576 435.6 at 96 against 463.5 at 64 and
// 441.3 at 128), and grows until the per-workgroup rows fit the kernel's
// task slots; it stays at or below the CU count (every workgroup must be
// resident) and at or above the query head count.  PBX_SMALL_WGS sets the
// start.
static int plan_small_step(pbx_model *m) {
  m->small_step = false;
  const pbx_model_config &g = m->cfg;
  pbx_ctx *c = m->c;
  const int nl = g.n_layers, hd = g.head_dim, kvdim = m->kvdim;
  if (!m->small_ok || nl < 1 || g.dim % 32 || g.hidden_dim % 32 || g.dim > 1024 ||
      g.hidden_dim > 4096 || hd > 64 || hd % 4 || g.n_heads % g.n_kv_heads ||
      m->qkv_rows != g.dim + 2 * kvdim)
    return PBX_OK;
  const int B = g.dim / 32, BH = g.hidden_dim / 32;
  for (int l = 0; l < nl; ++l) {
    const Layer &L = m->layers[l];
    const pbx_weight *w[4] = {L.wqkv, L.wo, L.wgu, L.wd};
    const int64_t rows[4] = {m->qkv_rows, g.dim, 2 * (int64_t)g.hidden_dim, g.dim};
    const int64_t blocks[4] = {B, B, B, BH};
    for (int k = 0; k < 4; ++k)
      if (w[k]->type != PBX_TYPE_Q8_0 || w[k]->N != rows[k] || w[k]->B != blocks[k]) return PBX_OK;
  }
  hipFunction_t f = pbx_kernel_by_name(c, "pbx_small_step_q8");
  if (!f) return PBX_OK;
  int G = 0, rq = 0, ro = 0, rg = 0, rd = 0;
  int g0 = std::max(32, (g.dim / 6 + 7) / 8 * 8);
  if (const char *e = getenv("PBX_SMALL_WGS")) g0 = std::max(8, atoi(e));
  for (int cand = g0; cand <= c->cu_count; cand += 8) {
    rq = 2 * ((m->qkv_rows + 2 * cand - 1) / (2 * cand));
    ro = (g.dim + cand - 1) / cand;
    rg = (g.hidden_dim + cand - 1) / cand;
    rd = (g.dim + cand - 1) / cand;
    // task slots a thread of 512: q|k|v 2, o 1, gate|up 4 (<= 256 rows), down 2
    if (cand >= g.n_heads && rq * B <= 1024 && ro * B <= 512 && 2 * rg * B <= 2048 &&
        2 * rg <= 256 && rd * BH <= 1024) {
      G = cand;
      break;
    }
  }
  if (!G) return PBX_OK;
  const long long stride = ((long long)m->qkv_rows + 3LL * g.dim + g.hidden_dim + 63) / 64 * 64;
  int rc;
  if (!m->small_layers) {
    std::vector<SmallLayerHost> tab(nl);
    for (int l = 0; l < nl; ++l) {
      const Layer &L = m->layers[l];
      tab[l] = SmallLayerHost{L.wqkv->qs, L.wo->qs, L.wgu->qs, L.wd->qs, L.wqkv->d, L.wo->d,
                              L.wgu->d,   L.wd->d, L.attn_norm, L.ffn_norm};
    }
    const size_t cb = (size_t)nl * stride * 8;
    if ((rc = dalloc(m, (void **)&m->small_layers, tab.size() * sizeof(SmallLayerHost))) ||
        (rc = dalloc(m, (void **)&m->small_cells, cb)) ||
        (rc = dalloc(m, (void **)&m->small_sync, 64)))
      return rc;
    // tag 0 (cleared cells) is never published; epoch 0, no workgroup done
    if (hipMemcpy(m->small_layers, tab.data(), tab.size() * sizeof(SmallLayerHost),
                  hipMemcpyHostToDevice) != hipSuccess ||
        hipMemsetAsync(m->small_cells, 0, cb, c->stream) != hipSuccess ||
        hipMemsetAsync(m->small_sync, 0, 64, c->stream) != hipSuccess)
      return pbx_fail(c, PBX_EHIP, "model: small-step set-up failed");
  }
  Op s;
  s.kind = ARG_SMALL;
  s.name = "pbx_small_step_q8";
  s.f = f;
  s.role = "layers";
  s.grid = dim3(G);
  s.block = dim3(512);
  SmallArgsHost &a = s.small;
  a.layers = m->small_layers;
  a.at = AttnArgsHost{nullptr, m->kcache, m->vcache, m->rope, nullptr, m->state, g.n_heads,
                      g.n_kv_heads, hd, (float)(1.0 / sqrt((double)hd)), g.max_seq};
  a.at.status = m->state + 3;
  a.at.spin = m->test_layer >= 0 ? m->test_spin : 0;
  a.layer_kv = (long long)g.max_seq * kvdim;
  a.cells = m->small_cells;
  a.cell_stride = stride;
  a.epoch = m->small_sync;
  a.done = reinterpret_cast<unsigned *>(m->small_sync + 1);
  a.x = m->x;
  a.n_layers = nl;
  a.dim = g.dim;
  a.hidden = g.hidden_dim;
  a.qkv_rows = m->qkv_rows;
  a.eps = g.rms_eps;
  a.rq = rq;
  a.ro = ro;
  a.rg = rg;
  a.rd = rd;
  a.test_layer = m->test_layer;
  a.skew = m->test_skew;
  // K and V of one cached position in every layer; every layer's weights,
  // norms and its cells (written once, read by every workgroup)
  s.bytes = 8.0 * kvdim * nl;
  for (int l = 0; l < nl; ++l) {
    const Layer &L = m->layers[l];
    for (const pbx_weight *w : {L.wqkv, L.wo, L.wgu, L.wd})
      s.fixed_bytes += (double)w->N * pbx_type_row_bytes(w->type, w->K);
    s.fixed_bytes += 8.0 * g.dim;
  }
  const size_t head = m->layer_op[nl];
  std::vector<Op> ops;
  ops.push_back(s);
  ops.insert(ops.end(), m->ops.begin() + head, m->ops.end());
  m->ops.swap(ops);
  for (int l = 0; l < nl; ++l) m->layer_op[l] = 0;
  m->layer_op[nl] = 1;
  m->small_step = true;
  return PBX_OK;
}

static int build_ops(pbx_model *m) {
  pbx_ctx *c = m->c;
  const pbx_model_config &g = m->cfg;
  m->ops.clear();
  m->layer_op.assign(g.n_layers + 1, 0);
  Op e;
  e.kind = ARG_EMBED;
  e.name = "pbx_embed";
  e.f = pbx_kernel_by_name(c, e.name);
  if (!e.f) return pbx_fail(c, PBX_ELOAD, "model: kernel pbx_embed not found");
  e.grid = dim3((g.dim + 255) / 256);
  e.block = dim3(256);
  e.role = "embed";
  e.bytes = (double)pbx_type_row_bytes(m->embd->type, g.dim) + 4.0 * g.dim;
  e.embed = EmbedArgsHost{m->embd->qs, m->embd->d, m->x, m->state, kernel_type(m->embd->type),
                          g.dim, g.vocab_size, m->embd->m};
  m->embed_op = e;
  hipFunction_t fattn = pbx_kernel_by_name(c, "pbx_attention_decode");
  hipFunction_t fhead = pbx_kernel_by_name(c, "pbx_attention_head");
  if (!fattn || !fhead) return pbx_fail(c, PBX_ELOAD, "model: attention kernels not found");
  hipFunction_t fsplit = pbx_kernel_by_name(c, "pbx_attention_split");
  hipFunction_t fcomb = pbx_kernel_by_name(c, "pbx_attention_combine");
  if (!fsplit || !fcomb)
    return pbx_fail(c, PBX_ELOAD, "model: split attention kernels not found");
  const size_t layer_kv = (size_t)g.max_seq * m->kvdim;
  // The head attention on the cache-complete layout when the q|k|v GEMV is
  // the integer-limb kernel with even row tiles: that kernel rotates q and
  // k and appends k and v (EPI_ROPE), the attention reads every position
  // from the cache.
  bool cached = false;
  if (m->attn_mode == ATTN_HEAD && g.head_dim % 2 == 0 && g.dim % 4 == 0 && m->kvdim % 4 == 0) {
    std::string shape;
    dim3 gr, bl;
    int nt;
    const pbx_weight *w0 = m->layers[0].wqkv;
    plan_gemv(c, m->gemv_int, "qkv", "qkv", w0->type, (int)w0->N, (int)w0->B, &shape, &gr, &bl, &nt);
    cached = shape == "i4x4b1";
  }
  hipFunction_t fheadc = pbx_kernel_by_name(c, "pbx_attention_head_c");
  if (cached && !fheadc) return pbx_fail(c, PBX_ELOAD, "model: kernel pbx_attention_head_c not found");
  // The o projection fused into the cached attention (pbx_attention_o_c<IPT>,
  // 256 * IPT output rows a workgroup): head_dim 64, Q4_0 o projection and
  // gate|up / down GEMVs whose planned shapes have the pending-update
  // variants (IPT from PBX_ATTN_O at model creation; 0 keeps the separate
  // o GEMV).
  int o_ipt = 0;
  hipFunction_t fattno = nullptr;
  // the q|k|v GEMV can join the launch: Q4_0 at K = 2048 in 32-row tiles
  // (16-row with IPT 1), a multiple of 8 tiles
  const bool qa_fit = m->qkv_attn && m->layers[0].wqkv->type == PBX_TYPE_Q4_0 &&
                      m->layers[0].wqkv->B == 64 && m->qkv_rows % 256 == 0;
  if (cached && g.head_dim == 64 && m->layers[0].wo->type == PBX_TYPE_Q4_0 &&
      m->layers[0].wo->B == 2 * g.n_heads) {
    const int ipt = m->attn_o_ipt >= 0 ? m->attn_o_ipt : qa_fit ? 2 : 1;
    if ((ipt == 1 || ipt == 2 || ipt == 4) && g.dim % (256 * ipt) == 0) {
      auto variant = [&](const pbx_weight *w, const char *plan_mode, const char *mode,
                         const char *role) {
        std::string shape;
        dim3 gr, bl;
        int nt;
        plan_gemv(c, m->gemv_int, plan_mode, role, w->type, (int)w->N, (int)w->B, &shape, &gr,
                  &bl, &nt);
        return pbx_kernel_by_name(c, std::string("pbx_dk_") + type_tag(w->type) + "_" + shape +
                                         "_" + mode) != nullptr;
      };
      fattno = pbx_kernel_by_name(c, "pbx_attention_o_c" + std::to_string(ipt));
      if (fattno && variant(m->layers[0].wgu, "gua", "gua", "gate_up") &&
          variant(m->layers[0].wd, "add", "adda", "down"))
        o_ipt = ipt;
    }
  }
  // The q|k|v GEMV and the attention + o projection in one launch
  // (pbx_qkvr_attn_o_r<RT>c<IPT>: IPT 1 with 16-row GEMV tiles, IPT 2 with
  // 32-row tiles).
  hipFunction_t fqa = nullptr;
  const size_t cell_stride = (size_t)m->qkv_rows + 64;
  const int qa_rows = o_ipt == 2 ? 32 : 16;
  const std::string qa_name = o_ipt == 2 ? "pbx_qkvr_attn_o_r8c2" : "pbx_qkvr_attn_o_r4c1";
  if ((o_ipt == 1 || o_ipt == 2) && qa_fit) fqa = pbx_kernel_by_name(c, qa_name);
  if (fqa && !m->qa_cells) {
    const size_t cb = (size_t)g.n_layers * cell_stride * 8;
    int rc = dalloc(m, (void **)&m->qa_cells, cb);
    if (rc) return rc;
    if (hipMemsetAsync(m->qa_cells, 0, cb, c->stream) != hipSuccess)
      return pbx_fail(c, PBX_EHIP, "model: clearing the q|k|v cells failed");
  }
  // The FFN in one launch (pbx_ffn_q4_d2048_h8192): Llama-3.2-1B's shapes
  // with Q4_0 layers, after the joined q|k|v + attention launch (whose epoch
  // and pending-update scheme it continues).
  hipFunction_t fffn = nullptr;
  // Its slices wait for each other's gate|up outputs, so all 256 workgroups
  // (one a CU) must be resident at once: only on parts with >= 256 CUs.
  if (fqa && m->ffn_join && c->cu_count >= 256 && g.dim == 2048 && g.hidden_dim == 8192 &&
      o_ipt == 2 &&
      m->layers[0].wgu->type == PBX_TYPE_Q4_0 && m->layers[0].wd->type == PBX_TYPE_Q4_0)
    fffn = pbx_kernel_by_name(c, "pbx_ffn_q4_d2048_h8192");
  const size_t h_stride = (size_t)g.hidden_dim + 64;
  if (fffn && !m->x2) {
    const size_t hb = (size_t)g.n_layers * h_stride * 8;
    int rc;
    if ((rc = dalloc(m, (void **)&m->x2, (size_t)g.dim * 4)) ||
        (rc = dalloc(m, (void **)&m->ffn_cell, (size_t)g.dim * 8)) ||
        (rc = dalloc(m, (void **)&m->h_cells, hb)))
      return rc;
    if (hipMemsetAsync(m->ffn_cell, 0, (size_t)g.dim * 8, c->stream) != hipSuccess ||
        hipMemsetAsync(m->h_cells, 0, hb, c->stream) != hipSuccess)
      return pbx_fail(c, PBX_EHIP, "model: clearing the FFN cells failed");
  }
  for (int l = 0; l < g.n_layers; ++l) {
    Layer &L = m->layers[l];
    int rc;
    m->layer_op[l] = m->ops.size();
    unsigned long long *cells = fqa ? m->qa_cells + l * cell_stride : nullptr;
    // joined FFN: layer l reads its residual row from x (even l) or x2 and
    // accumulates the attention's update in xacc[l % 2]
    const int par = fffn ? l & 1 : 0;
    float *xin = par ? m->x2 : m->x;
    long long *acc_l = m->xacc + (size_t)par * g.dim;
    if ((rc = add_gemv(m, L.wqkv, cached ? "qkvr" : "qkv", "qkv", xin, nullptr, L.attn_norm,
                       m->qkv, nullptr)))
      return rc;
    if (cached) {
      pbx_gemv_args &ga = m->ops.back().gemv;
      ga.state = m->state;
      ga.rope = m->rope;
      ga.kcache = m->kcache + l * layer_kv;
      ga.vcache = m->vcache + l * layer_kv;
      ga.qdim = g.dim;
      ga.kvdim = m->kvdim;
      ga.head_dim = g.head_dim;
    }
    Op a;
    a.role = "attn";
    a.bytes = 2.0 * 4.0 * m->kvdim;  // K and V of one cached position, all KV heads
    a.block = dim3(256);
    if (o_ipt) {
      a.kind = ARG_ATTN;
      a.name = "pbx_attention_o_c" + std::to_string(o_ipt);
      a.f = fattno;
      a.role = "attn_o";
      a.grid = dim3(g.n_heads * (g.dim / (256 * o_ipt)));
      a.block = dim3(512);
      a.attn = AttnArgsHost{m->qkv, m->kcache + l * layer_kv, m->vcache + l * layer_kv, m->rope,
                            m->attn, m->state, g.n_heads, g.n_kv_heads, g.head_dim,
                            (float)(1.0 / sqrt((double)g.head_dim)), g.max_seq};
      a.attn.oqs = L.wo->qs;
      a.attn.odsc = L.wo->d;
      a.attn.oacc = acc_l;
      a.attn.ox = xin;
      // the o projection's weights, its head outputs' update (read and written)
      a.fixed_bytes = (double)L.wo->N * pbx_type_row_bytes(L.wo->type, L.wo->K) + 16.0 * g.dim;
      if (cells) {
        // one launch: the q|k|v op's GEMV arguments, publishing into the
        // layer's cells, and these attention arguments reading them
        Op q = m->ops.back();
        m->ops.pop_back();
        a.kind = ARG_FUSED;
        a.name = qa_name;
        a.f = fqa;
        a.role = "qkv_attn_o";
        a.np = m->qkv_rows / qa_rows;
        a.grid = dim3(a.np + a.grid.x);
        a.gemv = q.gemv;
        a.gemv.xcell = cells;
        a.attn.cells = cells;
        a.attn.cell_n = m->qkv_rows;
        a.attn.qdim = g.dim;
        a.attn.status = m->state + 3;
        if (l == m->test_layer) {
          a.attn.skew = m->test_skew;
          a.attn.spin = m->test_spin;
        }
        if (fffn) {
          // the other pending update (the previous layer's, read by its FFN
          // launch) is cleared for the next layer; the FFN's cell epoch
          // advances (no FFN launch runs meanwhile)
          a.gemv.clr = m->xacc + (size_t)(1 - par) * g.dim;
          a.gemv.clr_n = g.dim;
          a.gemv.adv = m->h_cells + l * h_stride + g.hidden_dim;
        }
        a.fixed_bytes += q.bytes;
      }
      m->ops.push_back(a);
    } else if (cached) {
      a.kind = ARG_ATTN;
      a.name = "pbx_attention_head_c";
      a.f = fheadc;
      a.grid = dim3(g.n_heads);
      a.block = dim3(512);
      a.attn = AttnArgsHost{m->qkv, m->kcache + l * layer_kv, m->vcache + l * layer_kv, m->rope,
                            m->attn, m->state, g.n_heads, g.n_kv_heads, g.head_dim,
                            (float)(1.0 / sqrt((double)g.head_dim)), g.max_seq};
      m->ops.push_back(a);
    } else if (m->attn_mode == ATTN_HEAD) {
      a.kind = ARG_ATTN;
      a.name = "pbx_attention_head";
      a.f = fhead;
      a.grid = dim3(g.n_heads);
      a.block = dim3(512);
      a.attn = AttnArgsHost{m->qkv, m->kcache + l * layer_kv, m->vcache + l * layer_kv, m->rope,
                            m->attn, m->state, g.n_heads, g.n_kv_heads, g.head_dim,
                            (float)(1.0 / sqrt((double)g.head_dim)), g.max_seq};
      m->ops.push_back(a);
    } else if (m->attn_splits > 0) {
      a.kind = ARG_ATTN_SPLIT;
      a.name = "pbx_attention_split";
      a.f = fsplit;
      a.grid = dim3(g.n_kv_heads, m->attn_splits);
      a.block = dim3(64 * (g.n_heads / g.n_kv_heads));
      a.split = AttnSplitArgsHost{m->qkv, m->kcache + l * layer_kv, m->vcache + l * layer_kv,
                                  m->rope, m->attn, m->state, m->attn_part,
                                  g.n_heads, g.n_kv_heads, g.head_dim, m->attn_splits,
                                  (float)(1.0 / sqrt((double)g.head_dim))};
      m->ops.push_back(a);
      Op cb;  // merges the S partials of every head into m->attn
      cb.kind = ARG_COMBINE;
      cb.name = "pbx_attention_combine";
      cb.f = fcomb;
      cb.role = "attn_combine";
      cb.grid = dim3(g.n_heads);
      cb.block = dim3(64);
      cb.bytes = (double)g.n_heads * m->attn_splits * (g.head_dim + 2) * 4 + 4.0 * g.dim;
      cb.comb = CombineArgsHost{m->attn_part, m->attn, g.head_dim, m->attn_splits};
      m->ops.push_back(cb);
    } else {
      a.kind = ARG_ATTN;
      a.name = "pbx_attention_decode";
      a.f = fattn;
      a.grid = dim3(g.n_heads);
      a.attn = AttnArgsHost{m->qkv, m->kcache + l * layer_kv, m->vcache + l * layer_kv, m->rope,
                            m->attn, m->state, g.n_heads, g.n_kv_heads, g.head_dim,
                            (float)(1.0 / sqrt((double)g.head_dim)), g.max_seq};
      m->ops.push_back(a);
    }
    if (fffn) {
      // gate|up (the integer-limb GEMV with the pending update, publishing
      // its outputs) and the down slices in one launch
      if ((rc = add_gemv(m, L.wgu, "gua", "gate_up", xin, nullptr, L.ffn_norm, m->gu, nullptr)))
        return rc;
      Op f = m->ops.back();
      m->ops.pop_back();
      if (f.name != "pbx_dk_q4_i8x8b1w8p4_gua" || f.grid.x != 256 || f.block.x != 1024)
        return pbx_fail(c, PBX_ENOTSUP, "model: joined FFN needs the 8x8 gate|up shape, got %s",
                        f.name.c_str());
      f.kind = ARG_FFN;
      f.name = "pbx_ffn_q4_d2048_h8192";
      f.f = fffn;
      f.role = "ffn";
      f.gemv.acc = acc_l;
      f.gemv.xcell = m->h_cells + l * h_stride;
      f.ffn.qs = L.wd->qs;
      f.ffn.dsc = L.wd->d;
      f.ffn.x = xin;
      f.ffn.acc = acc_l;
      f.ffn.cell = m->ffn_cell;
      f.ffn.xout = par ? m->x : m->x2;
      f.ffn.qepoch = cells + m->qkv_rows;
      f.ffn.status = m->state + 3;
      // gate|up's bytes, then W_down, its input h (read as 8-byte cells, each
      // slice once) and the residual row: x, the update, the next row
      f.bytes += (double)L.wd->N * pbx_type_row_bytes(L.wd->type, L.wd->K) +
                 8.0 * g.hidden_dim + 16.0 * g.dim;
      m->ops.push_back(f);
      continue;
    }
    if (o_ipt) {
      if ((rc = add_gemv(m, L.wgu, "gua", "gate_up", m->x, nullptr, L.ffn_norm, m->gu, nullptr)))
        return rc;
      m->ops.back().gemv.acc = m->xacc;
      if ((rc = add_gemv(m, L.wd, "adda", "down", m->gu, nullptr, nullptr, m->x, nullptr)))
        return rc;
      m->ops.back().gemv.acc = m->xacc;
      if (cells) m->ops.back().gemv.xcell = cells + m->qkv_rows;  // advances the epoch
      continue;
    }
    if ((rc = add_gemv(m, L.wo, "add", "o", m->attn, nullptr, nullptr, m->x, nullptr))) return rc;
    if ((rc = add_gemv(m, L.wgu, "gu", "gate_up", m->x, nullptr, L.ffn_norm, m->gu, nullptr))) return rc;
    if ((rc = add_gemv(m, L.wd, "add", "down", m->gu, nullptr, nullptr, m->x, nullptr))) return rc;
  }
  int n_tiles = 0;
  const pbx_weight *head = m->output ? m->output : m->embd;
  m->layer_op[g.n_layers] = m->ops.size();
  int rc = add_gemv(m, head, "lmh", "lm_head", fffn && (g.n_layers & 1) ? m->x2 : m->x, nullptr,
                    m->out_norm, m->logits, &n_tiles);
  if (rc) return rc;
  if (m->ops.back().name.rfind("pbx_dk_q6k_i", 0) == 0) {
    // Q6_K head on the integer-limb kernel: the same kernel on the
    // lane-packed copy (one 16-, 8- and 2-byte load per lane block)
    Op &op = m->ops.back();
    if (!m->head_lanes &&
        ((rc = dalloc(m, &m->head_lanes, (size_t)head->N * head->B * 26)) ||
         (rc = pack_head_lanes(m))))
      return rc;
    op.name.replace(0, strlen("pbx_dk_q6k_"), "pbx_dk_q6kp_");
    op.f = pbx_kernel_by_name(c, op.name);
    if (!op.f) return pbx_fail(c, PBX_ELOAD, "model: kernel %s not found", op.name.c_str());
    op.gemv.qs = m->head_lanes;
  }
  if (n_tiles > m->n_partials_cap)
    return pbx_fail(c, PBX_EINVAL, "model: %d argmax partials exceed capacity %d", n_tiles,
                    m->n_partials_cap);
  Op am;
  am.kind = ARG_ARGMAX;
  am.name = "pbx_argmax_final";
  am.f = pbx_kernel_by_name(c, am.name);
  if (!am.f) return pbx_fail(c, PBX_ELOAD, "model: kernel pbx_argmax_final not found");
  am.grid = dim3(1);
  am.block = dim3(1024);
  am.role = "argmax";  // + the next step's embedding
  am.bytes = 8.0 * n_tiles;
  am.amax = ArgmaxArgsHost{m->partials, m->state, m->hist, n_tiles, m->hist_cap, e.embed};
  if (fffn) {
    am.amax.clr = m->xacc;  // both pending updates zero at the next step's start
    am.amax.clr_n = 2 * g.dim;
  }
  m->ffn_joined = fffn != nullptr;
  am.bytes += (double)pbx_type_row_bytes(m->embd->type, g.dim) + 4.0 * g.dim;
  m->ops.push_back(am);
  if ((rc = plan_small_step(m))) return rc;
  m->ops_ready = true;
  return PBX_OK;
}

// Launches op on the model's stream; with t0 / t1, the kernel's own
// dispatch stamps them (its execution time, for measurement).
static int enqueue_op(pbx_model *m, Op &op, hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr) {
  void *arg;
  void *comb[] = {&op.comb.part, &op.comb.out, &op.comb.head_dim, &op.comb.S};
  switch (op.kind) {
    case ARG_GEMV: arg = &op.gemv; break;
    case ARG_ATTN: arg = &op.attn; break;
    case ARG_ATTN_SPLIT: arg = &op.split; break;
    case ARG_EMBED: arg = &op.embed; break;
    case ARG_SMALL: arg = &op.small; break;
    default: arg = &op.amax; break;
  }
  void *one[] = {arg};
  void *fused[] = {&op.gemv, &op.attn, &op.np};
  void *ffn[] = {&op.gemv, &op.ffn};
  void **args = op.kind == ARG_COMBINE ? comb
                : op.kind == ARG_FUSED ? fused
                : op.kind == ARG_FFN   ? ffn
                                       : one;
  if (t0)
    return pbx_launch_fn_timed(m->c, op.f, op.name.c_str(), op.grid, op.block, args, m->c->stream,
                               t0, t1);
  return pbx_launch_fn(m->c, op.f, op.name.c_str(), op.grid, op.block, args, m->c->stream);
}

static void drop_graph(pbx_model *m) {
  if (m->exec) hipGraphExecDestroy(m->exec);
  if (m->graph) hipGraphDestroy(m->graph);
  m->exec = nullptr;
  m->graph = nullptr;
  m->graph_tried = m->graph_ok = false;
  if (m->exec_k) hipGraphExecDestroy(m->exec_k);
  if (m->graph_k) hipGraphDestroy(m->graph_k);
  if (m->exec_k4) hipGraphExecDestroy(m->exec_k4);
  if (m->graph_k4) hipGraphDestroy(m->graph_k4);
  m->exec_k = m->exec_k4 = nullptr;
  m->graph_k = m->graph_k4 = nullptr;
  m->graph_k_tried = m->graph_k_ok = m->graph_k4_tried = m->graph_k4_ok = false;
  for (auto &p : m->part) {
    if (p.exec) hipGraphExecDestroy(p.exec);
    if (p.graph) hipGraphDestroy(p.graph);
  }
  m->part.clear();
}

static bool use_graphs() {
  const char *e = getenv("PBX_GRAPHS");
  return !(e && e[0] == '0');
}

// The kernels of a step that runs the first L layers: ops [0, layer_op[L])
// then the LM head and the argmax.
static int enqueue_ops_layers(pbx_model *m, int L) {
  const size_t stop = m->layer_op[L], head = m->layer_op[m->cfg.n_layers];
  if (m->small_step) {
    // ops[0] runs the layers (the first L of them), then the head's ops
    int rc = PBX_OK;
    if (L > 0) {
      Op s = m->ops[0];
      s.small.n_layers = L;
      rc = enqueue_op(m, s);
    }
    for (size_t i = 1; i < m->ops.size() && !rc; ++i) rc = enqueue_op(m, m->ops[i]);
    return rc;
  }
  for (size_t i = 0; i < m->ops.size(); ++i) {
    if (i >= stop && i < head) continue;
    int rc;
    if (i == head && m->ffn_joined && L < m->cfg.n_layers) {
      // the joined FFN alternates the residual rows: after L layers the
      // head reads x (L even) or x2
      Op h = m->ops[i];
      h.gemv.X = (L & 1) ? m->x2 : m->x;
      rc = enqueue_op(m, h);
    } else {
      rc = enqueue_op(m, m->ops[i]);
    }
    if (rc) return rc;
  }
  return PBX_OK;
}

// Captures the step of the first L layers into a graph (false: capture
// failed, the caller launches kernel by kernel).
static bool capture_step(pbx_model *m, int L, hipGraph_t *graph, hipGraphExec_t *exec,
                         int steps = 1) {
  bool ok = false;
  hipStream_t s = m->c->stream;
  if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) == hipSuccess) {
    int rc = PBX_OK;
    for (int i = 0; i < steps && !rc; ++i) rc = enqueue_ops_layers(m, L);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (!rc && e == hipSuccess && g && hipGraphInstantiate(exec, g, nullptr, nullptr, 0) == hipSuccess) {
      *graph = g;
      ok = true;
      // the executable's one-time device set-up now, not in its first launch
      (void)hipGraphUpload(*exec, s);
    } else if (g) {
      hipGraphDestroy(g);
    }
  }
  (void)hipGetLastError();
  return ok;
}

// One decode step through the first L layers (L = n_layers: the whole
// step) on the context's stream: graph replay when capture worked.
static int run_step_layers(pbx_model *m, int L) {
  if (!m->ops_ready) {
    int rc = build_ops(m);
    if (rc) return rc;
  }
  const int nl = m->cfg.n_layers;
  bool *tried = &m->graph_tried, *ok = &m->graph_ok;
  hipGraph_t *graph = &m->graph;
  hipGraphExec_t *exec = &m->exec;
  if (L < nl) {
    if ((int)m->part.size() < nl) m->part.resize(nl);
    auto &p = m->part[L];
    tried = &p.tried;
    ok = &p.ok;
    graph = &p.graph;
    exec = &p.exec;
  }
  if (use_graphs() && !*tried) {
    *tried = true;
    *ok = capture_step(m, L, graph, exec);
  }
  if (*ok) {
    if (hipGraphLaunch(*exec, m->c->stream) != hipSuccess)
      return pbx_fail(m->c, PBX_EHIP, "model: hipGraphLaunch failed");
    return PBX_OK;
  }
  return enqueue_ops_layers(m, L);
}

static int run_step(pbx_model *m) { return run_step_layers(m, m->cfg.n_layers); }

// Up to `left` whole decode steps: graph_steps of them in one graph launch
// when that graph is available, else 4 in one launch, else one step.
// *done: the steps enqueued.
static int run_steps(pbx_model *m, int left, int *done) {
  *done = 1;
  struct Multi {
    int steps;
    hipGraph_t *graph;
    hipGraphExec_t *exec;
    bool *tried, *ok;
  } multi[2] = {
      {m->graph_steps, &m->graph_k, &m->exec_k, &m->graph_k_tried, &m->graph_k_ok},
      {4, &m->graph_k4, &m->exec_k4, &m->graph_k4_tried, &m->graph_k4_ok}};
  for (int i = 0; i < 2; ++i) {
    const Multi &g = multi[i];
    if (g.steps <= 1 || left < g.steps || !use_graphs() || (i == 1 && m->graph_steps <= 4))
      continue;
    if (!m->ops_ready) {
      int rc = build_ops(m);
      if (rc) return rc;
    }
    if (!*g.tried) {
      *g.tried = true;
      *g.ok = capture_step(m, m->cfg.n_layers, g.graph, g.exec, g.steps);
    }
    if (*g.ok) {
      if (hipGraphLaunch(*g.exec, m->c->stream) != hipSuccess)
        return pbx_fail(m->c, PBX_EHIP, "model: hipGraphLaunch failed");
      *done = g.steps;
      return PBX_OK;
    }
  }
  return run_step(m);
}

// Device state for a host-driven step; with `embed`, also the token's
// embedding row into x (a step's argmax embeds the token it picks).
static int set_state(pbx_model *m, int pos, int token, int step, bool embed) {
  hipFunction_t f = pbx_kernel_by_name(m->c, "pbx_set_state");
  if (!f) return pbx_fail(m->c, PBX_ELOAD, "model: kernel pbx_set_state not found");
  int *st = m->state;
  void *args[] = {&st, &pos, &token, &step};
  int rc = pbx_launch_fn(m->c, f, "pbx_set_state", dim3(1), dim3(64), args, m->c->stream);
  if (rc || !embed) return rc;
  if (!m->ops_ready && (rc = build_ops(m))) return rc;
  return enqueue_op(m, m->embed_op);
}

static int kv_fill(pbx_model *m, int from) {
  hipFunction_t f = pbx_kernel_by_name(m->c, "pbx_kv_fill");
  if (!f) return pbx_fail(m->c, PBX_ELOAD, "model: kernel pbx_kv_fill not found");
  int64_t stride = (int64_t)m->cfg.max_seq * m->kvdim;
  int64_t off = (int64_t)from * m->kvdim;
  int64_t count = stride - off;
  int nl = m->cfg.n_layers;
  if (count <= 0) return PBX_OK;
  float *k = m->kcache, *v = m->vcache;
  void *args[] = {&k, &v, &stride, &off, &count, &nl};
  const int64_t total = count * nl;
  return pbx_launch_fn(m->c, f, "pbx_kv_fill", dim3((unsigned)((total + 255) / 256)), dim3(256),
                       args, m->c->stream);
}

// After a call's work has been synchronised: st is the device state copied
// with it.  A bounded device-side wait that gave up (a hand-off between the
// workgroups of a launch whose data never arrived) marks the status word;
// its results are then NaN, so the call fails with PBX_ETIMEOUT instead of
// returning them.  The word is cleared for the next call.
static int check_status(pbx_model *m, const int *st, const char *who) {
  if (!st[3]) return PBX_OK;
  if (hipMemsetAsync(m->state + 3, 0, 4, m->c->stream) != hipSuccess ||
      hipStreamSynchronize(m->c->stream) != hipSuccess)
    return pbx_fail(m->c, PBX_EHIP, "%s: clearing the device status failed", who);
  return pbx_fail(m->c, PBX_ETIMEOUT,
                  "%s: a device-side wait for data published inside a launch gave up "
                  "(status 0x%x); the results of this call are invalid",
                  who, (unsigned)st[3]);
}

// Captures every step graph pbx_model_generate replays (one step, the
// multi-step graph and the 4-step one), so that no capture happens inside
// a timed or latency-sensitive generate call.
static int prepare_graphs(pbx_model *m) {
  if (!use_graphs()) return PBX_OK;
  if (!m->ops_ready) {
    int rc = build_ops(m);
    if (rc) return rc;
  }
  const int nl = m->cfg.n_layers;
  if (!m->graph_tried) {
    m->graph_tried = true;
    m->graph_ok = capture_step(m, nl, &m->graph, &m->exec);
  }
  if (m->graph_steps > 1 && !m->graph_k_tried) {
    m->graph_k_tried = true;
    m->graph_k_ok = capture_step(m, nl, &m->graph_k, &m->exec_k, m->graph_steps);
  }
  if (m->graph_steps > 4 && !m->graph_k4_tried) {
    m->graph_k4_tried = true;
    m->graph_k4_ok = capture_step(m, nl, &m->graph_k4, &m->exec_k4, 4);
  }
  return PBX_OK;
}

static int dalloc(pbx_model *m, void **p, size_t bytes) {
  if (hipMalloc(p, bytes) != hipSuccess) {
    *p = nullptr;
    return pbx_fail(m->c, PBX_ENOMEM, "model: hipMalloc(%zu) failed", bytes);
  }
  m->bytes += bytes;
  return PBX_OK;
}

static void model_release(pbx_model *m) {
  if (!m) return;
  drop_graph(m);
  for (Layer &L : m->layers) {
    pbx_weight_release(L.wqkv);
    pbx_weight_release(L.wo);
    pbx_weight_release(L.wgu);
    pbx_weight_release(L.wd);
    if (L.attn_norm) hipFree(L.attn_norm);
    if (L.ffn_norm) hipFree(L.ffn_norm);
  }
  pbx_weight_release(m->embd);
  pbx_weight_release(m->output);
  if (m->tok_ev) hipEventSynchronize(m->tok_ev);
  if (m->h_tok) hipHostFree(m->h_tok);
  if (m->h_next) hipHostFree(m->h_next);
  if (m->tok_ev) hipEventDestroy(m->tok_ev);
  for (void *p : {(void *)m->out_norm, (void *)m->kcache, (void *)m->vcache, (void *)m->rope,
                  (void *)m->x, (void *)m->xacc, (void *)m->qkv, (void *)m->attn, (void *)m->gu,
                  (void *)m->logits,
                  (void *)m->partials, (void *)m->state, (void *)m->hist,
                  (void *)m->attn_part, m->head_lanes, (void *)m->qa_cells, (void *)m->x2,
                  (void *)m->ffn_cell, (void *)m->h_cells, (void *)m->small_layers,
                  (void *)m->small_cells, (void *)m->small_sync})
    if (p) hipFree(p);
  for (void *p : {(void *)m->bx, (void *)m->bxn, (void *)m->bqkv, (void *)m->battn,
                  (void *)m->bgu, (void *)m->bh, (void *)m->btmp, (void *)m->blogits,
                  (void *)m->bnext, (void *)m->bkeys, (void *)m->mr_cell,
                  m->g16, m->g16lo,
                  (void *)m->ginv, (void *)m->gpart})
    if (p) hipFree(p);
  m->magic = 0;
  delete m;
}

void pbx_model_release_all(pbx_ctx *c) {
  auto *list = (std::vector<pbx_model *> *)c->models;
  if (!list) return;
  for (pbx_model *m : *list) model_release(m);
  delete list;
  c->models = nullptr;
}

// Decode attention kernel: "head" (pbx_attention_head, one workgroup per
// query head with in-workgroup position splits; head_dim <= 64), "split"
// (pbx_attention_split + pbx_attention_combine; head_dim <= 128) or
// "decode" (pbx_attention_decode).  The default is the first that applies;
// PBX_ATTENTION=split|decode at model creation forces one (and the older
// PBX_SPLIT_ATTENTION=0 selects "decode").
static AttnMode attention_mode(const pbx_model_config &g) {
  const bool split_ok = g.head_dim <= 128 && g.n_heads / g.n_kv_heads <= 16;
  const char *e = getenv("PBX_ATTENTION");
  const char *legacy = getenv("PBX_SPLIT_ATTENTION");
  if (legacy && legacy[0] == '0') return ATTN_DECODE;
  if (e && strcmp(e, "decode") == 0) return ATTN_DECODE;
  if (e && strcmp(e, "split") == 0) return split_ok ? ATTN_SPLIT : ATTN_DECODE;
  if (g.head_dim <= 64) return ATTN_HEAD;
  return split_ok ? ATTN_SPLIT : ATTN_DECODE;
}

static bool is_weight_type(int t) {
  return t == PBX_TYPE_Q4_0 || t == PBX_TYPE_Q4_1 || t == PBX_TYPE_Q8_0 || t == PBX_TYPE_F32 ||
         t == PBX_TYPE_F16 || t == PBX_TYPE_Q6_K;
}

extern "C" int pbx_model_create(pbx_ctx *c, const pbx_model_config *cfg, pbx_model **out) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_create: ctx is NULL");
  if (!cfg || !out) return pbx_fail(c, PBX_EINVAL, "pbx_model_create: NULL argument");
  *out = nullptr;
  const pbx_model_config &g = *cfg;
  if (g.dim <= 0 || g.hidden_dim <= 0 || g.n_layers <= 0 || g.n_heads <= 0 ||
      g.n_kv_heads <= 0 || g.head_dim <= 0 || g.vocab_size <= 0 || g.max_seq <= 0)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_create: every size must be positive");
  if (g.dim % 32 || g.hidden_dim % 32)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_create: dim and hidden_dim must be multiples of 32");
  if (g.n_heads * g.head_dim != g.dim || g.n_heads % g.n_kv_heads)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_model_create: need n_heads*head_dim == dim and n_kv_heads | n_heads");
  if (g.head_dim % 4 || g.head_dim < 32 || g.head_dim > 256)
    return pbx_fail(c, PBX_ENOTSUP, "pbx_model_create: head_dim %d unsupported (32..256, %%4)",
                    g.head_dim);
  if (g.max_seq > 8192)
    return pbx_fail(c, PBX_ENOTSUP, "pbx_model_create: max_seq %d > 8192", g.max_seq);
  if (!is_weight_type(g.weight_type) || !is_weight_type(g.embed_type) ||
      (g.output_type >= 0 && !is_weight_type(g.output_type)))
    return pbx_fail(c, PBX_EINVAL, "pbx_model_create: unsupported weight type");
  if (g.rope_theta <= 0 || !(g.rms_eps >= 0))
    return pbx_fail(c, PBX_EINVAL, "pbx_model_create: bad rope_theta / rms_eps");
  if (hipSetDevice(c->device) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_create: hipSetDevice failed");

  pbx_model *m = new pbx_model();
  m->magic = PBX_MODEL_MAGIC;
  m->c = c;
  m->cfg = g;
  m->kvdim = g.n_kv_heads * g.head_dim;
  m->qkv_rows = g.dim + 2 * m->kvdim;
  m->gemv_int = !int_gemv_disabled();
  m->layers.resize(g.n_layers);
  int rc = PBX_OK;
  for (int l = 0; l < g.n_layers && !rc; ++l) {
    Layer &L = m->layers[l];
    if (!rc) rc = pbx_weight_alloc(c, g.weight_type, m->qkv_rows, g.dim, &L.wqkv);
    if (!rc) rc = pbx_weight_alloc(c, g.weight_type, g.dim, g.dim, &L.wo);
    if (!rc) rc = pbx_weight_alloc(c, g.weight_type, 2 * (int64_t)g.hidden_dim, g.dim, &L.wgu);
    if (!rc) rc = pbx_weight_alloc(c, g.weight_type, g.dim, g.hidden_dim, &L.wd);
    if (!rc) rc = dalloc(m, (void **)&L.attn_norm, (size_t)g.dim * 4);
    if (!rc) rc = dalloc(m, (void **)&L.ffn_norm, (size_t)g.dim * 4);
    if (!rc)
      m->bytes += L.wqkv->bytes + L.wo->bytes + L.wgu->bytes + L.wd->bytes;
  }
  if (!rc) rc = pbx_weight_alloc(c, g.embed_type, g.vocab_size, g.dim, &m->embd);
  if (!rc) m->bytes += m->embd->bytes;
  if (!rc && g.output_type >= 0) {
    rc = pbx_weight_alloc(c, g.output_type, g.vocab_size, g.dim, &m->output);
    if (!rc) m->bytes += m->output->bytes;
  }
  const size_t kv_bytes = (size_t)g.n_layers * g.max_seq * m->kvdim * 4;
  if (!rc) rc = dalloc(m, (void **)&m->out_norm, (size_t)g.dim * 4);
  if (!rc) rc = dalloc(m, (void **)&m->kcache, kv_bytes);
  if (!rc) rc = dalloc(m, (void **)&m->vcache, kv_bytes);
  if (!rc) rc = dalloc(m, (void **)&m->rope, (size_t)g.max_seq * g.head_dim * 4);
  if (!rc) rc = dalloc(m, (void **)&m->x, (size_t)g.dim * 4);
  if (!rc) rc = dalloc(m, (void **)&m->xacc, (size_t)g.dim * 16);
  if (!rc && hipMemsetAsync(m->xacc, 0, (size_t)g.dim * 16, c->stream) != hipSuccess)
    rc = pbx_fail(c, PBX_EHIP, "pbx_model_create: clearing the pending update failed");
  if (!rc) rc = dalloc(m, (void **)&m->qkv, (size_t)m->qkv_rows * 4);
  if (!rc) rc = dalloc(m, (void **)&m->attn, (size_t)g.dim * 4);
  if (!rc) rc = dalloc(m, (void **)&m->gu, (size_t)g.hidden_dim * 2 * 4);
  if (!rc) rc = dalloc(m, (void **)&m->logits, (size_t)g.vocab_size * 4);
  m->n_partials_cap = g.vocab_size + 256;  // at most one tile per row (+ small-kernel slack)
  if (!rc) rc = dalloc(m, (void **)&m->partials, (size_t)m->n_partials_cap * 8);
  if (!rc) rc = dalloc(m, (void **)&m->state, 64);
  if (!rc && hipMemsetAsync(m->state, 0, 64, c->stream) != hipSuccess)
    rc = pbx_fail(c, PBX_EHIP, "pbx_model_create: clearing the device state failed");
  m->hist_cap = g.max_seq;
  if (!rc) rc = dalloc(m, (void **)&m->hist, (size_t)m->hist_cap * 4);
  // Split-position attention when its tiles fit (head_dim <= 128, <= 16
  // query heads per KV head): about 256 workgroups per layer, at most 64
  // splits, never more splits than positions.
  m->attn_mode = attention_mode(g);
  if (const char *e = getenv("PBX_QKV_ATTN")) m->qkv_attn = e[0] != '0';
  if (const char *e = getenv("PBX_ATTN_O")) m->attn_o_ipt = atoi(e);
  if (const char *e = getenv("PBX_GRAPH_STEPS")) m->graph_steps = atoi(e);
  if (const char *e = getenv("PBX_FFN")) m->ffn_join = e[0] != '0';
  if (const char *e = getenv("PBX_SMALL_STEP")) m->small_ok = e[0] != '0';
  if (!rc && m->attn_mode == ATTN_SPLIT) {
    m->attn_splits = std::min({64, g.max_seq, std::max(4, (256 + g.n_kv_heads - 1) / g.n_kv_heads)});
    rc = dalloc(m, (void **)&m->attn_part,
                (size_t)g.n_heads * m->attn_splits * (g.head_dim + 2) * 4);
  }
  if (!rc) {
    // RoPE table, llama.js:163-190: pair i of a head rotates by
    // pos / theta^(2i/head_dim), evaluated in double as the reference does.
    std::vector<float> tab((size_t)g.max_seq * g.head_dim);
    for (int p = 0; p < g.max_seq; ++p)
      for (int i = 0; i < g.head_dim; i += 2) {
        const double freq = 1.0 / pow(g.rope_theta, (double)i / g.head_dim);
        const double ang = p * freq;
        tab[(size_t)p * g.head_dim + i] = (float)cos(ang);
        tab[(size_t)p * g.head_dim + i + 1] = (float)sin(ang);
      }
    if (hipMemcpy(m->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemsetAsync(m->kcache, 0, kv_bytes, c->stream) != hipSuccess ||
        hipMemsetAsync(m->vcache, 0, kv_bytes, c->stream) != hipSuccess ||
        hipMemsetAsync(m->state, 0, 64, c->stream) != hipSuccess ||
        hipMemsetAsync(m->xacc, 0, (size_t)g.dim * 16, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
      rc = pbx_fail(c, PBX_EHIP, "pbx_model_create: initialisation copies failed");
  }
  if (rc) {
    hipStreamSynchronize(c->stream);
    model_release(m);
    return rc;
  }
  auto *list = (std::vector<pbx_model *> *)c->models;
  if (!list) c->models = list = new std::vector<pbx_model *>();
  list->push_back(m);
  *out = m;
  return PBX_OK;
}

extern "C" int pbx_model_free(pbx_model *m) {
  if (!m) return PBX_OK;
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_free: not a live model");
  pbx_ctx *c = m->c;
  hipStreamSynchronize(c->stream);
  auto *list = (std::vector<pbx_model *> *)c->models;
  if (list) list->erase(std::remove(list->begin(), list->end(), m), list->end());
  model_release(m);
  return PBX_OK;
}

static size_t expect_bytes(int type, int64_t N, int64_t K) {
  return (size_t)N * pbx_type_row_bytes(type, K);
}

extern "C" int pbx_model_set_tensor(pbx_model *m, int tensor, int layer, const void *data,
                                    size_t nbytes) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_set_tensor: not a live model");
  pbx_ctx *c = m->c;
  const pbx_model_config &g = m->cfg;
  if (!data) return pbx_fail(c, PBX_EINVAL, "pbx_model_set_tensor: data is NULL");
  if (hipSetDevice(c->device) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_set_tensor: hipSetDevice failed");
  const bool per_layer = tensor >= PBX_T_ATTN_NORM;
  if (per_layer && (layer < 0 || layer >= g.n_layers))
    return pbx_fail(c, PBX_EINVAL, "pbx_model_set_tensor: layer %d out of range [0, %d)", layer,
                    g.n_layers);
  auto copy_f32 = [&](float *dst, int64_t n) -> int {
    if (nbytes < (size_t)n * 4)
      return pbx_fail(c, PBX_EINVAL, "pbx_model_set_tensor: %zu bytes, tensor %d needs %lld",
                      nbytes, tensor, (long long)n * 4);
    if (hipMemcpy(dst, data, (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess)
      return pbx_fail(c, PBX_EHIP, "pbx_model_set_tensor: copy failed");
    return PBX_OK;
  };
  auto rows = [&](pbx_weight *w, int64_t row0, int64_t n) -> int {
    const size_t need = expect_bytes(w->type, n, w->K);
    if (nbytes < need)
      return pbx_fail(c, PBX_EINVAL, "pbx_model_set_tensor: %zu bytes, tensor %d needs %zu",
                      nbytes, tensor, need);
    return pbx_weight_write_rows(c, w, row0, n, data);
  };
  int rc;
  unsigned bit = 1u << tensor;
  switch (tensor) {
    case PBX_T_TOKEN_EMBD: rc = rows(m->embd, 0, g.vocab_size); break;
    case PBX_T_OUTPUT:
      if (!m->output)
        return pbx_fail(c, PBX_EINVAL, "pbx_model_set_tensor: LM head is tied to token_embd");
      rc = rows(m->output, 0, g.vocab_size);
      break;
    case PBX_T_OUTPUT_NORM: rc = copy_f32(m->out_norm, g.dim); break;
    case PBX_T_ATTN_NORM: rc = copy_f32(m->layers[layer].attn_norm, g.dim); break;
    case PBX_T_FFN_NORM: rc = copy_f32(m->layers[layer].ffn_norm, g.dim); break;
    case PBX_T_ATTN_Q: rc = rows(m->layers[layer].wqkv, 0, g.dim); break;
    case PBX_T_ATTN_K: rc = rows(m->layers[layer].wqkv, g.dim, m->kvdim); break;
    case PBX_T_ATTN_V: rc = rows(m->layers[layer].wqkv, g.dim + m->kvdim, m->kvdim); break;
    case PBX_T_ATTN_OUTPUT: rc = rows(m->layers[layer].wo, 0, g.dim); break;
    case PBX_T_FFN_GATE: rc = rows(m->layers[layer].wgu, 0, g.hidden_dim); break;
    case PBX_T_FFN_UP: rc = rows(m->layers[layer].wgu, g.hidden_dim, g.hidden_dim); break;
    case PBX_T_FFN_DOWN: rc = rows(m->layers[layer].wd, 0, g.dim); break;
    default:
      return pbx_fail(c, PBX_EINVAL, "pbx_model_set_tensor: unknown tensor id %d", tensor);
  }
  if (rc) return rc;
  // a rewritten LM head: refresh its lane-packed copy
  if (m->head_lanes && tensor == (m->output ? PBX_T_OUTPUT : PBX_T_TOKEN_EMBD) &&
      (rc = pack_head_lanes(m)))
    return rc;
  if (per_layer)
    m->layers[layer].set_mask |= bit;
  else
    m->global_mask |= bit;
  return PBX_OK;
}

static int check_complete(pbx_model *m) {
  const unsigned layer_all = (1u << PBX_T_ATTN_NORM) | (1u << PBX_T_FFN_NORM) |
                             (1u << PBX_T_ATTN_Q) | (1u << PBX_T_ATTN_K) | (1u << PBX_T_ATTN_V) |
                             (1u << PBX_T_ATTN_OUTPUT) | (1u << PBX_T_FFN_GATE) |
                             (1u << PBX_T_FFN_UP) | (1u << PBX_T_FFN_DOWN);
  unsigned global_all = (1u << PBX_T_TOKEN_EMBD) | (1u << PBX_T_OUTPUT_NORM);
  if (m->output) global_all |= 1u << PBX_T_OUTPUT;
  if ((m->global_mask & global_all) != global_all)
    return pbx_fail(m->c, PBX_EINVAL, "model: token_embd/output_norm%s not set",
                    m->output ? "/output" : "");
  for (int l = 0; l < m->cfg.n_layers; ++l)
    if ((m->layers[l].set_mask & layer_all) != layer_all)
      return pbx_fail(m->c, PBX_EINVAL, "model: layer %d is missing tensors (mask 0x%x)", l,
                      m->layers[l].set_mask);
  return PBX_OK;
}

// ---------------------------------------------------------------------------
// Row-batched forward: llama.js:204-371 with seqLen = n > 1.  Every linear
// takes all n rows at once (the MFMA GEMM for Q4_0/Q8_0, the multi-row GEMV
// for f32), so each weight is read once per forward instead of once per
// token.  The KV rows of all n positions are appended before attention, and
// attention row t sees positions 0..start+t (the causal mask of
// llama.js:274-286).
// ---------------------------------------------------------------------------

static int grow(pbx_model *m, void **p, size_t bytes) {
  if (*p) {
    hipStreamSynchronize(m->c->stream);
    hipFree(*p);
    *p = nullptr;
  }
  if (hipMalloc(p, bytes) != hipSuccess) {
    *p = nullptr;
    return pbx_fail(m->c, PBX_ENOMEM, "model: hipMalloc(%zu) for the batch failed", bytes);
  }
  return PBX_OK;
}

#define MR_MAX 5
#define MR_XS 15  // K slices of the split rows GEMV at most (4-bit counts)

static int ensure_batch(pbx_model *m, int rows, bool all_logits) {
  const pbx_model_config &g = m->cfg;
  int rc = PBX_OK;
  if (!m->mr_cell) {
    if ((rc = grow(m, (void **)&m->mr_cell, (size_t)MR_MAX * g.dim * 8))) return rc;
    if (hipMemsetAsync(m->mr_cell, 0, (size_t)MR_MAX * g.dim * 8, m->c->stream) != hipSuccess)
      return pbx_fail(m->c, PBX_EHIP, "model: clearing the split cells failed");
  }
  if (rows > m->batch_cap) {
    const size_t R = (size_t)rows;
    const size_t tmp_cols = std::max({(size_t)g.dim, (size_t)m->qkv_rows, 2 * (size_t)g.hidden_dim});
    if (!rc) rc = grow(m, (void **)&m->bx, R * g.dim * 4);
    if (!rc) rc = grow(m, (void **)&m->bxn, R * g.dim * 4);
    if (!rc) rc = grow(m, (void **)&m->bqkv, R * m->qkv_rows * 4);
    if (!rc) rc = grow(m, (void **)&m->battn, R * g.dim * 4);
    if (!rc) rc = grow(m, (void **)&m->bgu, R * 2 * g.hidden_dim * 4);
    if (!rc) rc = grow(m, (void **)&m->bh, R * g.hidden_dim * 4);
    // accumulating linears without an MFMA path go through a temporary
    if (!rc) rc = grow(m, (void **)&m->btmp, R * tmp_cols * 4);
    if (!rc) rc = grow(m, (void **)&m->bnext, R * 4);
    if (!rc && !m->tok_ev && hipEventCreateWithFlags(&m->tok_ev, hipEventDisableTiming) != hipSuccess)
      rc = pbx_fail(m->c, PBX_EHIP, "model: event creation failed");
    if (!rc) {
      hipEventSynchronize(m->tok_ev);
      if (m->h_tok) hipHostFree(m->h_tok);
      if (m->h_next) hipHostFree(m->h_next);
      m->h_tok = m->h_next = nullptr;
      const unsigned fl = hipHostMallocMapped | hipHostMallocCoherent;
      if (hipHostMalloc((void **)&m->h_tok, R * 4, fl) != hipSuccess ||
          hipHostMalloc((void **)&m->h_next, R * 4, fl) != hipSuccess ||
          hipHostGetDevicePointer((void **)&m->d_tok, m->h_tok, 0) != hipSuccess ||
          hipHostGetDevicePointer((void **)&m->d_next, m->h_next, 0) != hipSuccess)
        rc = pbx_fail(m->c, PBX_ENOMEM, "model: pinned token buffers failed");
    }
    if (rc) {
      m->batch_cap = 0;
      return rc;
    }
    m->batch_cap = rows;
  }
  if (all_logits && rows > m->logits_cap) {
    if ((rc = grow(m, (void **)&m->blogits, (size_t)rows * g.vocab_size * 4)) ||
        (rc = grow(m, (void **)&m->bkeys, (size_t)rows * 64 * 8))) {
      m->logits_cap = 0;
      return rc;
    }
    // pbx_argmax_rows' cells start at zero (and each launch leaves them so)
    if (hipMemsetAsync(m->bkeys, 0, (size_t)rows * 64 * 8, m->c->stream) != hipSuccess) {
      m->logits_cap = 0;
      return pbx_fail(m->c, PBX_EHIP, "model: clearing the argmax cells failed");
    }
    m->logits_cap = rows;
  }
  return PBX_OK;
}

// The causal MFMA attention of a batched forward: the key stages of a
// workgroup split over two groups of four waves (PBX_PREFILL_ATTN_GROUPS=1:
// one group, the 256-thread form)
static bool prefill_attention_one_group() {
  const char *e = getenv("PBX_PREFILL_ATTN_GROUPS");
  return e && atoi(e) == 1;
}
static const char *prefill_attention_mfma() {
  return prefill_attention_one_group() ? "pbx_attention_mfma" : "pbx_attention_mfma_g2";
}
static int prefill_attention_threads() { return prefill_attention_one_group() ? 256 : 512; }

static int launch_k(pbx_model *m, const char *name, dim3 grid, dim3 block, void **args) {
  hipFunction_t f = pbx_kernel_by_name(m->c, name);
  if (!f) return pbx_fail(m->c, PBX_ELOAD, "model: kernel %s not found", name);
  return pbx_launch_fn(m->c, f, name, grid, block, args, m->c->stream);
}

// Y[n][N] (+)= X[n][K] . W^T over all rows.
static int linear_rows(pbx_model *m, const pbx_weight *w, const float *X, int n, float *Y,
                       bool accumulate) {
  pbx_ctx *c = m->c;
  if (w->type != PBX_TYPE_Q6_K && n >= PBX_GEMM_MIN_M)
    return pbx_gemm_launch(c, w, X, n, nullptr, Y, accumulate ? 1 : 0, c->stream);
  if (!accumulate) return pbx_linear_enqueue(c, w, X, n, nullptr, Y, c->stream);
  int rc = pbx_linear_enqueue(c, w, X, n, nullptr, m->btmp, c->stream);
  if (rc) return rc;
  int64_t count = (int64_t)n * w->N;
  float *y = Y, *t = m->btmp;
  void *args[] = {&y, &t, &count};
  return launch_k(m, "pbx_add_inplace", dim3((unsigned)((count + 255) / 256)), dim3(256), args);
}

// Row-batched integer-limb GEMVs (pbx_dk_q4_*r<MR>_*): one pass over the
// weights for up to MR activation rows, with the RMSNorm prologue and the
// residual / SwiGLU epilogues fused, for 1..8 rows (speculative verify,
// short prompts) of a Q4_0 model with dim <= 2048 and hidden_dim 6145..8192.
#define ROWS_MAX 8
static bool rows_int_ok(const pbx_model *m) {
  const pbx_model_config &g = m->cfg;
  if (!m->gemv_int || g.weight_type != PBX_TYPE_Q4_0 || g.dim > 2048 || g.hidden_dim > 8192 ||
      g.hidden_dim <= 6144)
    return false;
  const pbx_weight *head = m->output ? m->output : m->embd;
  return head->type == PBX_TYPE_Q4_0;
}

// Launches kernel `name` (MR rows a launch) over n rows in groups of MR.
static int launch_rows(pbx_model *m, const char *name, const pbx_weight *w, const float *X,
                       const float *normw, float *Y, int n, int MR, int rows_per_wg,
                       int wg_cap) {
  hipFunction_t f = pbx_kernel_by_name(m->c, name);
  if (!f) return pbx_fail(m->c, PBX_ELOAD, "model: kernel %s not found", name);
  const bool pair = strstr(name, "_gu") != nullptr;
  const int NO = pair ? (int)w->N / 2 : (int)w->N;
  int tiles = (NO + rows_per_wg - 1) / rows_per_wg;
  if (wg_cap > 0) tiles = std::min(tiles, wg_cap);
  for (int r0 = 0; r0 < n; r0 += MR) {
    pbx_gemv_args g{w->qs, w->d, X + (size_t)r0 * w->K, nullptr, normw, nullptr,
                    Y + (size_t)r0 * NO, nullptr, (int)w->N, (int)w->B, m->cfg.rms_eps, w->m,
                    std::min(MR, n - r0)};
    void *args[] = {&g};
    int rc = pbx_launch_fn(m->c, f, name, dim3((unsigned)tiles), dim3(512), args, m->c->stream);
    if (rc) return rc;
  }
  return PBX_OK;
}

// Row-batched GEMVs on int8 MFMAs (pbx_mr_q4_<RW>x<KS>b<IB>[s<XS>]_<mode>,
// gemv_mr) for 1..5 rows: RW 16-row weight tiles (8 gate + 8 up rows for gu)
// a workgroup of RW x KS waves; XS > 1: the K blocks split over XS
// workgroups (grid y, residual add only).  rope: q|k|v rows at positions
// start.. with RoPE and the cache append (the KV caches of layer l).
// Rows-kernel shape of a role (IB 64-block groups a row, K split over XS
// workgroups); for tuning, PBX_MR_SHAPES="role=RWxKS,..." (roles qkv, o,
// gate_up, down) picks another compiled shape.
struct MrShape {
  int rw, ks, ib, xs;
  std::string name(const char *mode) const {
    return "pbx_mr_q4_" + std::to_string(rw) + "x" + std::to_string(ks) + "b" +
           std::to_string(ib) + (xs > 1 ? "s" + std::to_string(xs) : "") + "_" + mode;
  }
};
static MrShape mr_shape(const char *role, int rw, int ks, int ib = 1, int xs = 1) {
  MrShape sh{rw, ks, ib, xs};
  const char *e = getenv("PBX_MR_SHAPES");
  if (!e) return sh;
  const std::string s(e), key = std::string(role) + "=";
  const size_t p = s.find(key);
  if (p != std::string::npos && (p == 0 || s[p - 1] == ','))
    sscanf(s.c_str() + p + key.size(), "%dx%d", &sh.rw, &sh.ks);
  return sh;
}

static int launch_mr(pbx_model *m, const char *name, const pbx_weight *w, const float *X,
                     const float *normw, float *Y, int n, int RW, int KS, int rope_layer = -1,
                     int start = 0, bool loop = false, int XS = 1) {
  hipFunction_t f = pbx_kernel_by_name(m->c, name);
  if (!f) return pbx_fail(m->c, PBX_ELOAD, "model: kernel %s not found", name);
  // the kernels take whole 64-block rows and whole 4-block steps a slice;
  // the split kernel's scratch holds MR_XS slices of dim rows
  if (w->type != PBX_TYPE_Q4_0 || w->B % 64 != 0 || w->B % (4 * KS * XS) != 0 || n > MR_MAX ||
      (XS > 1 && (XS > MR_XS || w->N > m->cfg.dim || !m->mr_cell)))
    return pbx_fail(m->c, PBX_EINVAL, "model: %s does not take this shape", name);
  const bool pair = strstr(name, "_gu") != nullptr;
  const int NO = pair ? (int)w->N / 2 : (int)w->N;
  const int tiles = (NO + (pair ? 7 : 15)) / (pair ? 8 : 16);
  pbx_gemv_args g{w->qs, w->d, X, nullptr, normw, nullptr, Y, nullptr, (int)w->N, (int)w->B,
                  m->cfg.rms_eps, w->m, n};
  if (rope_layer >= 0) {
    const size_t layer_kv = (size_t)m->cfg.max_seq * m->kvdim;
    g.rope = m->rope;
    g.kcache = m->kcache + rope_layer * layer_kv;
    g.vcache = m->vcache + rope_layer * layer_kv;
    g.qdim = m->cfg.dim;
    g.kvdim = m->kvdim;
    g.head_dim = m->cfg.head_dim;
    g.pos0 = start;
  }
  g.xcell = m->mr_cell;
  void *args[] = {&g};
  int grid = (tiles + RW - 1) / RW;
  if (loop) grid = std::min(grid, 2 * m->c->cu_count);  // tile loop: two workgroups a CU
  return pbx_launch_fn(m->c, f, name, dim3((unsigned)grid, (unsigned)XS), dim3(64 * RW * KS),
                       args, m->c->stream);
}

// Skinny Q4_0 MFMA kernels (pbx_sk_q4_*) for up to 8 rows: Y[r] (+)= W .
// (RMSNorm(X[r]) if normw) per row r < n, n <= 8.
struct SkinnyArgsHost {
  const void *qs;
  const void *dsc;
  const float *X;
  const float *normw;
  float *Y;
  int N, B, M, ldy;
  float eps;
};
static int launch_skinny(pbx_model *m, const char *name, const pbx_weight *w, const float *X,
                         const float *normw, float *Y, int n) {
  hipFunction_t f = pbx_kernel_by_name(m->c, name);
  if (!f) return pbx_fail(m->c, PBX_ELOAD, "model: kernel %s not found", name);
  const bool pair = strstr(name, "swiglu") != nullptr;
  const int NO = pair ? (int)w->N / 2 : (int)w->N;
  const int tiles = (NO + (pair ? 15 : 31)) / (pair ? 16 : 32);
  const int K = (int)w->B * 32;
  const int grid = K > 2048 ? tiles : std::min(tiles, 2 * m->c->cu_count);
  SkinnyArgsHost g{w->qs, w->d, X, normw, Y, (int)w->N, (int)w->B, n, NO, m->cfg.rms_eps};
  void *args[] = {&g};
  return pbx_launch_fn(m->c, f, name, dim3((unsigned)grid), dim3(256), args, m->c->stream);
}

static int rmsnorm_rows(pbx_model *m, const float *x, const float *w, float *out, int n) {
  int dim = m->cfg.dim;
  float eps = m->cfg.rms_eps;
  void *args[] = {(void *)&x, (void *)&w, &out, &dim, &eps};
  return launch_k(m, "pbx_rmsnorm_rows", dim3(n), dim3(256), args);
}

// Fused batched layers (fp16 MFMA GEMMs): the activation preparation of
// each GEMM is folded into the kernel that produces its input, and split-K
// partials are summed by the kernel that consumes them.  Per layer:
//   qkv GEMM -> RoPE + KV append (+ partial sum) -> attention -> prep -> o GEMM
//   -> residual add (+ partial sum) + RMSNorm + prep -> gate|up GEMM
//   -> SwiGLU + prep -> down GEMM -> residual add + next layer's RMSNorm + prep.
static bool fused_ok(const pbx_model *m, int n) {
  const pbx_model_config &g = m->cfg;
  const int t = g.weight_type;
  return n >= PBX_GEMM_MIN_M &&
         (t == PBX_TYPE_Q4_0 || t == PBX_TYPE_Q8_0 || t == PBX_TYPE_Q4_1 || t == PBX_TYPE_F16) &&
         g.dim <= 8192 && g.hidden_dim <= 8192;
}

struct FusedPlans {
  pbx_gemm_plan qkv, o, gu, d;
};

static int fused_plans(pbx_model *m, int n, FusedPlans *P) {
  pbx_ctx *c = m->c;
  const Layer &L = m->layers[0];
  int rc;
  if ((rc = pbx_gemm_make_plan(c, L.wqkv, n, &P->qkv)) || (rc = pbx_gemm_make_plan(c, L.wo, n, &P->o)) ||
      (rc = pbx_gemm_make_plan(c, L.wgu, n, &P->gu, true)) ||
      (rc = pbx_gemm_make_plan(c, L.wd, n, &P->d)))
    return rc;
  const pbx_model_config &g = m->cfg;
  const size_t kmax = std::max(g.dim, g.hidden_dim);
  const size_t act = ((size_t)P->qkv.Mpad * kmax * 2 + 255) / 256 * 256;
  size_t part = 0;
  for (const pbx_gemm_plan *p : {&P->qkv, &P->o, &P->gu, &P->d}) {
    const pbx_weight *w = p == &P->qkv ? L.wqkv : p == &P->o ? L.wo : p == &P->gu ? L.wgu : L.wd;
    if (p->KS > 1) part = std::max(part, (size_t)p->KS * n * w->N * 4);
  }
  if (act > m->g16_cap) {
    m->g16_cap = 0;
    if ((rc = grow(m, &m->g16, act)) || (rc = grow(m, &m->g16lo, act)) ||
        (rc = grow(m, (void **)&m->ginv, (size_t)P->qkv.Mpad * 4)))
      return rc;
    m->g16_cap = act;
  }
  if (part > m->gpart_cap) {
    m->gpart_cap = 0;
    if ((rc = grow(m, (void **)&m->gpart, part))) return rc;
    m->gpart_cap = part;
  }
  return PBX_OK;
}

// The GEMM of plan p on the prepared activations into Y (KS == 1; += if
// accumulate) or into the partials.
static int fused_gemm(pbx_model *m, const pbx_weight *w, const pbx_gemm_plan &p, float *Y,
                      bool accumulate) {
  return pbx_gemm_run(m->c, w, p, m->g16, m->g16lo, m->ginv, nullptr, p.KS == 1 ? Y : m->gpart,
                      accumulate ? 1 : 0, m->c->stream);
}

static int launch_k(pbx_model *m, const char *name, dim3 grid, dim3 block, void **args);

// Y (+)= the sum of the partials of a split GEMM (plain reduce).
static int fused_reduce(pbx_model *m, const pbx_gemm_plan &p, int N, float *Y, bool accumulate) {
  const float *part = m->gpart, *bias = nullptr;
  int M = p.M, n = N, ks = p.KS, acc = accumulate ? 1 : 0;
  const int64_t total = (int64_t)M * N;
  void *args[] = {(void *)&part, (void *)&bias, &Y, &M, &n, &ks, &acc};
  return launch_k(m, "pbx_gemm_reduce", dim3((unsigned)((total + 255) / 256)), dim3(256), args);
}

// x += the partials of the GEMM of plan p if it was split (p null: nothing to
// add), then the prepared RMSNorm(x) * normw for the next GEMM (none if
// normw is null).  M rows, Mpad prepared rows.
static int fused_residual_norm(pbx_model *m, const pbx_gemm_plan *p, int M, int Mpad, float *x,
                               const float *normw) {
  const pbx_model_config &g = m->cfg;
  int rows = M, K = g.dim;
  float eps = g.rms_eps;
  void *x16 = m->g16, *x16lo = m->g16lo;
  float *inv = m->ginv;
  if (p && p->KS > 1) {
    const float *part = m->gpart;
    int ks = p->KS;
    void *args[] = {(void *)&part, &ks, &x, (void *)&normw, &eps, &x16, &x16lo, &inv, &rows, &K};
    return launch_k(m, "pbx_gemm_reduce_rms", dim3(normw ? Mpad : M), dim3(256), args);
  }
  if (!normw) return PBX_OK;
  void *args[] = {(void *)&x, (void *)&normw, &eps, &x16, &x16lo, &inv, &rows, &K};
  return launch_k(m, "pbx_gemm_prep_rms", dim3(Mpad), dim3(256), args);
}

// Runs the first nl layers of the stack over n rows (the KV cache of later
// layers is not written, as llama-streaming.js:765-792 with maxLayers);
// leaves the residual stream in m->bx.
static int batch_layers(pbx_model *m, const int32_t *tokens, int n, int start, int nl) {
  pbx_ctx *c = m->c;
  const pbx_model_config &g = m->cfg;
  int rc;
  if (n <= 16) {
    // a short batch: the tokens as a kernel argument
    struct {
      int32_t t[16];
    } toks = {};
    memcpy(toks.t, tokens, (size_t)n * 4);
    const void *qs = m->embd->qs, *dsc = m->embd->d, *msc = m->embd->m;
    float *x = m->bx;
    int type = kernel_type(m->embd->type), dim = g.dim, vocab = g.vocab_size;
    void *args[] = {(void *)&qs, (void *)&dsc, (void *)&msc, &toks, &x, &type, &dim, &vocab};
    if ((rc = launch_k(m, "pbx_embed_rows_arg", dim3((g.dim + 255) / 256, n), dim3(256), args)))
      return rc;
  } else {
    // the embedding kernel reads the tokens from the pinned buffer (once the
    // previous kernel that read it is done)
    if (hipEventSynchronize(m->tok_ev) != hipSuccess)
      return pbx_fail(c, PBX_EHIP, "model: token staging wait failed");
    memcpy(m->h_tok, tokens, (size_t)n * 4);
    const void *qs = m->embd->qs, *dsc = m->embd->d, *msc = m->embd->m;
    int *tok = m->d_tok;
    float *x = m->bx;
    int type = kernel_type(m->embd->type), dim = g.dim, vocab = g.vocab_size;
    void *args[] = {(void *)&qs, (void *)&dsc, (void *)&msc, &tok, &x, &type, &dim, &vocab};
    if ((rc = launch_k(m, "pbx_embed_rows", dim3((g.dim + 255) / 256, n), dim3(256), args))) return rc;
    if (hipEventRecord(m->tok_ev, c->stream) != hipSuccess)
      return pbx_fail(c, PBX_EHIP, "model: token event failed");
  }
  const size_t layer_kv = (size_t)g.max_seq * m->kvdim;
  const bool rows_int = n <= ROWS_MAX && rows_int_ok(m);
  if (!rows_int && fused_ok(m, n)) {
    FusedPlans P;
    if ((rc = fused_plans(m, n, &P))) return rc;
    if (nl > 0 &&
        (rc = fused_residual_norm(m, nullptr, n, P.qkv.Mpad, m->bx, m->layers[0].attn_norm)))
      return rc;
    for (int l = 0; l < nl; ++l) {
      Layer &L = m->layers[l];
      float *kc = m->kcache + l * layer_kv, *vc = m->vcache + l * layer_kv;
      if ((rc = fused_gemm(m, L.wqkv, P.qkv, m->bqkv, false))) return rc;
      {
        float *qkv = m->bqkv, *rope = m->rope;
        const float *part = P.qkv.KS > 1 ? m->gpart : nullptr;
        int st = start, nh = g.n_heads, nkv = g.n_kv_heads, hd = g.head_dim, ks = P.qkv.KS;
        void *args[] = {&qkv, &kc, &vc, &rope, &st, &nh, &nkv, &hd, (void *)&part, &ks};
        if ((rc = launch_k(m, "pbx_rope_append_rows", dim3(n), dim3(256), args))) return rc;
      }
      {
        float *qkv = m->bqkv, *out = m->battn;
        int st = start, nh = g.n_heads, nkv = g.n_kv_heads, hd = g.head_dim, rows = n;
        float scale = (float)(1.0 / sqrt((double)g.head_dim));
        if (g.head_dim <= 64 && n >= 16) {
          void *args[] = {&qkv, &kc, &vc, &out, &st, &rows, &nh, &nkv, &hd, &scale};
          const bool mf = g.head_dim % 16 == 0;
          rc = launch_k(m, mf ? prefill_attention_mfma() : "pbx_attention_tiled",
                        dim3(g.n_heads, (n + 63) / 64), dim3(mf ? prefill_attention_threads() : 256),
                        args);
        } else {
          void *args[] = {&qkv, &kc, &vc, &out, &st, &nh, &nkv, &hd, &scale};
          if (g.head_dim <= 64)
            rc = launch_k(m, "pbx_attention_head_rows", dim3(g.n_heads, n), dim3(512), args);
          else
            rc = launch_k(m, "pbx_attention_rows", dim3(g.n_heads, n), dim3(256), args);
        }
        if (rc) return rc;
      }
      {
        float *x = m->battn;
        void *x16 = m->g16, *x16lo = m->g16lo;
        float *inv = m->ginv;
        int M = n, K = g.dim;
        void *args[] = {&x, &x16, &x16lo, &inv, &M, &K};
        if ((rc = launch_k(m, "pbx_gemm_prep_x", dim3(P.o.Mpad), dim3(256), args))) return rc;
      }
      if ((rc = fused_gemm(m, L.wo, P.o, m->bx, true)) ||
          (rc = fused_residual_norm(m, &P.o, n, P.o.Mpad, m->bx, L.ffn_norm)) ||
          (rc = fused_gemm(m, L.wgu, P.gu, m->bgu, false)))
        return rc;
      if (P.gu.KS > 1 && (rc = fused_reduce(m, P.gu, (int)L.wgu->N, m->bgu, false))) return rc;
      {
        // the down GEMM's input: silu(gate) * up, from the gate|up GEMM's
        // epilogue ([n][hidden]) or computed here from gate and up
        float *gu = m->bgu;
        void *x16 = m->g16, *x16lo = m->g16lo;
        float *inv = m->ginv;
        int M = n, hidden = g.hidden_dim;
        void *args[] = {&gu, &x16, &x16lo, &inv, &M, &hidden};
        if ((rc = launch_k(m, P.gu.swiglu ? "pbx_gemm_prep_x" : "pbx_gemm_prep_swiglu",
                           dim3(P.gu.Mpad), dim3(256), args)))
          return rc;
      }
      if ((rc = fused_gemm(m, L.wd, P.d, m->bx, true)) ||
          (rc = fused_residual_norm(m, &P.d, n, P.d.Mpad, m->bx,
                                    l + 1 < nl ? m->layers[l + 1].attn_norm : nullptr)))
        return rc;
    }
    return PBX_OK;
  }
  for (int l = 0; l < nl; ++l) {
    Layer &L = m->layers[l];
    float *kc = m->kcache + l * layer_kv, *vc = m->vcache + l * layer_kv;
    // 1..5 rows with head_dim <= 64: q|k|v on the MFMA rows kernel with RoPE
    // and the cache append (no pbx_rope_append_rows)
    const bool mr = rows_int && n <= MR_MAX && (int)L.wqkv->B == 64 && g.head_dim <= 64 &&
                    g.head_dim % 2 == 0 && g.dim % 16 == 0 && m->kvdim % 16 == 0;
    if (mr) {
      const MrShape qs = mr_shape("qkv", 1, 8);
      if ((rc = launch_mr(m, qs.name("qkvr").c_str(), L.wqkv, m->bx, L.attn_norm, m->bqkv, n,
                          qs.rw, qs.ks, l, start)))
        return rc;
    } else if (rows_int) {
      if ((rc = launch_rows(m, "pbx_dk_q4_i8x2b1r8_qkv", L.wqkv, m->bx, L.attn_norm, m->bqkv, n,
                            8, 16, 0)))
        return rc;
    } else {
      if ((rc = rmsnorm_rows(m, m->bx, L.attn_norm, m->bxn, n))) return rc;
      if ((rc = linear_rows(m, L.wqkv, m->bxn, n, m->bqkv, false))) return rc;
    }
    if (!mr) {
      float *qkv = m->bqkv, *rope = m->rope;
      int st = start, nh = g.n_heads, nkv = g.n_kv_heads, hd = g.head_dim;
      const float *part = nullptr;
      int ks = 1;
      void *args[] = {&qkv, &kc, &vc, &rope, &st, &nh, &nkv, &hd, (void *)&part, &ks};
      if ((rc = launch_k(m, "pbx_rope_append_rows", dim3(n), dim3(256), args))) return rc;
    }
    {
      float *qkv = m->bqkv, *out = m->battn;
      int st = start, nh = g.n_heads, nkv = g.n_kv_heads, hd = g.head_dim, rows = n;
      float scale = (float)(1.0 / sqrt((double)g.head_dim));
      // 64-row query tiles sharing K/V tiles in LDS pay off from 16 rows; a
      // few rows (speculative verify) spread better one workgroup per row.
      if (g.head_dim <= 64 && n >= 16) {
        // MFMA kernel for head dims that are a multiple of 16, else fp32 FMAs
        void *args[] = {&qkv, &kc, &vc, &out, &st, &rows, &nh, &nkv, &hd, &scale};
        const bool mf = g.head_dim % 16 == 0;
        rc = launch_k(m, mf ? prefill_attention_mfma() : "pbx_attention_tiled",
                      dim3(g.n_heads, (n + 63) / 64), dim3(mf ? prefill_attention_threads() : 256),
                      args);
      } else {
        void *args[] = {&qkv, &kc, &vc, &out, &st, &nh, &nkv, &hd, &scale};
        // head_dim <= 64: the decode kernel's flash layout per (head, row);
        // the generic one-workgroup-per-(head, row) kernel otherwise
        if (g.head_dim <= 64)
          rc = launch_k(m, "pbx_attention_head_rows", dim3(g.n_heads, n), dim3(512), args);
        else
          rc = launch_k(m, "pbx_attention_rows", dim3(g.n_heads, n), dim3(256), args);
      }
      if (rc) return rc;
    }
    if (mr && (int)L.wd->B == 256) {
      // 8 or 16 waves a workgroup (K slices across waves): the dots of a wave
      // wait on LDS round trips, so more waves hide them (verify M=5: 4 waves
      // 0.757 ms, these 0.673)
      const MrShape os = mr_shape("o", 1, 8), gs = mr_shape("gate_up", 4, 4),
                    ds = mr_shape("down", 4, 4, 4, 8);
      if ((rc = launch_mr(m, os.name("add").c_str(), L.wo, m->battn, nullptr, m->bx, n, os.rw,
                          os.ks)) ||
          (rc = launch_mr(m, gs.name("gu").c_str(), L.wgu, m->bx, L.ffn_norm, m->bh, n, gs.rw,
                          gs.ks)) ||
          (rc = launch_mr(m, ds.name("add").c_str(), L.wd, m->bh, nullptr, m->bx, n, ds.rw, ds.ks,
                          -1, 0, false, ds.xs)))
        return rc;
      continue;
    }
    if (rows_int) {
      // RMSNorm + gate|up + SwiGLU on the skinny MFMA kernel (17 us against 19
      // for the integer-limb rows kernel at 5 rows); q|k|v, o and down stay on
      // the integer-limb kernels, which are faster at these shapes
      if ((rc = launch_rows(m, "pbx_dk_q4_i8x1b1r8_add", L.wo, m->battn, nullptr, m->bx, n, 8, 8,
                            0)) ||
          (rc = launch_skinny(m, "pbx_sk_q4_swiglu", L.wgu, m->bx, L.ffn_norm, m->bh, n)) ||
          (rc = launch_rows(m, "pbx_dk_q4_i8x1b4r5_add", L.wd, m->bh, nullptr, m->bx, n, 5, 8, 0)))
        return rc;
      continue;
    }
    if ((rc = linear_rows(m, L.wo, m->battn, n, m->bx, true))) return rc;
    if ((rc = rmsnorm_rows(m, m->bx, L.ffn_norm, m->bxn, n))) return rc;
    if ((rc = linear_rows(m, L.wgu, m->bxn, n, m->bgu, false))) return rc;
    {
      float *gu = m->bgu, *h = m->bh;
      int hidden = g.hidden_dim;
      void *args[] = {&gu, &h, &hidden};
      if ((rc = launch_k(m, "pbx_swiglu_rows", dim3((g.hidden_dim + 255) / 256, n), dim3(256), args)))
        return rc;
    }
    if ((rc = linear_rows(m, L.wd, m->bh, n, m->bx, true))) return rc;
  }
  return PBX_OK;
}

// Prefill: the layer stack over n rows, then the decode step's own LM head
// and argmax on the last row, which leave the device state at
// (start + n, next token) as n sequential steps would.
static int prefill_batched(pbx_model *m, const int32_t *tokens, int n, int start, int nl) {
  int rc = ensure_batch(m, n, false);
  if (rc) return rc;
  if (!m->ops_ready && (rc = build_ops(m))) return rc;
  if ((rc = batch_layers(m, tokens, n, start, nl))) return rc;
  if ((rc = set_state(m, start + n - 1, tokens[n - 1], 0, false))) return rc;
  if (hipMemcpyAsync(m->x, m->bx + (size_t)(n - 1) * m->cfg.dim, (size_t)m->cfg.dim * 4,
                     hipMemcpyDeviceToDevice, m->c->stream) != hipSuccess)
    return pbx_fail(m->c, PBX_EHIP, "model: residual copy failed");
  // the LM head (on x, where the last row now is) and the argmax
  for (size_t i = m->layer_op[m->cfg.n_layers]; i < m->ops.size(); ++i) {
    Op op = m->ops[i];
    if (i == m->layer_op[m->cfg.n_layers]) op.gemv.X = m->x;
    if ((rc = enqueue_op(m, op))) return rc;
  }
  return PBX_OK;
}

static bool batched_prefill_enabled() {
  const char *e = getenv("PBX_BATCHED_PREFILL");
  return !(e && e[0] == '0');
}

extern "C" int pbx_model_forward(pbx_model *m, const int32_t *tokens, int n_tokens,
                                 int start_pos, float *logits, int32_t *next_token) {
  return pbx_model_forward_layers(m, tokens, n_tokens, start_pos, 0, logits, next_token, nullptr);
}

extern "C" int pbx_model_forward_layers(pbx_model *m, const int32_t *tokens, int n_tokens,
                                        int start_pos, int max_layers, float *logits,
                                        int32_t *next_token, int *layers_used) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_forward: not a live model");
  pbx_ctx *c = m->c;
  const pbx_model_config &g = m->cfg;
  if (!tokens || n_tokens <= 0)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_forward: need at least one token");
  if (start_pos < 0 || (int64_t)start_pos + n_tokens > g.max_seq)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_forward: positions [%d, %lld) exceed max_seq %d",
                    start_pos, (long long)start_pos + n_tokens, g.max_seq);
  for (int t = 0; t < n_tokens; ++t)
    if (tokens[t] < 0 || tokens[t] >= g.vocab_size)
      return pbx_fail(c, PBX_EINVAL, "pbx_model_forward: token %d out of range [0, %d)",
                      tokens[t], g.vocab_size);
  int rc = check_complete(m);
  if (rc) return rc;
  if (hipSetDevice(c->device) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_forward: hipSetDevice failed");
  // llama-streaming.js:745, 764: `options.maxLayers || nLayers`, then
  // min(maxLayers, nLayers) (a negative limit runs no layer)
  const int nl = max_layers == 0 ? g.n_layers : std::max(0, std::min(max_layers, g.n_layers));
  if (n_tokens >= PBX_GEMM_MIN_M && batched_prefill_enabled()) {
    if ((rc = prefill_batched(m, tokens, n_tokens, start_pos, nl))) return rc;
  } else {
    for (int t = 0; t < n_tokens; ++t) {
      if ((rc = set_state(m, start_pos + t, tokens[t], 0, true))) return rc;
      if ((rc = run_step_layers(m, nl))) return rc;
    }
  }
  if (layers_used) *layers_used = nl;
  if (logits && hipMemcpyAsync(logits, m->logits, (size_t)g.vocab_size * 4,
                               hipMemcpyDeviceToHost, c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_forward: logits copy failed");
  int st[4] = {0, 0, 0, 0};
  if (hipMemcpyAsync(st, m->state, sizeof st, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_forward: step failed on the device");
  if ((rc = check_status(m, st, "pbx_model_forward"))) return rc;
  if (next_token) *next_token = st[1];
  return PBX_OK;
}

extern "C" int pbx_model_forward_batch(pbx_model *m, const int32_t *tokens, int n_tokens,
                                       int start_pos, float *logits, int32_t *next_tokens) {
  if (!model_ok(m))
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_forward_batch: not a live model");
  pbx_ctx *c = m->c;
  const pbx_model_config &g = m->cfg;
  if (!tokens || n_tokens <= 0)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_forward_batch: need at least one token");
  if (n_tokens > 65535)
    return pbx_fail(c, PBX_ENOTSUP, "pbx_model_forward_batch: %d rows exceed 65535", n_tokens);
  if (start_pos < 0 || (int64_t)start_pos + n_tokens > g.max_seq)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_model_forward_batch: positions [%d, %lld) exceed max_seq %d", start_pos,
                    (long long)start_pos + n_tokens, g.max_seq);
  for (int t = 0; t < n_tokens; ++t)
    if (tokens[t] < 0 || tokens[t] >= g.vocab_size)
      return pbx_fail(c, PBX_EINVAL, "pbx_model_forward_batch: token %d out of range [0, %d)",
                      tokens[t], g.vocab_size);
  int rc = check_complete(m);
  if (rc) return rc;
  if (hipSetDevice(c->device) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_forward_batch: hipSetDevice failed");
  const int n = n_tokens;
  if ((rc = ensure_batch(m, n, true))) return rc;
  if ((rc = batch_layers(m, tokens, n, start_pos, g.n_layers))) return rc;
  const pbx_weight *head = m->output ? m->output : m->embd;
  if (n <= ROWS_MAX && rows_int_ok(m)) {
    // RMSNorm + LM head over the rows: a Q4_0 head at K = 2048 on the rows
    // kernel, 8 tiles a workgroup (5 rows: 46 us against 64 on the skinny
    // MFMA kernel, which takes the other heads)
    const bool mr_head = head->type == PBX_TYPE_Q4_0 && head->B == 64 && n <= MR_MAX;
    if (mr_head) {
      const MrShape hs = mr_shape("lm_head", 8, 1);
      if ((rc = launch_mr(m, hs.name("store").c_str(), head, m->bx, m->out_norm, m->blogits, n,
                          hs.rw, hs.ks)))
        return rc;
    } else if ((rc = launch_skinny(m, "pbx_sk_q4_store", head, m->bx, m->out_norm, m->blogits, n)))
      return rc;
  } else {
    if ((rc = rmsnorm_rows(m, m->bx, m->out_norm, m->bxn, n))) return rc;
    if ((rc = linear_rows(m, head, m->bxn, n, m->blogits, false))) return rc;
  }
  {
    // P workgroups per row, ~2048 columns each, meeting in the row's cells
    const float *lg = m->blogits;
    int vocab = g.vocab_size;
    int P = std::min(64, (g.vocab_size + 2047) / 2048);
    int chunk = (g.vocab_size + P - 1) / P;
    unsigned long long *cells = (unsigned long long *)m->bkeys;
    int stride = 64;
    int *out = next_tokens ? m->d_next : m->bnext;  // straight into host memory
    void *a1[] = {(void *)&lg, &vocab, &chunk, &cells, &stride, &P, &out};
    if ((rc = launch_k(m, "pbx_argmax_rows", dim3(P, n), dim3(256), a1))) return rc;
  }
  if (logits && hipMemcpyAsync(logits, m->blogits, (size_t)n * g.vocab_size * 4,
                               hipMemcpyDeviceToHost, c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_forward_batch: logits copy failed");
  if (hipStreamSynchronize(c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_forward_batch: forward failed on the device");
  if (next_tokens) memcpy(next_tokens, m->h_next, (size_t)n * 4);
  return PBX_OK;
}

extern "C" int pbx_model_generate(pbx_model *m, int32_t token, int start_pos, int n_steps,
                                  int32_t *out_tokens, float *last_logits) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_generate: not a live model");
  pbx_ctx *c = m->c;
  const pbx_model_config &g = m->cfg;
  if (n_steps <= 0 || !out_tokens)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_generate: need n_steps > 0 and an output array");
  if (token < 0 || token >= g.vocab_size)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_generate: token %d out of range", token);
  if (start_pos < 0 || (int64_t)start_pos + n_steps > g.max_seq)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_generate: positions [%d, %lld) exceed max_seq %d",
                    start_pos, (long long)start_pos + n_steps, g.max_seq);
  int rc = check_complete(m);
  if (rc) return rc;
  if (hipSetDevice(c->device) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_generate: hipSetDevice failed");
  if ((rc = prepare_graphs(m))) return rc;
  if ((rc = set_state(m, start_pos, token, 0, true))) return rc;
  for (int i = 0, k = 0; i < n_steps; i += k)
    if ((rc = run_steps(m, n_steps - i, &k))) return rc;
  if (hipMemcpyAsync(out_tokens, m->hist, (size_t)n_steps * 4, hipMemcpyDeviceToHost,
                     c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_generate: token copy failed");
  if (last_logits && hipMemcpyAsync(last_logits, m->logits, (size_t)g.vocab_size * 4,
                                    hipMemcpyDeviceToHost, c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_generate: logits copy failed");
  int st[4] = {0, 0, 0, 0};
  if (hipMemcpyAsync(st, m->state, sizeof st, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_generate: step failed on the device");
  return check_status(m, st, "pbx_model_generate");
}

extern "C" int pbx_model_generate_eos(pbx_model *m, int32_t token, int start_pos, int max_steps,
                                      const int32_t *eos_ids, int n_eos, int32_t *out_tokens,
                                      int *n_out) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_generate_eos: not a live model");
  pbx_ctx *c = m->c;
  const pbx_model_config &g = m->cfg;
  if (max_steps <= 0 || !out_tokens || !n_out || n_eos < 0 || (n_eos > 0 && !eos_ids))
    return pbx_fail(c, PBX_EINVAL, "pbx_model_generate_eos: bad arguments");
  if (token < 0 || token >= g.vocab_size)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_generate_eos: token %d out of range", token);
  if (start_pos < 0 || (int64_t)start_pos + max_steps > g.max_seq)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_model_generate_eos: positions [%d, %lld) exceed max_seq %d", start_pos,
                    (long long)start_pos + max_steps, g.max_seq);
  *n_out = 0;
  int rc = check_complete(m);
  if (rc) return rc;
  if (hipSetDevice(c->device) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_generate_eos: hipSetDevice failed");
  if ((rc = prepare_graphs(m))) return rc;
  if ((rc = set_state(m, start_pos, token, 0, true))) return rc;
  // chunks of whole graph launches; after each, the chunk's tokens come back
  // and the loop stops at the first EOS, as llama.js:475-489 does
  const int chunk = std::max(1, m->graph_steps);
  int done = 0;
  while (done < max_steps) {
    const int want = std::min(chunk, max_steps - done);
    for (int i = 0, k = 0; i < want; i += k)
      if ((rc = run_steps(m, want - i, &k))) return rc;
    int st[4] = {0, 0, 0, 0};
    if (hipMemcpyAsync(out_tokens + done, m->hist + done, (size_t)want * 4, hipMemcpyDeviceToHost,
                       c->stream) != hipSuccess ||
        hipMemcpyAsync(st, m->state, sizeof st, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
      return pbx_fail(c, PBX_EHIP, "pbx_model_generate_eos: step failed on the device");
    if ((rc = check_status(m, st, "pbx_model_generate_eos"))) return rc;
    for (int i = 0; i < want; ++i) {
      const int32_t t = out_tokens[done + i];
      bool eos = false;
      for (int e = 0; e < n_eos; ++e) eos |= t == eos_ids[e];
      if (!eos) continue;
      // step done + i chose EOS; the steps after it fed tokens the
      // reference never feeds: drop their cache rows
      *n_out = done + i + 1;
      const int stop = start_pos + done + i + 1;
      if (stop < start_pos + done + want && (rc = pbx_model_clear_range(m, stop, start_pos + done + want)))
        return rc;
      if (hipStreamSynchronize(c->stream) != hipSuccess)
        return pbx_fail(c, PBX_EHIP, "pbx_model_generate_eos: device failure");
      return PBX_OK;
    }
    done += want;
  }
  *n_out = done;
  return PBX_OK;
}

// The greedy chain of pbx_model_generate with every step stopping after the
// first max_layers layers: the self-speculative draft (speculative.js:96-111,
// forward([t], pos, {maxLayers}) then argmax, repeated), replayed on the
// device.  out_tokens receives the n_steps drafted tokens.
int pbx_model_generate_layers(pbx_model *m, int32_t token, int start_pos, int n_steps,
                              int max_layers, int32_t *out_tokens) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_generate: not a live model");
  pbx_ctx *c = m->c;
  const pbx_model_config &g = m->cfg;
  if (n_steps <= 0 || !out_tokens || max_layers < 0)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_generate: bad arguments");
  if (token < 0 || token >= g.vocab_size)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_generate: token %d out of range", token);
  if (start_pos < 0 || (int64_t)start_pos + n_steps > g.max_seq)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_generate: positions [%d, %lld) exceed max_seq %d",
                    start_pos, (long long)start_pos + n_steps, g.max_seq);
  int rc = check_complete(m);
  if (rc) return rc;
  const int nl = max_layers == 0 ? g.n_layers : std::min(max_layers, g.n_layers);
  if ((rc = set_state(m, start_pos, token, 0, true))) return rc;
  for (int i = 0; i < n_steps; ++i)
    if ((rc = run_step_layers(m, nl))) return rc;
  int st[4] = {0, 0, 0, 0};
  if (hipMemcpyAsync(out_tokens, m->hist, (size_t)n_steps * 4, hipMemcpyDeviceToHost,
                     c->stream) != hipSuccess ||
      hipMemcpyAsync(st, m->state, sizeof st, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_generate: step failed on the device");
  return check_status(m, st, "pbx_model_generate");
}

extern "C" int pbx_model_reset_cache(pbx_model *m) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_reset_cache: not a live model");
  return kv_fill(m, 0);
}

extern "C" int pbx_model_rollback(pbx_model *m, int pos) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_rollback: not a live model");
  if (pos < 0 || pos > m->cfg.max_seq)
    return pbx_fail(m->c, PBX_EINVAL, "pbx_model_rollback: pos %d outside [0, %d]", pos,
                    m->cfg.max_seq);
  return kv_fill(m, pos);
}

// Zeroes cache positions [from, to) of every layer: the part of
// rollbackCache (llama-streaming.js:845-862) that a verify round can have
// written, without touching the never-written tail.
int pbx_model_clear_range(pbx_model *m, int from, int to) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "model: not a live model");
  from = std::max(from, 0);
  to = std::min(to, m->cfg.max_seq);
  if (to <= from) return PBX_OK;
  hipFunction_t f = pbx_kernel_by_name(m->c, "pbx_kv_fill");
  if (!f) return pbx_fail(m->c, PBX_ELOAD, "model: kernel pbx_kv_fill not found");
  int64_t stride = (int64_t)m->cfg.max_seq * m->kvdim;
  int64_t off = (int64_t)from * m->kvdim;
  int64_t count = (int64_t)(to - from) * m->kvdim;
  int nl = m->cfg.n_layers;
  float *k = m->kcache, *v = m->vcache;
  void *args[] = {&k, &v, &stride, &off, &count, &nl};
  const int64_t total = count * nl;
  return pbx_launch_fn(m->c, f, "pbx_kv_fill", dim3((unsigned)((total + 255) / 256)), dim3(256),
                       args, m->c->stream);
}

const pbx_model_config *pbx_model_cfg(const pbx_model *m) {
  return model_ok(m) ? &m->cfg : nullptr;
}

pbx_ctx *pbx_model_ctx(const pbx_model *m) { return model_ok(m) ? m->c : nullptr; }

extern "C" int pbx_model_info(const pbx_model *m, size_t *device_bytes, int *uses_graph) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_info: not a live model");
  if (device_bytes) *device_bytes = m->bytes;
  if (uses_graph) *uses_graph = m->graph_ok ? 1 : 0;
  return PBX_OK;
}

extern "C" int pbx_model_profile(pbx_model *m, int32_t token, int start_pos, int n_steps,
                                 double *op_us, double *op_bytes, int cap, int *n_ops) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_profile: not a live model");
  pbx_ctx *c = m->c;
  if (!op_us || !n_ops || cap <= 0 || n_steps <= 0)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_profile: bad arguments");
  if (token < 0 || token >= m->cfg.vocab_size || start_pos < 0 ||
      (int64_t)start_pos + n_steps > m->cfg.max_seq)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_profile: token/positions out of range");
  int rc = check_complete(m);
  if (rc) return rc;
  if (!m->ops_ready && (rc = build_ops(m))) return rc;
  const int n = (int)m->ops.size();
  // a start and a stop event per kernel, stamped by the kernel's dispatch
  std::vector<hipEvent_t> ev(2 * n, nullptr);
  for (auto &e : ev)
    if (hipEventCreate(&e) != hipSuccess) {
      for (auto &f : ev)
        if (f) hipEventDestroy(f);
      return pbx_fail(c, PBX_EHIP, "pbx_model_profile: hipEventCreate failed");
    }
  std::vector<double> acc(n, 0.0), bytes(n, 0.0);
  if ((rc = set_state(m, start_pos, token, 0, true))) goto out;
  for (int s = 0; s < n_steps && !rc; ++s) {
    for (int i = 0; i < n && !rc; ++i) rc = enqueue_op(m, m->ops[i], ev[2 * i], ev[2 * i + 1]);
    if (rc || hipEventSynchronize(ev[2 * n - 1]) != hipSuccess) {
      if (!rc) rc = pbx_fail(c, PBX_EHIP, "pbx_model_profile: step failed on the device");
      break;
    }
    for (int i = 0; i < n; ++i) {
      float ms = 0.f;
      hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]);
      acc[i] += ms * 1e3;
      const Op &op = m->ops[i];
      bytes[i] += (op.kind == ARG_ATTN || op.kind == ARG_ATTN_SPLIT || op.kind == ARG_FUSED ||
                   op.kind == ARG_SMALL)
                      ? op.bytes * (start_pos + s + 1)
                      : op.bytes;
      bytes[i] += op.fixed_bytes;
    }
  }
  if (!rc) {
    int st[4] = {0, 0, 0, 0};
    if (hipMemcpy(st, m->state, sizeof st, hipMemcpyDeviceToHost) != hipSuccess)
      rc = pbx_fail(c, PBX_EHIP, "pbx_model_profile: state copy failed");
    else
      rc = check_status(m, st, "pbx_model_profile");
  }
  if (!rc) {
    const int k = std::min(n, cap);
    for (int i = 0; i < k; ++i) {
      op_us[i] = acc[i] / n_steps;
      if (op_bytes) op_bytes[i] = bytes[i] / n_steps;
    }
    *n_ops = n;
  }
out:
  for (auto &e : ev) hipEventDestroy(e);
  return rc;
}

extern "C" int pbx_model_op_name(const pbx_model *m, int i, char *buf, size_t cap) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_op_name: not a live model");
  if (i < 0 || i >= (int)m->ops.size() || !buf || !cap)
    return pbx_fail(m->c, PBX_EINVAL, "pbx_model_op_name: op %d out of range", i);
  snprintf(buf, cap, "%s:%s", m->ops[i].role.c_str(), m->ops[i].name.c_str());
  return PBX_OK;
}

extern "C" int pbx_model_test_handoff(pbx_model *m, int layer, int skew, int spin) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_test_handoff: not a live model");
  if (layer >= m->cfg.n_layers || spin < 0)
    return pbx_fail(m->c, PBX_EINVAL, "pbx_model_test_handoff: layer %d / spin %d out of range",
                    layer, spin);
  m->test_layer = layer;
  m->test_skew = skew;
  m->test_spin = spin;
  // the kernels' arguments change: rebuild them and every captured graph
  drop_graph(m);
  m->ops_ready = false;
  int rc = check_complete(m);
  if (rc || (rc = build_ops(m))) return rc;
  for (const Op &op : m->ops)
    if (op.kind == ARG_FUSED || op.kind == ARG_SMALL) return PBX_OK;
  return layer < 0 ? PBX_OK
                   : pbx_fail(m->c, PBX_ENOTSUP,
                              "pbx_model_test_handoff: the step has no joined q|k|v + attention launch");
}

extern "C" int pbx_model_bench_role(pbx_model *m, const char *role, int reps,
                                    double *us_per_launch, double *bytes_per_launch,
                                    int *launches_per_rep) {
  if (!model_ok(m)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_model_bench_role: not a live model");
  pbx_ctx *c = m->c;
  if (!role || reps <= 0 || !us_per_launch)
    return pbx_fail(c, PBX_EINVAL, "pbx_model_bench_role: bad arguments");
  int rc = check_complete(m);
  if (rc) return rc;
  if (!m->ops_ready && (rc = build_ops(m))) return rc;
  std::vector<Op *> sel;
  double bytes = 0;
  for (Op &op : m->ops)
    if (op.kind == ARG_GEMV && op.role == role) {
      sel.push_back(&op);
      bytes += op.bytes;
    }
  if (sel.empty())
    return pbx_fail(c, PBX_EINVAL, "pbx_model_bench_role: no GEMV with role '%s'", role);
  for (Op *op : sel)  // warm-up pass
    if ((rc = enqueue_op(m, *op))) return rc;
  if (hipEventRecord(c->ev0, c->stream) != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "pbx_model_bench_role: hipEventRecord failed");
  for (int r = 0; r < reps; ++r)
    for (Op *op : sel)
      if ((rc = enqueue_op(m, *op))) return rc;
  double ms = 0;
  if ((rc = pbx_timer_stop(c, &ms))) return rc;
  *us_per_launch = ms * 1e3 / ((double)reps * sel.size());
  if (bytes_per_launch) *bytes_per_launch = bytes / sel.size();
  if (launches_per_rep) *launches_per_rep = (int)sel.size();
  return PBX_OK;
}
