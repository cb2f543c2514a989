/*
 * llama_ref.c -- TEST INFRASTRUCTURE, NOT PART OF THE PRODUCT.
 *
 * The reference's Llama forward pass, LlamaRuntime.forward (llama.js:204-371),
 * restated in C on fp32 weights (for GGUF Q4_0/Q8_0 models: the exactly
 * dequantised weights, as gguf.js:219-367 produces them).  JavaScript
 * computes in double and stores into Float32Array; so does this file, at the
 * same points:
 *   RMS_NORM        engine.js:429-449   sum of squares in double, f32 store
 *   LINEAR          engine.js:180-244   products summed in double, f32 store
 *   RoPE            llama.js:159-191    angle, cos, sin in double, f32 store
 *   attention       llama.js:258-301    scores/exp stored f32, sums in double
 *   TENSOR_ADD      engine.js:94-104
 *   SILU/ELEMENT_MUL engine.js:459-481
 *   LM head         llama.js:343-367    last position only
 * Weights use GGUF orientation W[n][k] (n = output feature).
 * Rows of a LINEAR are independent, so they run under OpenMP.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  int dim, hidden, n_layers, n_heads, n_kv, head_dim, vocab, max_seq;
  double theta, eps;
} pbo_cfg;

typedef struct {
  float *wq, *wk, *wv, *wo, *w1, *w2, *w3, *att_norm, *ffn_norm;
  float *kc, *vc; /* [max_seq][kv_dim] */
} pbo_layer;

typedef struct {
  pbo_cfg c;
  int kv_dim;
  pbo_layer *L;
  float *emb, *out_w, *out_norm; /* out_w == NULL: tied to emb */
} pbo_llama;

/* same ids as the product's PBX_T_* (tensor names of gguf.js:378-410) */
enum { T_EMBD = 0, T_OUTPUT, T_OUTPUT_NORM, T_ATTN_NORM, T_FFN_NORM, T_Q, T_K, T_V, T_O,
       T_GATE, T_UP, T_DOWN };

pbo_llama *pbo_llama_create(const pbo_cfg *c) {
  pbo_llama *m = (pbo_llama *)calloc(1, sizeof *m);
  m->c = *c;
  m->kv_dim = c->n_kv * c->head_dim;
  m->L = (pbo_layer *)calloc((size_t)c->n_layers, sizeof(pbo_layer));
  for (int l = 0; l < c->n_layers; ++l) {
    m->L[l].kc = (float *)calloc((size_t)c->max_seq * m->kv_dim, 4);
    m->L[l].vc = (float *)calloc((size_t)c->max_seq * m->kv_dim, 4);
  }
  return m;
}

static float *dup(const float *p, size_t n) {
  float *q = (float *)malloc(n * 4);
  memcpy(q, p, n * 4);
  return q;
}

void pbo_llama_set(pbo_llama *m, int tensor, int layer, const float *data) {
  const pbo_cfg *c = &m->c;
  const size_t D = c->dim, H = c->hidden, KV = m->kv_dim, V = c->vocab;
  pbo_layer *L = (layer >= 0 && layer < c->n_layers) ? &m->L[layer] : NULL;
  switch (tensor) {
    case T_EMBD: free(m->emb); m->emb = dup(data, V * D); break;
    case T_OUTPUT: free(m->out_w); m->out_w = dup(data, V * D); break;
    case T_OUTPUT_NORM: free(m->out_norm); m->out_norm = dup(data, D); break;
    case T_ATTN_NORM: free(L->att_norm); L->att_norm = dup(data, D); break;
    case T_FFN_NORM: free(L->ffn_norm); L->ffn_norm = dup(data, D); break;
    case T_Q: free(L->wq); L->wq = dup(data, D * D); break;
    case T_K: free(L->wk); L->wk = dup(data, KV * D); break;
    case T_V: free(L->wv); L->wv = dup(data, KV * D); break;
    case T_O: free(L->wo); L->wo = dup(data, D * D); break;
    case T_GATE: free(L->w1); L->w1 = dup(data, H * D); break;
    case T_UP: free(L->w3); L->w3 = dup(data, H * D); break;
    case T_DOWN: free(L->w2); L->w2 = dup(data, D * H); break;
  }
}

void pbo_llama_free(pbo_llama *m) {
  if (!m) return;
  for (int l = 0; l < m->c.n_layers; ++l) {
    pbo_layer *L = &m->L[l];
    free(L->wq); free(L->wk); free(L->wv); free(L->wo); free(L->w1); free(L->w2); free(L->w3);
    free(L->att_norm); free(L->ffn_norm); free(L->kc); free(L->vc);
  }
  free(m->L);
  free(m->emb); free(m->out_w); free(m->out_norm);
  free(m);
}

/* resetCache (llama.js:376-385) / rollbackCache (llama-streaming.js:845-862) */
void pbo_llama_rollback(pbo_llama *m, int pos) {
  for (int l = 0; l < m->c.n_layers; ++l)
    for (int p = pos; p < m->c.max_seq; ++p) {
      memset(m->L[l].kc + (size_t)p * m->kv_dim, 0, (size_t)m->kv_dim * 4);
      memset(m->L[l].vc + (size_t)p * m->kv_dim, 0, (size_t)m->kv_dim * 4);
    }
}

/* engine.js:429-449 */
static void rmsnorm(const float *x, const float *w, int S, int D, double eps, float *out) {
  for (int s = 0; s < S; ++s) {
    double ss = 0;
    for (int d = 0; d < D; ++d) ss += (double)x[s * D + d] * x[s * D + d];
    const double rms = sqrt(ss / D + eps);
    for (int d = 0; d < D; ++d) out[s * D + d] = (float)((x[s * D + d] / rms) * w[d]);
  }
}

/* LINEAR without bias: out[s][n] = sum_k x[s][k] * W[n][k], each sum in k
 * order in double.  Four weight rows share the loop over k (four
 * independent sums, so the double adds do not wait on each other) and the
 * rows s run inside the loop over n, so a weight row is read from memory
 * once for all of them; every sum is the same as the one-at-a-time loop's. */
static void linear(const float *x, int S, int K, const float *W, int N, float *out) {
#pragma omp parallel for schedule(static)
  for (int n0 = 0; n0 < N; n0 += 4) {
    const int nn = N - n0 < 4 ? N - n0 : 4;
    const float *w0 = W + (size_t)n0 * K;
    for (int s = 0; s < S; ++s) {
      const float *xs = x + (size_t)s * K;
      if (nn == 4) {
        const float *w1 = w0 + K, *w2 = w1 + K, *w3 = w2 + K;
        double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
        for (int k = 0; k < K; ++k) {
          const double xv = xs[k];
          a0 += xv * w0[k];
          a1 += xv * w1[k];
          a2 += xv * w2[k];
          a3 += xv * w3[k];
        }
        float *o = out + (size_t)s * N + n0;
        o[0] = (float)a0;
        o[1] = (float)a1;
        o[2] = (float)a2;
        o[3] = (float)a3;
      } else {
        for (int i = 0; i < nn; ++i) {
          const float *w = w0 + (size_t)i * K;
          double acc = 0;
          for (int k = 0; k < K; ++k) acc += (double)xs[k] * w[k];
          out[(size_t)s * N + n0 + i] = (float)acc;
        }
      }
    }
  }
}

/* llama.js:204-371 for tokens[0..S) at start_pos; logits of the last position.
 * max_layers: StreamingLlamaRuntime.forward's {maxLayers}
 * (llama-streaming.js:745, 764-792): `maxLayers || nLayers` layers, at most
 * n_layers, then the final norm and head on their output; later layers'
 * caches are not written. */
void pbo_llama_forward_layers(pbo_llama *m, const int *tokens, int S, int start_pos,
                              int max_layers, float *logits) {
  const pbo_cfg *c = &m->c;
  int nl = max_layers == 0 ? c->n_layers : max_layers;
  if (nl > c->n_layers) nl = c->n_layers;
  if (nl < 0) nl = 0;
  const int D = c->dim, H = c->hidden, HD = c->head_dim, NH = c->n_heads, KV = m->kv_dim;
  const int cacheLen = start_pos + S;
  float *x = (float *)malloc((size_t)S * D * 4), *xn = (float *)malloc((size_t)S * D * 4);
  float *q = (float *)malloc((size_t)S * D * 4), *k = (float *)malloc((size_t)S * KV * 4);
  float *v = (float *)malloc((size_t)S * KV * 4), *att = (float *)malloc((size_t)S * D * 4);
  float *proj = (float *)malloc((size_t)S * D * 4);
  float *g = (float *)malloc((size_t)S * H * 4), *u = (float *)malloc((size_t)S * H * 4);
  float *sc = (float *)malloc((size_t)cacheLen * 4);

  for (int i = 0; i < S; ++i) memcpy(x + (size_t)i * D, m->emb + (size_t)tokens[i] * D, (size_t)D * 4);

  const int per_kv = NH / c->n_kv;
  const double scale = 1.0 / sqrt((double)HD);
  for (int l = 0; l < nl; ++l) {
    pbo_layer *L = &m->L[l];
    rmsnorm(x, L->att_norm, S, D, c->eps, xn);
    linear(xn, S, D, L->wq, D, q);
    linear(xn, S, D, L->wk, KV, k);
    linear(xn, S, D, L->wv, KV, v);
    /* RoPE, llama.js:159-191 */
    for (int t = 0; t < S; ++t) {
      const int pos = start_pos + t;
      for (int i = 0; i < HD; i += 2) {
        const double freq = 1.0 / pow(c->theta, (double)i / HD);
        const double ang = pos * freq, ca = cos(ang), sa = sin(ang);
        for (int h = 0; h < NH; ++h) {
          float *p = q + (size_t)t * D + h * HD + i;
          const double q0 = p[0], q1 = p[1];
          p[0] = (float)(q0 * ca - q1 * sa);
          p[1] = (float)(q0 * sa + q1 * ca);
        }
        for (int h = 0; h < c->n_kv; ++h) {
          float *p = k + (size_t)t * KV + h * HD + i;
          const double k0 = p[0], k1 = p[1];
          p[0] = (float)(k0 * ca - k1 * sa);
          p[1] = (float)(k0 * sa + k1 * ca);
        }
      }
    }
    for (int t = 0; t < S; ++t) {
      memcpy(L->kc + (size_t)(start_pos + t) * KV, k + (size_t)t * KV, (size_t)KV * 4);
      memcpy(L->vc + (size_t)(start_pos + t) * KV, v + (size_t)t * KV, (size_t)KV * 4);
    }
    /* attention, llama.js:258-301 */
    for (int t = 0; t < S; ++t)
      for (int h = 0; h < NH; ++h) {
        const int kvh = h / per_kv;
        for (int j = 0; j < cacheLen; ++j) {
          if (j > start_pos + t) {
            sc[j] = -INFINITY;
            continue;
          }
          double dot = 0;
          for (int d = 0; d < HD; ++d)
            dot += (double)q[(size_t)t * D + h * HD + d] * L->kc[(size_t)j * KV + kvh * HD + d];
          sc[j] = (float)(dot * scale);
        }
        float mx = -INFINITY;
        for (int j = 0; j < cacheLen; ++j)
          if (sc[j] > mx) mx = sc[j];
        double sum = 0;
        for (int j = 0; j < cacheLen; ++j) {
          sc[j] = (float)exp((double)sc[j] - mx);
          sum += sc[j];
        }
        for (int j = 0; j < cacheLen; ++j) sc[j] = (float)(sc[j] / sum);
        for (int d = 0; d < HD; ++d) {
          double val = 0;
          for (int j = 0; j < cacheLen; ++j) val += (double)sc[j] * L->vc[(size_t)j * KV + kvh * HD + d];
          att[(size_t)t * D + h * HD + d] = (float)val;
        }
      }
    linear(att, S, D, L->wo, D, proj);
    for (size_t i = 0; i < (size_t)S * D; ++i) x[i] = (float)((double)x[i] + proj[i]);
    rmsnorm(x, L->ffn_norm, S, D, c->eps, xn);
    linear(xn, S, D, L->w1, H, g);
    for (size_t i = 0; i < (size_t)S * H; ++i) g[i] = (float)(g[i] / (1 + exp(-(double)g[i])));
    linear(xn, S, D, L->w3, H, u);
    for (size_t i = 0; i < (size_t)S * H; ++i) g[i] = (float)((double)g[i] * u[i]);
    linear(g, S, H, L->w2, D, proj);
    for (size_t i = 0; i < (size_t)S * D; ++i) x[i] = (float)((double)x[i] + proj[i]);
  }
  rmsnorm(x, m->out_norm, S, D, c->eps, xn);
  const float *last = xn + (size_t)(S - 1) * D;
  linear(last, 1, D, m->out_w ? m->out_w : m->emb, c->vocab, logits);
  free(x); free(xn); free(q); free(k); free(v); free(att); free(proj); free(g); free(u); free(sc);
}

void pbo_llama_forward(pbo_llama *m, const int *tokens, int S, int start_pos, float *logits) {
  pbo_llama_forward_layers(m, tokens, S, start_pos, 0, logits);
}

/* llama.js:432-442: first index of the maximum (strict >). */
int pbo_argmax(const float *v, int n) {
  float best = -INFINITY;
  int idx = 0;
  for (int i = 0; i < n; ++i)
    if (v[i] > best) {
      best = v[i];
      idx = i;
    }
  return idx;
}
