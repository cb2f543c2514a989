/*
 * cpu_baseline.c -- TEST / MEASUREMENT INFRASTRUCTURE, NOT PART OF THE PRODUCT.
 *
 * The reference's CPU path for the Q4_0 decode matvec, restated in C so it
 * can be timed on the GPU box's host cores beside the GPU kernels (bench.py's
 * cpu_baseline leg).  The reference itself is Node.js + runtime-generated
 * WebAssembly SIMD; it cannot travel to the GPU box, and this container's
 * Node 12 can neither parse gguf.js nor compile final-opcode WASM SIMD.
 *
 *  - q4_0 kernel: wasm-q4.js:118-267, one SSE instruction per f32x4/i32x4
 *    operation (byte shuffle, and 0x0F, shift right 4, subtract 8, convert,
 *    multiply, add; no FMA), same accumulation order; its output is
 *    bit-identical to pbo_q4_0_matvec_wasm (tests/test_oracle.py).
 *  - host wrapper: wasm-q4.js:716-747 copies x and the whole raw row slice
 *    into the module's linear memory on every call; so does this.
 *  - thread pool: thread-pool.js:165-246 with worker-matvec.js:79-145:
 *    T threads = (T-1) persistent workers + the calling thread; rows split
 *    floor(N/T) each, the first N%T workers take one more, the caller takes
 *    the tail; the call returns when every slice is written.
 *  - LM head: wasmQ4.lmHead (wasm-q4.js:798-839), single-threaded, 1024-row
 *    chunks copied into linear memory, batch_dot (447-566) on each.
 */
#define _GNU_SOURCE
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <tmmintrin.h>

static float f16_wasm(uint16_t bits) {
  const uint32_t exp = (bits >> 10) & 0x1f;
  if (exp == 0) return 0.0f;
  const uint32_t u = ((uint32_t)(bits >> 15) << 31) | ((exp + 112u) << 23) |
                     ((uint32_t)(bits & 0x3ff) << 13);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static void q4_0_kernel_sse(const float *x, const uint8_t *raw, int64_t N, int64_t K, float *out) {
  const __m128i mask0f = _mm_set1_epi32(0x0f), sub8 = _mm_set1_epi32(8);
  const __m128i spread[4] = {
      _mm_setr_epi8(0, -1, -1, -1, 1, -1, -1, -1, 2, -1, -1, -1, 3, -1, -1, -1),
      _mm_setr_epi8(4, -1, -1, -1, 5, -1, -1, -1, 6, -1, -1, -1, 7, -1, -1, -1),
      _mm_setr_epi8(8, -1, -1, -1, 9, -1, -1, -1, 10, -1, -1, -1, 11, -1, -1, -1),
      _mm_setr_epi8(12, -1, -1, -1, 13, -1, -1, -1, 14, -1, -1, -1, 15, -1, -1, -1)};
  const int64_t bpr = K >> 5, row_bytes = bpr * 18;
  for (int64_t n = 0; n < N; ++n) {
    __m128 acc = _mm_setzero_ps();
    const uint8_t *row = raw + n * row_bytes;
    for (int64_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = row + b * 18;
      const float scale = f16_wasm((uint16_t)(blk[0] | (blk[1] << 8)));
      const float *xb = x + b * 32;
      const __m128i nib = _mm_loadu_si128((const __m128i *)(blk + 2));
      __m128 ba = _mm_setzero_ps();
      for (int g = 0; g < 4; ++g) {
        const __m128i t = _mm_shuffle_epi8(nib, spread[g]);
        const __m128 lo = _mm_cvtepi32_ps(_mm_sub_epi32(_mm_and_si128(t, mask0f), sub8));
        ba = _mm_add_ps(_mm_mul_ps(lo, _mm_loadu_ps(xb + 4 * g)), ba);
        const __m128 hi = _mm_cvtepi32_ps(_mm_sub_epi32(_mm_srli_epi32(t, 4), sub8));
        ba = _mm_add_ps(_mm_mul_ps(hi, _mm_loadu_ps(xb + 16 + 4 * g)), ba);
      }
      acc = _mm_add_ps(_mm_mul_ps(ba, _mm_set1_ps(scale)), acc);
    }
    const __m128 t = _mm_add_ps(acc, _mm_shuffle_ps(acc, acc, _MM_SHUFFLE(1, 0, 3, 2)));
    const __m128 r = _mm_add_ps(_mm_shuffle_ps(t, t, _MM_SHUFFLE(0, 0, 0, 1)), t);
    out[n] = _mm_cvtss_f32(r);
  }
}

static void batch_dot_sse(const float *x, const float *W, int64_t N, int64_t K, float *out) {
  const int64_t K4 = K & ~(int64_t)3;
  for (int64_t n = 0; n < N; ++n) {
    const float *w = W + n * K;
    __m128 acc = _mm_setzero_ps();
    int64_t k = 0;
    for (; k < K4; k += 4) acc = _mm_add_ps(acc, _mm_mul_ps(_mm_loadu_ps(x + k), _mm_loadu_ps(w + k)));
    const __m128 t = _mm_add_ps(acc, _mm_shuffle_ps(acc, acc, _MM_SHUFFLE(1, 0, 3, 2)));
    const __m128 r = _mm_add_ps(_mm_shuffle_ps(t, t, _MM_SHUFFLE(0, 0, 0, 1)), t);
    float sum = _mm_cvtss_f32(r);
    for (; k < K; ++k) sum = sum + x[k] * w[k];
    out[n] = sum;
  }
}

/* A thread's private "linear memory": x and the raw slice are copied in on
 * every call, as the WASM host wrapper does (wasm-q4.js:735-738). */
typedef struct {
  uint8_t *mem;
  size_t cap;
} linmem;

static void *linmem_need(linmem *m, size_t bytes) {
  if (m->cap < bytes) {
    free(m->mem);
    m->mem = (uint8_t *)aligned_alloc(64, (bytes + 63) & ~(size_t)63);
    m->cap = m->mem ? bytes : 0;
  }
  return m->mem;
}

static void q4_0_matvec_wrapped(linmem *lm, const float *x, const uint8_t *raw, int64_t N,
                                int64_t K, float *out) {
  const size_t xb = (size_t)K * 4, rb = (size_t)N * (K >> 5) * 18;
  const size_t rawp = (xb + 15) & ~(size_t)15, outp = (rawp + rb + 15) & ~(size_t)15;
  uint8_t *mem = (uint8_t *)linmem_need(lm, outp + (size_t)N * 4);
  memcpy(mem, x, xb);
  memcpy(mem + rawp, raw, rb);
  q4_0_kernel_sse((const float *)mem, mem + rawp, N, K, (float *)(mem + outp));
  memcpy(out, mem + outp, (size_t)N * 4);
}

/* Single-call entry: the kernel through its wrapper, one thread. */
void pbo_cpu_q4_0_matvec(const float *x, const uint8_t *raw, int64_t N, int64_t K, float *out) {
  linmem lm = {0, 0};
  q4_0_matvec_wrapped(&lm, x, raw, N, K, out);
  free(lm.mem);
}

/* ---- the pool ---------------------------------------------------------- */
typedef struct pbo_pool pbo_pool;
typedef struct {
  pbo_pool *pool;
  int id;
  linmem lm;
  pthread_t th;
} worker;

struct pbo_pool {
  int nthreads;  /* workers + the caller */
  worker *w;
  pthread_mutex_t mu;
  pthread_cond_t cv_work, cv_done;
  uint64_t gen;
  int pending;
  int shutdown;
  /* the current job */
  const float *x;
  const uint8_t *raw;
  int64_t N, K;
  float *out;
  int64_t start[256], end[256];
  linmem main_lm;
};

static void *worker_main(void *arg) {
  worker *me = (worker *)arg;
  pbo_pool *p = me->pool;
  uint64_t seen = 0;
  for (;;) {
    pthread_mutex_lock(&p->mu);
    while (p->gen == seen && !p->shutdown) pthread_cond_wait(&p->cv_work, &p->mu);
    if (p->shutdown) {
      pthread_mutex_unlock(&p->mu);
      return NULL;
    }
    seen = p->gen;
    const int64_t s = p->start[me->id], e = p->end[me->id];
    pthread_mutex_unlock(&p->mu);
    if (e > s) {
      const int64_t row_bytes = (p->K >> 5) * 18;
      q4_0_matvec_wrapped(&me->lm, p->x, p->raw + s * row_bytes, e - s, p->K, p->out + s);
    }
    pthread_mutex_lock(&p->mu);
    if (--p->pending == 0) pthread_cond_signal(&p->cv_done);
    pthread_mutex_unlock(&p->mu);
  }
}

pbo_pool *pbo_pool_create(int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  pbo_pool *p = (pbo_pool *)calloc(1, sizeof *p);
  p->nthreads = nthreads;
  pthread_mutex_init(&p->mu, NULL);
  pthread_cond_init(&p->cv_work, NULL);
  pthread_cond_init(&p->cv_done, NULL);
  p->w = (worker *)calloc((size_t)nthreads, sizeof(worker));
  for (int i = 0; i < nthreads - 1; ++i) {
    p->w[i].pool = p;
    p->w[i].id = i;
    pthread_create(&p->w[i].th, NULL, worker_main, &p->w[i]);
  }
  return p;
}

void pbo_pool_destroy(pbo_pool *p) {
  if (!p) return;
  pthread_mutex_lock(&p->mu);
  p->shutdown = 1;
  pthread_cond_broadcast(&p->cv_work);
  pthread_mutex_unlock(&p->mu);
  for (int i = 0; i < p->nthreads - 1; ++i) {
    pthread_join(p->w[i].th, NULL);
    free(p->w[i].lm.mem);
  }
  free(p->main_lm.mem);
  free(p->w);
  free(p);
}

/* AtomicsThreadPool.matvec, thread-pool.js:165-246. */
void pbo_pool_q4_0_matvec(pbo_pool *p, const float *x, const uint8_t *raw, int64_t N, int64_t K,
                          float *out) {
  const int active = (int)(p->nthreads < N ? p->nthreads : N);
  const int workers = active - 1;
  const int64_t per = N / active, extra = N % active;
  pthread_mutex_lock(&p->mu);
  p->x = x;
  p->raw = raw;
  p->N = N;
  p->K = K;
  p->out = out;
  int64_t r = 0;
  for (int w = 0; w < p->nthreads - 1; ++w) {
    if (w < workers) {
      const int64_t rows = per + (w < extra ? 1 : 0);
      p->start[w] = r;
      p->end[w] = r + rows;
      r += rows;
    } else {
      p->start[w] = p->end[w] = 0;
    }
  }
  p->pending = p->nthreads - 1;
  p->gen++;
  pthread_cond_broadcast(&p->cv_work);
  pthread_mutex_unlock(&p->mu);
  const int64_t row_bytes = (K >> 5) * 18;
  if (N - r > 0) q4_0_matvec_wrapped(&p->main_lm, x, raw + r * row_bytes, N - r, K, out + r);
  pthread_mutex_lock(&p->mu);
  while (p->pending > 0) pthread_cond_wait(&p->cv_done, &p->mu);
  pthread_mutex_unlock(&p->mu);
}

/* wasmQ4.lmHead, wasm-q4.js:798-839: one thread, 1024-row chunks. */
void pbo_cpu_lm_head(const float *hidden, const float *emb, int64_t vocab, int64_t dim,
                     float *logits) {
  const int64_t CHUNK = 1024;
  const size_t xb = (size_t)dim * 4, wp = (xb + 15) & ~(size_t)15;
  uint8_t *mem = (uint8_t *)aligned_alloc(64, (wp + CHUNK * dim * 4 + CHUNK * 4 + 16 + 63) & ~(size_t)63);
  memcpy(mem, hidden, xb);
  for (int64_t v0 = 0; v0 < vocab; v0 += CHUNK) {
    const int64_t n = (vocab - v0 < CHUNK) ? vocab - v0 : CHUNK;
    const size_t wb = (size_t)n * dim * 4, op = (wp + wb + 15) & ~(size_t)15;
    memcpy(mem + wp, emb + v0 * dim, wb);
    batch_dot_sse((const float *)mem, (const float *)(mem + wp), n, dim, (float *)(mem + op));
    memcpy(logits + v0, mem + op, (size_t)n * 4);
  }
  free(mem);
}
