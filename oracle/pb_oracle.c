/*
 * pb_oracle.c -- TEST INFRASTRUCTURE, NOT PART OF THE PRODUCT.
 *
 * A plain-C restatement of the arithmetic of PureBee's quantized matvec /
 * matmul path (sammcj/purebee, JavaScript), used only by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker.
 * The product (purebee_amd/) never links, loads or calls anything here.
 *
 * Every function names the reference lines it follows.  Where the reference
 * computes in JavaScript numbers (IEEE double) and stores into Float32Array,
 * this file does the same: double temporaries, (float) at the store.  Where
 * the reference runs WebAssembly f32x4 code, this file replays the same f32
 * operations in the same order (compile with -ffp-contract=off so no multiply
 * and add are fused).
 *
 * Parity pins (see tests/test_oracle.py):
 *   - f16 conversions: all 65,536 bit patterns against numpy float16.
 *   - Q4_0 matvec: the reference's own known-answer test, wasm-q4.js:673-704.
 *   - Q4_1 matvec: no reference KAT; pinned by the Q4_0 KAT through the
 *     identity Q4_1(d, m = -8d) == Q4_0(d), by the dequantised product, and
 *     by closed forms on constant blocks.
 *   - f32 matmul: the reference KATs wasm-simd.js:367-385 and main.js:65-74.
 *   - dequant: closed forms (gguf.js:239-286) on every byte value.
 *   - quantizers: ECMAScript Math.round tie cases and invariants.
 *   - the Q4_0 quantizer of the synthetic workload has no producer in the
 *     reference (GGUF Q4_0 files come from llama.cpp, not vendored): its
 *     parity is UNPINNED by the reference; invariants only.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---- fp16 ------------------------------------------------------------ */

/* float16ToFloat32, gguf.js:55-70 (same as f16 in llama-streaming.js:51-61):
 * sign * 2^-14 * frac/1024 for subnormals, +-inf, NaN, normals. */
float pbo_f16_to_f32(uint16_t bits) {
  const int sign = (bits >> 15) & 1;
  const int exp = (bits >> 10) & 0x1f;
  const int frac = bits & 0x3ff;
  double v;
  if (exp == 0) {
    if (frac == 0) return sign ? -0.0f : 0.0f;
    v = ldexp((double)frac / 1024.0, -14);
  } else if (exp == 0x1f) {
    return frac ? NAN : (sign ? -INFINITY : INFINITY);
  } else {
    v = ldexp(1.0 + (double)frac / 1024.0, exp - 15);
  }
  return (float)(sign ? -v : v);
}

/* emitF16toF32, wasm-q4.js:88-109: exp == 0 -> +0 (subnormals flushed);
 * otherwise rebias the exponent by 112 and shift the fraction, which maps
 * exp == 31 (inf/NaN) to the finite value 2^16 * (1 + frac/1024). */
float pbo_f16_to_f32_wasm(uint16_t bits) {
  const uint32_t exp = (bits >> 10) & 0x1f;
  if (exp == 0) return 0.0f;
  const uint32_t u = ((uint32_t)(bits >> 15) << 31) | ((exp + 112u) << 23) |
                     ((uint32_t)(bits & 0x3ff) << 13);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* double -> binary16 bits, round to nearest even (one rounding from the
 * double).  Used by the quantisers to store block scales as fp16. */
uint16_t pbo_f64_to_f16(double v) {
  uint16_t s = 0;
  if (v != v) return 0x7e00;
  if (v < 0 || (v == 0 && 1.0 / v < 0)) {
    s = 0x8000;
    v = -v;
  }
  if (v == 0) return s;
  /* exponent e with 2^e <= v < 2^(e+1) */
  int e = (int)floor(log2(v));
  if (ldexp(1.0, e) > v) e -= 1;
  if (ldexp(1.0, e + 1) <= v) e += 1;
  if (e < -14) {
    /* subnormal grid: multiples of 2^-24 */
    double q = v * 16777216.0, f = floor(q), r = q - f;
    double m = (r > 0.5 || (r == 0.5 && fmod(f, 2.0) != 0.0)) ? f + 1 : f;
    return (uint16_t)(s | (uint16_t)m);
  }
  double q = ldexp(v, 10 - e), f = floor(q), r = q - f; /* q in [1024, 2048) */
  double m = (r > 0.5 || (r == 0.5 && fmod(f, 2.0) != 0.0)) ? f + 1 : f;
  if (m == 2048) {
    m = 1024;
    e += 1;
  }
  if (e > 15) return (uint16_t)(s | 0x7c00);
  return (uint16_t)(s | (uint16_t)((e + 15) << 10) | (uint16_t)((int)m - 1024));
}

/* ECMAScript Math.round: nearest integer, ties toward +infinity. */
static double js_round(double v) {
  const double f = floor(v);
  return (v - f >= 0.5) ? f + 1.0 : f;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---- dequantisation ---------------------------------------------------- */

/* loadTensorData Q4_0 branch, gguf.js:259-286: per 18-byte block, fp16 scale
 * then 16 bytes; element j = (lo nibble of byte j - 8) * scale, element j+16 =
 * (hi nibble - 8) * scale; a short last block is truncated. */
void pbo_dequant_q4_0(const uint8_t *raw, int64_t n, float *out) {
  int64_t o = 0;
  const uint8_t *p = raw;
  while (o < n) {
    const double scale = pbo_f16_to_f32(rd16(p));
    const int64_t remaining = (n - o) < 32 ? (n - o) : 32;
    const int64_t half = remaining < 16 ? remaining : 16;
    for (int64_t j = 0; j < half; ++j) {
      const int byte = p[2 + j];
      out[o + j] = (float)(((byte & 0x0f) - 8) * scale);
      if (j + 16 < remaining) out[o + j + 16] = (float)(((byte >> 4) - 8) * scale);
    }
    o += remaining;
    p += 18;
  }
}

/* loadTensorData Q8_0 branch, gguf.js:239-257: int8 * fp16 scale. */
void pbo_dequant_q8_0(const uint8_t *raw, int64_t n, float *out) {
  int64_t o = 0;
  const uint8_t *p = raw;
  while (o < n) {
    const double scale = pbo_f16_to_f32(rd16(p));
    const int64_t remaining = (n - o) < 32 ? (n - o) : 32;
    for (int64_t i = 0; i < remaining; ++i) out[o + i] = (float)((int8_t)p[2 + i] * scale);
    o += remaining;
    p += 34;
  }
}

/* loadTensorData Q4_1 branch, gguf.js:288-314: per 20-byte block, fp16 d,
 * fp16 m, 16 bytes; element j = lo(byte j) * d + m, element j+16 =
 * hi(byte j) * d + m, each a double expression rounded once to f32. */
void pbo_dequant_q4_1(const uint8_t *raw, int64_t n, float *out) {
  int64_t o = 0;
  const uint8_t *p = raw;
  while (o < n) {
    const double d = pbo_f16_to_f32(rd16(p));
    const double m = pbo_f16_to_f32(rd16(p + 2));
    const int64_t remaining = (n - o) < 32 ? (n - o) : 32;
    const int64_t half = remaining < 16 ? remaining : 16;
    for (int64_t j = 0; j < half; ++j) {
      const int byte = p[4 + j];
      out[o + j] = (float)((byte & 0x0f) * d + m);
      if (j + 16 < remaining) out[o + j + 16] = (float)((byte >> 4) * d + m);
    }
    o += remaining;
    p += 20;
  }
}

/* loadTensorData F16 branch, gguf.js:231-237. */
void pbo_dequant_f16(const uint8_t *raw, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = pbo_f16_to_f32(rd16(raw + 2 * i));
}

/* loadTensorData Q6_K branch, gguf.js:317-364: 210-byte blocks of 256 values
 * (ql[128], qh[64], int8 scales[16], fp16 d).  For half h and l < 32, with
 * the scale index is = 8h + l/16:
 *   out[128h + l]      = d * sc[is]     * ((ql[64h+l]    & 15 | (qh[32h+l]      & 3) << 4) - 32)
 *   out[128h + l + 32] = d * sc[is + 2] * ((ql[64h+l+32] & 15 | (qh[32h+l] >> 2 & 3) << 4) - 32)
 *   out[128h + l + 64] = d * sc[is + 4] * ((ql[64h+l]   >> 4 | (qh[32h+l] >> 4 & 3) << 4) - 32)
 *   out[128h + l + 96] = d * sc[is + 6] * ((ql[64h+l+32] >> 4 | (qh[32h+l] >> 6 & 3) << 4) - 32)
 * each a double product rounded once; outputs past n are dropped. */
void pbo_dequant_q6_k(const uint8_t *raw, int64_t n, float *out) {
  const int64_t nb = (n + 255) / 256;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t *blk = raw + b * 210;
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    const double d = pbo_f16_to_f32(rd16(blk + 208));
    for (int h = 0; h < 2; ++h)
      for (int l = 0; l < 32; ++l) {
        const int is = h * 8 + l / 16;
        const int a = ql[h * 64 + l], c = ql[h * 64 + l + 32], hb = qh[h * 32 + l];
        const int q[4] = {((a & 15) | ((hb & 3) << 4)) - 32, ((c & 15) | (((hb >> 2) & 3) << 4)) - 32,
                          ((a >> 4) | (((hb >> 4) & 3) << 4)) - 32, ((c >> 4) | (((hb >> 6) & 3) << 4)) - 32};
        for (int k = 0; k < 4; ++k) {
          const int64_t idx = b * 256 + h * 128 + l + 32 * k;
          if (idx < n) out[idx] = (float)(d * sc[is + 2 * k] * q[k]);
        }
      }
  }
}

/* dequantize_q8, quantize.js:170-181: out[i] = q[i] * scales[floor(i/32)]. */
void pbo_dequant_q8_ref(const int8_t *q, const float *scales, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = (float)((double)q[i] * (double)scales[i / 32]);
}

/* ---- matvecs ----------------------------------------------------------- */

/* q4_0_matvec JS version, llama-streaming.js:72-104: double accumulation,
 * lo and hi terms of byte j interleaved, block sum times scale, f32 store. */
void pbo_q4_0_matvec_js(const float *x, const uint8_t *raw, int64_t N, int64_t K, float *out) {
  const int64_t bpr = K / 32, row_bytes = bpr * 18;
  for (int64_t n = 0; n < N; ++n) {
    double sum = 0;
    const uint8_t *row = raw + n * row_bytes;
    for (int64_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = row + b * 18;
      const double scale = pbo_f16_to_f32(rd16(blk));
      const float *xb = x + b * 32;
      double bs = 0;
      for (int j = 0; j < 16; ++j) {
        const int byte = blk[2 + j];
        bs += (double)xb[j] * ((byte & 0x0f) - 8);
        bs += (double)xb[j + 16] * ((byte >> 4) - 8);
      }
      sum += bs * scale;
    }
    out[n] = (float)sum;
  }
}

/* q4_0_matvec WebAssembly kernel, wasm-q4.js:118-267, replayed lane by lane
 * in f32: four lanes; for byte groups g = 0,4,8,12 lane i adds
 * (lo(g+i) - 8) * x[g+i] then (hi(g+i) - 8) * x[g+16+i] (multiply, then add);
 * acc += blockAcc * scale per block; horizontal sum (a1+a3) + (a0+a2). */
void pbo_q4_0_matvec_wasm(const float *x, const uint8_t *raw, int64_t N, int64_t K, float *out) {
  const int64_t bpr = K >> 5, row_bytes = bpr * 18;
  for (int64_t n = 0; n < N; ++n) {
    float acc[4] = {0, 0, 0, 0};
    const uint8_t *row = raw + n * row_bytes;
    for (int64_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = row + b * 18;
      const float scale = pbo_f16_to_f32_wasm(rd16(blk));
      const float *xb = x + b * 32;
      float ba[4] = {0, 0, 0, 0};
      for (int g = 0; g < 16; g += 4)
        for (int i = 0; i < 4; ++i) {
          const int byte = blk[2 + g + i];
          const float lo = (float)((byte & 0x0f) - 8);
          const float hi = (float)((byte >> 4) - 8);
          float t = lo * xb[g + i];
          ba[i] = t + ba[i];
          t = hi * xb[g + 16 + i];
          ba[i] = t + ba[i];
        }
      for (int i = 0; i < 4; ++i) {
        const float t = ba[i] * scale;
        acc[i] = t + acc[i];
      }
    }
    const float t0 = acc[0] + acc[2], t1 = acc[1] + acc[3];
    out[n] = t1 + t0;
  }
}

/* q4_1_matvec JS version, llama-streaming.js:115-151: per block, in double,
 * nibbleSum += x[j]*lo(j) then += x[j+16]*hi(j); xBlockSum += (x[j] +
 * x[j+16]); sum += delta*nibbleSum + min*xBlockSum; f32 store. */
void pbo_q4_1_matvec_js(const float *x, const uint8_t *raw, int64_t N, int64_t K, float *out) {
  const int64_t bpr = K >> 5, row_bytes = bpr * 20;
  for (int64_t n = 0; n < N; ++n) {
    double sum = 0;
    const uint8_t *row = raw + n * row_bytes;
    for (int64_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = row + b * 20;
      const double delta = pbo_f16_to_f32(rd16(blk));
      const double mn = pbo_f16_to_f32(rd16(blk + 2));
      const float *xb = x + b * 32;
      double nib_sum = 0, x_sum = 0;
      for (int j = 0; j < 16; ++j) {
        const int byte = blk[4 + j];
        nib_sum += (double)xb[j] * (byte & 0x0f);
        nib_sum += (double)xb[j + 16] * (byte >> 4);
        x_sum += (double)xb[j] + (double)xb[j + 16];
      }
      sum += delta * nib_sum + mn * x_sum;
    }
    out[n] = (float)sum;
  }
}

/* q4_1_matvec WebAssembly kernel, wasm-q4.js:275-435, replayed lane by lane
 * in f32: for byte groups g = 0,4,8,12 lane i adds lo(g+i) * x[g+i] to its
 * nibble accumulator and x[g+i] to its x accumulator, then the same for
 * hi(g+i) and x[g+16+i]; per block acc += (nib*delta + xs*min); horizontal
 * sum (a1+a3) + (a0+a2).  delta and min use the WASM f16 decode. */
void pbo_q4_1_matvec_wasm(const float *x, const uint8_t *raw, int64_t N, int64_t K, float *out) {
  const int64_t bpr = K >> 5, row_bytes = bpr * 20;
  for (int64_t n = 0; n < N; ++n) {
    float acc[4] = {0, 0, 0, 0};
    const uint8_t *row = raw + n * row_bytes;
    for (int64_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = row + b * 20;
      const float delta = pbo_f16_to_f32_wasm(rd16(blk));
      const float mn = pbo_f16_to_f32_wasm(rd16(blk + 2));
      const float *xb = x + b * 32;
      float na[4] = {0, 0, 0, 0}, xa[4] = {0, 0, 0, 0};
      for (int g = 0; g < 16; g += 4)
        for (int i = 0; i < 4; ++i) {
          const int byte = blk[4 + g + i];
          float t = (float)(byte & 0x0f) * xb[g + i];
          na[i] = t + na[i];
          xa[i] = xa[i] + xb[g + i];
          t = (float)(byte >> 4) * xb[g + 16 + i];
          na[i] = t + na[i];
          xa[i] = xa[i] + xb[g + 16 + i];
        }
      for (int i = 0; i < 4; ++i) {
        const float t1 = na[i] * delta, t2 = xa[i] * mn;
        const float t = t1 + t2;
        acc[i] = t + acc[i];
      }
    }
    const float t0 = acc[0] + acc[2], t1 = acc[1] + acc[3];
    out[n] = t1 + t0;
  }
}

/* GGUF Q8_0 through the reference's own route for Q8_0 files: dequantise
 * (gguf.js:239-257) then the f32 matvec; accumulated here in double. */
void pbo_q8_0_matvec_f64(const float *x, const uint8_t *raw, int64_t N, int64_t K, float *out) {
  const int64_t bpr = K / 32, row_bytes = bpr * 34;
  for (int64_t n = 0; n < N; ++n) {
    double sum = 0;
    const uint8_t *row = raw + n * row_bytes;
    for (int64_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = row + b * 34;
      const double scale = pbo_f16_to_f32(rd16(blk));
      for (int j = 0; j < 32; ++j) sum += (double)x[b * 32 + j] * (double)(float)((int8_t)blk[2 + j] * scale);
    }
    out[n] = (float)sum;
  }
}

/* LM head of llama.js:359-367 (and the JS fallback of _computeLogits,
 * llama-streaming.js:665-675): logits[v] = sum_d h[d] * E[v,d], double. */
void pbo_f32_matvec_f64(const float *x, const float *W, int64_t N, int64_t K, float *out) {
  for (int64_t n = 0; n < N; ++n) {
    double s = 0;
    const float *w = W + n * K;
    for (int64_t k = 0; k < K; ++k) s += (double)x[k] * (double)w[k];
    out[n] = (float)s;
  }
}

/* batch_dot WebAssembly kernel, wasm-q4.js:447-566 (lmHead, 798-839): four
 * f32 lanes over k in steps of 4 (acc += x*w), horizontal (a1+a3)+(a0+a2),
 * then a scalar f32 tail for K % 4. */
void pbo_batch_dot_wasm(const float *x, const float *W, int64_t N, int64_t K, float *out) {
  const int64_t K4 = K & ~(int64_t)3;
  for (int64_t n = 0; n < N; ++n) {
    const float *w = W + n * K;
    float a[4] = {0, 0, 0, 0};
    int64_t k = 0;
    for (; k < K4; k += 4)
      for (int i = 0; i < 4; ++i) {
        const float t = x[k + i] * w[k + i];
        a[i] = a[i] + t;
      }
    const float t0 = a[0] + a[2], t1 = a[1] + a[3];
    float sum = t1 + t0;
    for (; k < K; ++k) {
      const float t = x[k] * w[k];
      sum = sum + t;
    }
    out[n] = sum;
  }
}

/* matmul of wasm-simd.js:94-329 as driven by matmulCached (469-506):
 * C starts at bias (or 0) and C[m,n] += A[m,k] * B[k,n] in f32, k ascending,
 * multiply then add.  B is [K,N] (the reference's transposed convention). */
void pbo_matmul_f32_axpy(const float *A, int64_t M, int64_t K, const float *B, int64_t N,
                         const float *bias, float *C) {
  for (int64_t m = 0; m < M; ++m) {
    float *c = C + m * N;
    for (int64_t n = 0; n < N; ++n) c[n] = bias ? bias[n] : 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float a = A[m * K + k];
      const float *b = B + k * N;
      for (int64_t n = 0; n < N; ++n) {
        const float t = a * b[n];
        c[n] = c[n] + t;
      }
    }
  }
}

/* matmul_q8, quantize.js:224-266: out starts at bias or 0; loop m, k (skip
 * a == 0), 32-wide column groups using the scale of the flat block holding
 * the group's first element; aScaled = a * scale and each += in double,
 * rounded into the Float32Array output. */
void pbo_matmul_q8_ref(const float *a, int64_t M, int64_t K, const int8_t *q,
                       const float *scales, int64_t N, const float *bias, float *out) {
  const int64_t bpr = (N + 31) / 32;
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) out[m * N + n] = bias ? bias[n] : 0.0f;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t k = 0; k < K; ++k) {
      const double av = a[m * K + k];
      if (av == 0) continue;
      const int64_t roff = k * N;
      for (int64_t bn = 0; bn < bpr; ++bn) {
        const int64_t n0 = bn * 32, n1 = (n0 + 32 < N) ? n0 + 32 : N;
        const double as = av * (double)scales[(roff + n0) / 32];
        for (int64_t n = n0; n < n1; ++n) {
          const double prod = as * (double)q[roff + n];
          out[m * N + n] = (float)((double)out[m * N + n] + prod);
        }
      }
    }
  }
}

/* ---- quantisers -------------------------------------------------------- */

/* quantize_q8, quantize.js:79-109: per flat 32-block, maxAbs, scale =
 * maxAbs/127 stored as f32, q = Math.round(x * (127/maxAbs)) in double. */
void pbo_quantize_q8_ref(const float *w, int64_t n, int8_t *q, float *scales) {
  const int64_t nb = (n + 31) / 32;
  for (int64_t b = 0; b < nb; ++b) {
    const int64_t lo = b * 32, hi = (lo + 32 < n) ? lo + 32 : n;
    double mx = 0;
    for (int64_t i = lo; i < hi; ++i) {
      const double a = fabs((double)w[i]);
      if (a > mx) mx = a;
    }
    const double scale = mx / 127;
    scales[b] = (float)scale;
    for (int64_t i = lo; i < hi; ++i) q[i] = 0;
    if (scale > 0) {
      const double inv = 127 / mx;
      for (int64_t i = lo; i < hi; ++i) q[i] = (int8_t)js_round((double)w[i] * inv);
    }
  }
}

/* GGUF Q8_0 bytes with quantize_q8's numerics (quantize.js:79-109) applied
 * per 32-block along K of each of the N rows; the block scale maxAbs/127 is
 * stored as fp16 (rounded once from the double). */
void pbo_quantize_q8_0(const float *w, int64_t N, int64_t K, uint8_t *raw) {
  const int64_t nb = N * (K / 32);
  for (int64_t b = 0; b < nb; ++b) {
    const float *x = w + b * 32;
    uint8_t *o = raw + b * 34;
    double mx = 0;
    for (int i = 0; i < 32; ++i)
      if (fabs((double)x[i]) > mx) mx = fabs((double)x[i]);
    const double scale = mx / 127;
    const uint16_t h = pbo_f64_to_f16(scale);
    o[0] = (uint8_t)h;
    o[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; ++i)
      o[2 + i] = scale > 0 ? (uint8_t)(int8_t)js_round((double)x[i] * (127 / mx)) : 0;
  }
}

/* Q4_0 of the synthetic workload (d = absmax/8 as fp16, nibble =
 * clamp(Math.round(x*8/absmax), -8, 7) + 8, GGUF nibble order of
 * gguf.js:259-286).  No reference producer exists: parity unpinned. */
void pbo_quantize_q4_0(const float *w, int64_t N, int64_t K, uint8_t *raw) {
  const int64_t nb = N * (K / 32);
  for (int64_t b = 0; b < nb; ++b) {
    const float *x = w + b * 32;
    uint8_t *o = raw + b * 18;
    double mx = 0;
    for (int i = 0; i < 32; ++i)
      if (fabs((double)x[i]) > mx) mx = fabs((double)x[i]);
    const uint16_t h = pbo_f64_to_f16(mx / 8);
    o[0] = (uint8_t)h;
    o[1] = (uint8_t)(h >> 8);
    int nib[32];
    for (int i = 0; i < 32; ++i) {
      double r = mx > 0 ? js_round((double)x[i] * (8 / mx)) : 0;
      if (r < -8) r = -8;
      if (r > 7) r = 7;
      nib[i] = (int)r + 8;
    }
    for (int j = 0; j < 16; ++j) o[2 + j] = (uint8_t)(nib[j] | (nib[j + 16] << 4));
  }
}

/* Q4_1 of synthetic workloads (no producer in the reference: parity
 * unpinned, invariants only): per block d = (max - min)/15 and m = min, both
 * stored as fp16; nibble = clamp(Math.round((x - m16) / d16), 0, 15) with
 * the stored values, so the rounding sees the scale the reader will use. */
void pbo_quantize_q4_1(const float *w, int64_t N, int64_t K, uint8_t *raw) {
  const int64_t nb = N * (K / 32);
  for (int64_t b = 0; b < nb; ++b) {
    const float *x = w + b * 32;
    uint8_t *o = raw + b * 20;
    double lo = x[0], hi = x[0];
    for (int i = 1; i < 32; ++i) {
      if (x[i] < lo) lo = x[i];
      if (x[i] > hi) hi = x[i];
    }
    const uint16_t hd = pbo_f64_to_f16((hi - lo) / 15);
    const uint16_t hm = pbo_f64_to_f16(lo);
    o[0] = (uint8_t)hd;
    o[1] = (uint8_t)(hd >> 8);
    o[2] = (uint8_t)hm;
    o[3] = (uint8_t)(hm >> 8);
    const double d = pbo_f16_to_f32(hd), m = pbo_f16_to_f32(hm);
    int nib[32];
    for (int i = 0; i < 32; ++i) {
      double r = d > 0 ? js_round(((double)x[i] - m) / d) : 0;
      if (r < 0) r = 0;
      if (r > 15) r = 15;
      nib[i] = (int)r;
    }
    for (int j = 0; j < 16; ++j) o[4 + j] = (uint8_t)(nib[j] | (nib[j + 16] << 4));
  }
}

/* Q6_K of synthetic workloads (no producer in the reference: parity
 * unpinned, invariants only).  Per 16-element sub-block s of a 256-block,
 * the ideal scale a_s = absmax_s / 31; d = max_s |a_s| / 127 as fp16;
 * sc_s = Math.round(a_s / d) (int8); q = clamp(Math.round(x / (d * sc_s)),
 * -32, 31) + 32 against the stored d, packed in the layout of
 * pbo_dequant_q6_k. */
void pbo_quantize_q6_k(const float *w, int64_t N, int64_t K, uint8_t *raw) {
  const int64_t nb = N * (K / 256);
  for (int64_t b = 0; b < nb; ++b) {
    const float *x = w + b * 256;
    uint8_t *o = raw + b * 210;
    memset(o, 0, 210);
    double a[16], amax = 0;
    for (int s = 0; s < 16; ++s) {
      double m = 0;
      for (int i = 0; i < 16; ++i)
        if (fabs((double)x[16 * s + i]) > m) m = fabs((double)x[16 * s + i]);
      a[s] = m / 31;
      if (a[s] > amax) amax = a[s];
    }
    const uint16_t hd = pbo_f64_to_f16(amax / 127);
    o[208] = (uint8_t)hd;
    o[209] = (uint8_t)(hd >> 8);
    const double d = pbo_f16_to_f32(hd);
    for (int s = 0; s < 16; ++s) {
      double sc = d > 0 ? js_round(a[s] / d) : 0;
      if (sc > 127) sc = 127;
      o[192 + s] = (uint8_t)(int8_t)sc;
      const double step = d * sc;
      for (int i = 0; i < 16; ++i) {
        const int e = 16 * s + i;
        double r = step > 0 ? js_round((double)x[e] / step) : 0;
        if (r < -32) r = -32;
        if (r > 31) r = 31;
        const int q = (int)r + 32;
        const int h = e / 128, g = (e % 128) / 32, l = e % 32;
        o[h * 64 + (g & 1) * 32 + l] |= (uint8_t)((q & 15) << (4 * (g >> 1)));
        o[128 + h * 32 + l] |= (uint8_t)(((q >> 4) & 3) << (2 * g));
      }
    }
  }
}

/* ---- synthetic inputs -------------------------------------------------- */

static uint64_t sm64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Element i of stream `seed`: SplitMix64 counters -> Box-Muller (double)
 * -> (float)(mean + std*z); pairs (2p, 2p+1) share one draw. */
void pbo_synth_normal(uint64_t seed, int64_t n, double mean, double std, float *out) {
  const uint64_t base = sm64(seed);
  for (int64_t p = 0; 2 * p < n; ++p) {
    const double u1 = ((double)(sm64(base + 2 * (uint64_t)p) >> 11) + 1.0) / 9007199254740992.0;
    const double u2 = (double)(sm64(base + 2 * (uint64_t)p + 1) >> 11) / 9007199254740992.0;
    const double r = sqrt(-2.0 * log(u1));
    const double ang = 6.283185307179586476925286766559 * u2;
    out[2 * p] = (float)(mean + std * r * cos(ang));
    if (2 * p + 1 < n) out[2 * p + 1] = (float)(mean + std * r * sin(ang));
  }
}
