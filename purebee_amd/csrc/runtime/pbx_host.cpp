// pbx_host.cpp -- CPU-side parts of the C ABI: quantisers and the seeded
// synthetic-data generator.  No HIP calls.

#include <math.h>
#include <string.h>

#include <algorithm>

#include "pbx_internal.h"

namespace {

// ECMAScript Math.round: the integer closest to v, ties toward +infinity.
// floor(v + 0.5) is wrong for v = 0.49999999999999994, so take the floor
// and compare the (exact) remainder instead.
inline double js_round(double v) {
  const double r = floor(v);
  return (v - r >= 0.5) ? r + 1.0 : r;
}

// double -> IEEE binary16 bits, round to nearest even, with subnormals,
// overflow to infinity and NaN.
uint16_t f64_to_f16_bits(double v) {
  uint16_t sign = 0;
  if (signbit(v)) {
    sign = 0x8000;
    v = -v;
  }
  if (isnan(v)) return 0x7E00;
  if (v >= 65520.0) return sign | 0x7C00;  // rounds past the largest finite half
  if (v == 0.0) return sign;
  int e;
  frexp(v, &e);       // v = m * 2^e, m in [0.5, 1)
  int exp16 = e - 1;  // v in [2^exp16, 2^(exp16+1))
  if (exp16 < -14) {
    // subnormal: units of 2^-24
    double q = v * 16777216.0;  // exact scaling by 2^24
    double r = nearbyint(q);    // round-half-even under the default mode
    return sign | (uint16_t)r;  // r == 1024 gives the smallest normal, as it should
  }
  double scaled = ldexp(v, 10 - exp16);  // in [1024, 2048)
  double r = nearbyint(scaled);
  int mant = (int)r;
  if (mant == 2048) {
    mant = 1024;
    exp16 += 1;
    if (exp16 > 15) return sign | 0x7C00;
  }
  return sign | (uint16_t)((exp16 + 15) << 10) | (uint16_t)(mant - 1024);
}

inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// binary16 bits -> double (finite values only; the quantisers never store
// inf or NaN for finite inputs below 65504).
double f16_bits_to_f64(uint16_t h) {
  const int e = (h >> 10) & 0x1f, f = h & 0x3ff;
  const double v = e == 0 ? ldexp((double)f, -24) : ldexp(1024.0 + f, e - 25);
  return (h & 0x8000) ? -v : v;
}

}  // namespace

extern "C" int pbx_quantize_q8_0(const float *w, int64_t N, int64_t K, uint8_t *out) {
  if (!w || !out || N <= 0 || K <= 0 || K % 32 != 0)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_quantize_q8_0: bad arguments (N=%lld K=%lld)",
                    (long long)N, (long long)K);
  const int64_t blocks = N * (K / 32);
#pragma omp parallel for schedule(static)
  for (int64_t blk = 0; blk < blocks; ++blk) {
    const float *x = w + blk * 32;
    uint8_t *dst = out + blk * 34;
    double max_abs = 0.0;
    for (int i = 0; i < 32; ++i) max_abs = std::max(max_abs, fabs((double)x[i]));
    const double scale = max_abs / 127.0;
    const uint16_t d = f64_to_f16_bits(scale);
    dst[0] = (uint8_t)(d & 0xFF);
    dst[1] = (uint8_t)(d >> 8);
    if (scale > 0) {
      const double inv = 127.0 / max_abs;
      for (int i = 0; i < 32; ++i) dst[2 + i] = (uint8_t)(int8_t)js_round((double)x[i] * inv);
    } else {
      memset(dst + 2, 0, 32);
    }
  }
  return PBX_OK;
}

extern "C" int pbx_quantize_q4_0(const float *w, int64_t N, int64_t K, uint8_t *out) {
  if (!w || !out || N <= 0 || K <= 0 || K % 32 != 0)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_quantize_q4_0: bad arguments (N=%lld K=%lld)",
                    (long long)N, (long long)K);
  const int64_t blocks = N * (K / 32);
#pragma omp parallel for schedule(static)
  for (int64_t blk = 0; blk < blocks; ++blk) {
    const float *x = w + blk * 32;
    uint8_t *dst = out + blk * 18;
    double max_abs = 0.0;
    for (int i = 0; i < 32; ++i) max_abs = std::max(max_abs, fabs((double)x[i]));
    const uint16_t d = f64_to_f16_bits(max_abs / 8.0);
    dst[0] = (uint8_t)(d & 0xFF);
    dst[1] = (uint8_t)(d >> 8);
    int q[32];
    if (max_abs > 0) {
      const double inv = 8.0 / max_abs;
      for (int i = 0; i < 32; ++i) {
        double r = js_round((double)x[i] * inv);
        r = std::min(7.0, std::max(-8.0, r));
        q[i] = (int)r + 8;
      }
    } else {
      for (int i = 0; i < 32; ++i) q[i] = 8;
    }
    for (int j = 0; j < 16; ++j) dst[2 + j] = (uint8_t)((q[j] & 0xF) | ((q[j + 16] & 0xF) << 4));
  }
  return PBX_OK;
}

extern "C" int pbx_quantize_q4_1(const float *w, int64_t N, int64_t K, uint8_t *out) {
  if (!w || !out || N <= 0 || K <= 0 || K % 32 != 0)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_quantize_q4_1: bad arguments (N=%lld K=%lld)",
                    (long long)N, (long long)K);
  const int64_t blocks = N * (K / 32);
#pragma omp parallel for schedule(static)
  for (int64_t blk = 0; blk < blocks; ++blk) {
    const float *x = w + blk * 32;
    uint8_t *dst = out + blk * 20;
    double lo = x[0], hi = x[0];
    for (int i = 1; i < 32; ++i) {
      lo = std::min(lo, (double)x[i]);
      hi = std::max(hi, (double)x[i]);
    }
    const uint16_t hd = f64_to_f16_bits((hi - lo) / 15.0);
    const uint16_t hm = f64_to_f16_bits(lo);
    dst[0] = (uint8_t)(hd & 0xFF);
    dst[1] = (uint8_t)(hd >> 8);
    dst[2] = (uint8_t)(hm & 0xFF);
    dst[3] = (uint8_t)(hm >> 8);
    const double d = f16_bits_to_f64(hd), m = f16_bits_to_f64(hm);
    int q[32];
    for (int i = 0; i < 32; ++i) {
      const double r = d > 0 ? js_round(((double)x[i] - m) / d) : 0.0;
      q[i] = (int)std::min(15.0, std::max(0.0, r));
    }
    for (int j = 0; j < 16; ++j) dst[4 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
  }
  return PBX_OK;
}

extern "C" int pbx_quantize_q6_k(const float *w, int64_t N, int64_t K, uint8_t *out) {
  if (!w || !out || N <= 0 || K <= 0 || K % 256 != 0)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_quantize_q6_k: bad arguments (N=%lld K=%lld)",
                    (long long)N, (long long)K);
  const int64_t blocks = N * (K / 256);
#pragma omp parallel for schedule(static)
  for (int64_t blk = 0; blk < blocks; ++blk) {
    const float *x = w + blk * 256;
    uint8_t *dst = out + blk * 210;
    memset(dst, 0, 210);
    double ideal[16], top = 0.0;
    for (int s = 0; s < 16; ++s) {
      double m = 0.0;
      for (int i = 0; i < 16; ++i) m = std::max(m, fabs((double)x[16 * s + i]));
      ideal[s] = m / 31.0;
      top = std::max(top, ideal[s]);
    }
    const uint16_t hd = f64_to_f16_bits(top / 127.0);
    dst[208] = (uint8_t)(hd & 0xFF);
    dst[209] = (uint8_t)(hd >> 8);
    const double d = f16_bits_to_f64(hd);
    for (int s = 0; s < 16; ++s) {
      const double sc = d > 0 ? std::min(127.0, js_round(ideal[s] / d)) : 0.0;
      dst[192 + s] = (uint8_t)(int8_t)sc;
      const double step = d * sc;
      for (int i = 0; i < 16; ++i) {
        const int e = 16 * s + i;
        const double r = step > 0 ? js_round((double)x[e] / step) : 0.0;
        const int q = (int)std::min(31.0, std::max(-32.0, r)) + 32;
        // element e = 128*half + 32*g + l: low nibble in ql[64*half + 32*(g&1) + l]
        // (high nibble for g >= 2), top two bits in qh[32*half + l] at 2*g
        const int half = e / 128, g = (e % 128) / 32, l = e % 32;
        dst[half * 64 + (g & 1) * 32 + l] |= (uint8_t)((q & 15) << (4 * (g >> 1)));
        dst[128 + half * 32 + l] |= (uint8_t)(((q >> 4) & 3) << (2 * g));
      }
    }
  }
  return PBX_OK;
}

extern "C" int pbx_quantize_q8_ref(const float *w, int64_t n, int8_t *q, float *scales) {
  if (!w || !q || !scales || n <= 0)
    return pbx_fail(nullptr, PBX_EINVAL, "pbx_quantize_q8_ref: bad arguments");
  const int64_t blocks = (n + 31) / 32;
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < blocks; ++b) {
    const int64_t lo = b * 32, hi = std::min(n, lo + 32);
    double max_abs = 0.0;
    for (int64_t i = lo; i < hi; ++i) max_abs = std::max(max_abs, fabs((double)w[i]));
    const double scale = max_abs / 127.0;
    scales[b] = (float)scale;
    if (scale > 0) {
      const double inv = 127.0 / max_abs;
      for (int64_t i = lo; i < hi; ++i) q[i] = (int8_t)js_round((double)w[i] * inv);
    } else {
      for (int64_t i = lo; i < hi; ++i) q[i] = 0;
    }
  }
  return PBX_OK;
}

extern "C" int pbx_synth_normal(uint64_t seed, int64_t n, double mean, double std,
                                float *out) {
  if (!out || n < 0) return pbx_fail(nullptr, PBX_EINVAL, "pbx_synth_normal: bad arguments");
  const uint64_t base = splitmix64(seed);
  const int64_t pairs = (n + 1) / 2;
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < pairs; ++p) {
    const uint64_t a = splitmix64(base + 2 * (uint64_t)p);
    const uint64_t b = splitmix64(base + 2 * (uint64_t)p + 1);
    const double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53;  // (0, 1]
    const double u2 = (double)(b >> 11) * 0x1.0p-53;          // [0, 1)
    const double r = sqrt(-2.0 * log(u1));
    out[2 * p] = (float)(mean + std * r * cos(two_pi * u2));
    if (2 * p + 1 < n) out[2 * p + 1] = (float)(mean + std * r * sin(two_pi * u2));
  }
  return PBX_OK;
}
