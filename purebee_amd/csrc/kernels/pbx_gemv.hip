// pbx_gemv.hip -- gfx950 kernels for PureBee's quantized matvec instruction:
// weight repack, exact dequantisation and the M=1 GEMV family.
//
// Built with `hipcc --genco --offload-arch=gfx950` into pbx_gemv.hsaco and
// loaded by the runtime with hipModuleLoad; every kernel is extern "C" so the
// runtime can look it up by name with hipModuleGetFunction.
//
// Device layout of a resident weight (N rows, K columns, B = K/32 blocks/row,
// Npad = N rounded up to 64 so row tiles never need a load guard):
//   Q4_0 : qs plane  [Npad][B][16] bytes   (the 16 nibble bytes of each block)
//          d  plane  [Npad/4][B][4] fp16   (4 rows' scales of one block are
//                                           contiguous: one 8-B load serves
//                                           a 4-row group)
//   Q8_0 : qs plane  [Npad][B][32] int8, d plane as Q4_0
//   Q4_1 : qs plane as Q4_0; d plane as Q4_0 and an m plane of the same
//          layout (fp16 minima), value = nibble * d + m
//   F32  : plane     [Npad][K] float
//   F16  : plane     [Npad][K] fp16
//   Q6_K : qs plane  [Npad][K/256][208] bytes (ql, qh, int8 scales of each
//          256-element super-block) and a d plane [Npad/4][K/256][4] fp16
// The GGUF block formats these come from are gguf.js:36-49 (sizes) and
// gguf.js:239-286 (element order: Q4_0 byte j holds element j in its low
// nibble and element j+16 in its high nibble; value = (nibble - 8) * d;
// Q4_1 is gguf.js:288-314: 20-byte blocks, fp16 d, fp16 m, the same nibbles).

#include "pbx_gemv_impl.h"

// ---------------------------------------------------------------------------
// Exported kernels.
// ---------------------------------------------------------------------------
using namespace pbx;

__device__ __forceinline__ GemvArgs plain_args(const uint8_t *qs, const uint16_t *dsc,
                                               const uint16_t *msc, const float *X,
                                               const float *bias, float *Y, int N, int B) {
  GemvArgs a;
  a.qs = qs; a.dsc = dsc; a.X = X; a.X2 = nullptr; a.normw = nullptr;
  a.bias = bias; a.Y = Y; a.partials = nullptr; a.N = N; a.B = B; a.eps = 0.f;
  a.msc = msc;
  return a;
}

#define PBX_WIDE(NAME, TYPE, R)                                               \
  extern "C" __global__ void __launch_bounds__(512)                           \
  NAME(const uint8_t *qs, const uint16_t *dsc, const uint16_t *msc,          \
       const float *X, const float *bias, float *Y, int N, int B) {           \
    gemv_wide<TYPE, R, PRO_NONE, EPI_STORE>(plain_args(qs, dsc, msc, X, bias, Y, N, B)); \
  }
PBX_WIDE(pbx_gemv_q4_0_wide_r4, PBX_Q4, 4)
PBX_WIDE(pbx_gemv_q4_0_wide_r8, PBX_Q4, 8)
PBX_WIDE(pbx_gemv_q4_0_wide_r16, PBX_Q4, 16)
PBX_WIDE(pbx_gemv_q4_1_wide_r4, PBX_Q41, 4)
PBX_WIDE(pbx_gemv_q4_1_wide_r8, PBX_Q41, 8)
PBX_WIDE(pbx_gemv_q4_1_wide_r16, PBX_Q41, 16)
PBX_WIDE(pbx_gemv_q8_0_wide_r4, PBX_Q8, 4)
PBX_WIDE(pbx_gemv_q8_0_wide_r8, PBX_Q8, 8)
PBX_WIDE(pbx_gemv_f16_wide_r4, PBX_F16, 4)
PBX_WIDE(pbx_gemv_f16_wide_r8, PBX_F16, 8)
PBX_WIDE(pbx_gemv_q6_k_wide_r4, PBX_Q6K, 4)
PBX_WIDE(pbx_gemv_q6_k_wide_r8, PBX_Q6K, 8)
PBX_WIDE(pbx_gemv_f32_wide_r2, PBX_F32, 2)
PBX_WIDE(pbx_gemv_f32_wide_r4, PBX_F32, 4)

#define PBX_SMALL(NAME, TYPE, P)                                              \
  extern "C" __global__ void __launch_bounds__(256)                           \
  NAME(const uint8_t *qs, const uint16_t *dsc, const uint16_t *msc,          \
       const float *X, const float *bias, float *Y, int N, int B) {           \
    gemv_small<TYPE, P, PRO_NONE, EPI_STORE>(plain_args(qs, dsc, msc, X, bias, Y, N, B)); \
  }
PBX_SMALL(pbx_gemv_q4_0_small, PBX_Q4, 8)
PBX_SMALL(pbx_gemv_q4_1_small, PBX_Q41, 8)
PBX_SMALL(pbx_gemv_q8_0_small, PBX_Q8, 4)
PBX_SMALL(pbx_gemv_f32_small, PBX_F32, 2)
PBX_SMALL(pbx_gemv_f16_small, PBX_F16, 4)
PBX_SMALL(pbx_gemv_q6_k_small, PBX_Q6K, 4)

// Integer-limb GEMVs (Q4_0 / Q8_0, K = 2048..8192; pbx_gemv_impl.h) for the
// instruction, launched with a GemvArgs block (X, bias, Y, N, B, the weight
// planes; grid y = activation rows).  Name: pbx_gemv_<type>_i<WV>x<RT>b<IB>,
// with a trailing l for the tile-loop variant (tall matrices, no bias).
#define PBX_INT(NAME, TYPE, WV, RT, IB, LOOP)                                 \
  extern "C" __global__ void __launch_bounds__(WV * 64) NAME(GemvArgs a) {   \
    gemv_int<TYPE, WV, RT, IB, PRO_NONE, EPI_STORE, LOOP>(a);                 \
  }
// Scheduled variants (pbx_gemv_impl.h): w<BW> = BW builder waves beside the
// WV row waves, p<PRE> = rows requested before the limb barrier.
#define PBX_INT_S(NAME, TYPE, WV, RT, IB, BW, PRE)                            \
  extern "C" __global__ void __launch_bounds__((WV + BW) * 64) NAME(GemvArgs a) { \
    gemv_int<TYPE, WV, RT, IB, PRO_NONE, EPI_STORE, false, 1, BW, PRE>(a);    \
  }
PBX_INT(pbx_gemv_q4_0_i16x4b1, PBX_Q4, 16, 4, 1, false)
PBX_INT_S(pbx_gemv_q4_0_i16x4b1p2, PBX_Q4, 16, 4, 1, 0, 2)
PBX_INT_S(pbx_gemv_q4_0_i4x2b4w8, PBX_Q4, 4, 2, 4, 8, 2)
PBX_INT(pbx_gemv_q4_0_i4x2b1, PBX_Q4, 4, 2, 1, false)
PBX_INT(pbx_gemv_q4_0_i4x1b1, PBX_Q4, 4, 1, 1, false)
PBX_INT(pbx_gemv_q4_0_i4x8b1l, PBX_Q4, 4, 8, 1, true)
PBX_INT(pbx_gemv_q4_0_i8x4b2, PBX_Q4, 8, 4, 2, false)
PBX_INT(pbx_gemv_q4_0_i4x2b2, PBX_Q4, 4, 2, 2, false)
PBX_INT(pbx_gemv_q4_0_i4x1b2, PBX_Q4, 4, 1, 2, false)
PBX_INT(pbx_gemv_q4_0_i4x2b4, PBX_Q4, 4, 2, 4, false)
PBX_INT(pbx_gemv_q4_0_i4x1b4, PBX_Q4, 4, 1, 4, false)
PBX_INT(pbx_gemv_q8_0_i8x4b1, PBX_Q8, 8, 4, 1, false)
PBX_INT(pbx_gemv_q8_0_i4x2b1, PBX_Q8, 4, 2, 1, false)
PBX_INT(pbx_gemv_q8_0_i4x1b1, PBX_Q8, 4, 1, 1, false)
PBX_INT(pbx_gemv_q8_0_i4x8b1l, PBX_Q8, 4, 8, 1, true)
PBX_INT(pbx_gemv_q8_0_i8x4b2, PBX_Q8, 8, 4, 2, false)
PBX_INT(pbx_gemv_q8_0_i4x2b2, PBX_Q8, 4, 2, 2, false)
PBX_INT(pbx_gemv_q8_0_i4x1b2, PBX_Q8, 4, 1, 2, false)
PBX_INT(pbx_gemv_q8_0_i4x2b4, PBX_Q8, 4, 2, 4, false)
PBX_INT(pbx_gemv_q8_0_i4x1b4, PBX_Q8, 4, 1, 4, false)

// Reference Q8 tensor (quantize.js:30-50, matmul_q8 quantize.js:224-266):
// q is the flat int8 [K,N] array, scales one f32 per 32 flat elements.  The
// scale used for (k, n) is the one matmul_q8 picks: the block holding the
// first element of n's 32-wide column group, floor((k*N + 32*floor(n/32))/32).
// The reference skips activations equal to 0 (quantize.js:248); so does this.
// Workgroup: 64 output columns x 8 waves over interleaved k.
extern "C" __global__ void __launch_bounds__(512)
pbx_gemv_q8ref(const int8_t *q, const float *scales, const float *X,
               const float *bias, float *Y, int N, int K) {
  __shared__ float part[8][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + lane;
  const float *x = X + (size_t)blockIdx.y * K;
  float *y = Y + (size_t)blockIdx.y * N;
  float s = 0.f;
  if (n < N) {
    const int64_t ng = (int64_t)(n / 32) * 32;
    for (int k = wave; k < K; k += 8) {
      const float xk = x[k];
      if (xk == 0.f) continue;
      const int64_t flat = (int64_t)k * N;
      const float sc = scales[(flat + ng) / 32];
      s = fmaf(xk * sc, (float)q[flat + n], s);
    }
  }
  part[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && n < N) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) t += part[w][lane];
    y[n] = t + (bias ? bias[n] : 0.f);
  }
}

// ---------------------------------------------------------------------------
// Upload repack: GGUF row-major blocks (18 B Q4_0 / 34 B Q8_0, 2-byte
// aligned) -> qs plane + d plane.  One thread per block of a chunk of rows
// [row0, row0+rows).
// ---------------------------------------------------------------------------
extern "C" __global__ void __launch_bounds__(256)
pbx_repack_q4_0(const uint16_t *raw, uint8_t *qs, uint16_t *dsc, int64_t row0,
                int64_t rows, int B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * B) return;
  const int64_t n = row0 + i / B;
  const int b = (int)(i % B);
  const uint16_t *src = raw + i * 9;  // 18 B = 9 halfwords
  unsigned h[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = src[1 + j];
  uint4 v;
  v.x = h[0] | (h[1] << 16); v.y = h[2] | (h[3] << 16);
  v.z = h[4] | (h[5] << 16); v.w = h[6] | (h[7] << 16);
  *reinterpret_cast<uint4 *>(qs + ((size_t)n * B + b) * 16) = v;
  dsc[dsc_index((int)n, b, B)] = src[0];
}

extern "C" __global__ void __launch_bounds__(256)
pbx_repack_q8_0(const uint16_t *raw, uint8_t *qs, uint16_t *dsc, int64_t row0,
                int64_t rows, int B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * B) return;
  const int64_t n = row0 + i / B;
  const int b = (int)(i % B);
  const uint16_t *src = raw + i * 17;  // 34 B = 17 halfwords
  unsigned h[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) h[j] = src[1 + j];
  uint4 v0, v1;
  v0.x = h[0] | (h[1] << 16);   v0.y = h[2] | (h[3] << 16);
  v0.z = h[4] | (h[5] << 16);   v0.w = h[6] | (h[7] << 16);
  v1.x = h[8] | (h[9] << 16);   v1.y = h[10] | (h[11] << 16);
  v1.z = h[12] | (h[13] << 16); v1.w = h[14] | (h[15] << 16);
  uint4 *dst = reinterpret_cast<uint4 *>(qs + ((size_t)n * B + b) * 32);
  dst[0] = v0;
  dst[1] = v1;
  dsc[dsc_index((int)n, b, B)] = src[0];
}

// Q4_1: 20-byte blocks (fp16 d, fp16 m, 16 nibble bytes) are 4-byte aligned
// in the staged rows, so each block is five 32-bit loads.
extern "C" __global__ void __launch_bounds__(256)
pbx_repack_q4_1(const uint32_t *raw, uint8_t *qs, uint16_t *dsc, uint16_t *msc, int64_t row0,
                int64_t rows, int B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * B) return;
  const int64_t n = row0 + i / B;
  const int b = (int)(i % B);
  const uint32_t *src = raw + i * 5;
  const uint32_t dm = src[0];
  *reinterpret_cast<uint4 *>(qs + ((size_t)n * B + b) * 16) =
      make_uint4(src[1], src[2], src[3], src[4]);
  const size_t di = dsc_index((int)n, b, B);
  dsc[di] = (uint16_t)(dm & 0xFFFFu);
  msc[di] = (uint16_t)(dm >> 16);
}

// Q6_K: 210-byte blocks (ql[128], qh[64], scales[16], fp16 d) are 2-byte
// aligned in the staged rows; the first 208 bytes move to the qs plane as
// thirteen 16-byte stores, d to the scale plane.  B is super-blocks per row.
extern "C" __global__ void __launch_bounds__(256)
pbx_repack_q6_k(const uint16_t *raw, uint8_t *qs, uint16_t *dsc, int64_t row0, int64_t rows,
                int B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * B) return;
  const int64_t n = row0 + i / B;
  const int b = (int)(i % B);
  const uint16_t *src = raw + i * 105;  // 210 B = 105 halfwords
  uint4 *dst = reinterpret_cast<uint4 *>(qs + ((size_t)n * B + b) * PBX_Q6K_BYTES);
#pragma unroll
  for (int v = 0; v < 13; ++v) {
    const uint16_t *h = src + 8 * v;
    dst[v] = make_uint4(h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16),
                        h[4] | ((unsigned)h[5] << 16), h[6] | ((unsigned)h[7] << 16));
  }
  dsc[dsc_index((int)n, b, B)] = src[104];
}

// ---------------------------------------------------------------------------
// Exact dequantisation to fp32 row-major [N,K] (gguf.js:239-286): the
// product of an fp16 scale and a small integer is exact in fp32.
// ---------------------------------------------------------------------------
extern "C" __global__ void __launch_bounds__(256)
pbx_dequant_q4_0(const uint8_t *qs, const uint16_t *dsc, float *out, int N, int B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)N * B) return;
  const int n = (int)(i / B), b = (int)(i % B);
  const uint4 q = *reinterpret_cast<const uint4 *>(qs + i * 16);
  const float d = f16_bits_to_f32(dsc[dsc_index((int)n, b, B)]);
  const unsigned w[4] = {q.x, q.y, q.z, q.w};
  float v[32];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const unsigned byte = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
    v[j] = (float)((int)(byte & 0xFu) - 8) * d;
    v[j + 16] = (float)((int)(byte >> 4) - 8) * d;
  }
  float4 *dst = reinterpret_cast<float4 *>(out + i * 32);
#pragma unroll
  for (int j = 0; j < 8; ++j) dst[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
}

extern "C" __global__ void __launch_bounds__(256)
pbx_dequant_q8_0(const uint8_t *qs, const uint16_t *dsc, float *out, int N, int B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)N * B) return;
  const int n = (int)(i / B), b = (int)(i % B);
  const int8_t *q = reinterpret_cast<const int8_t *>(qs + i * 32);
  const float d = f16_bits_to_f32(dsc[dsc_index((int)n, b, B)]);
  float4 *dst = reinterpret_cast<float4 *>(out + i * 32);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    dst[j] = make_float4((float)q[4 * j] * d, (float)q[4 * j + 1] * d,
                         (float)q[4 * j + 2] * d, (float)q[4 * j + 3] * d);
}

// Q4_1 (gguf.js:288-314): nibble * d + m.  nibble * d is exact in fp32, so
// the fused multiply-add rounds once, as the reference's double expression
// rounds once into its Float32Array.
extern "C" __global__ void __launch_bounds__(256)
pbx_dequant_q4_1(const uint8_t *qs, const uint16_t *dsc, const uint16_t *msc, float *out, int N,
                 int B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)N * B) return;
  const int n = (int)(i / B), b = (int)(i % B);
  const uint4 q = *reinterpret_cast<const uint4 *>(qs + i * 16);
  const size_t di = dsc_index(n, b, B);
  const float d = f16_bits_to_f32(dsc[di]);
  const float m = f16_bits_to_f32(msc[di]);
  const unsigned w[4] = {q.x, q.y, q.z, q.w};
  float v[32];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const unsigned byte = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
    v[j] = fmaf((float)(byte & 0xFu), d, m);
    v[j + 16] = fmaf((float)(byte >> 4), d, m);
  }
  float4 *dst = reinterpret_cast<float4 *>(out + i * 32);
#pragma unroll
  for (int j = 0; j < 8; ++j) dst[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
}

// F16 (gguf.js:231-237): exact conversion.
extern "C" __global__ void __launch_bounds__(256)
pbx_dequant_f16(const uint16_t *qs, float *out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = f16_bits_to_f32(qs[i]);
}

// Q6_K (gguf.js:317-364): one thread per 32 consecutive outputs of a row
// (element layout in load_lane); (d * sc) * (q - 32) is exact in fp32.
extern "C" __global__ void __launch_bounds__(256)
pbx_dequant_q6_k(const uint8_t *qs, const uint16_t *dsc, float *out, int N, int B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 32-block index
  if (i >= (int64_t)N * B * 8) return;
  const int n = (int)(i / (B * 8)), j = (int)(i % (B * 8));
  uint4 q[4];
  unsigned ex;
  load_lane<PBX_Q6K>(qs, n, j, B * 8, true, q, ex);
  const float d = f16_bits_to_f32(dsc[dsc_index(n, j >> 3, B)]);
  const int g = j & 3, sl = (g >> 1) * 4, sh = g * 2;
  const unsigned ql[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
  const unsigned qh[8] = {q[2].x, q[2].y, q[2].z, q[2].w, q[3].x, q[3].y, q[3].z, q[3].w};
  const float ds0 = d * (float)(int8_t)(ex & 0xFFu), ds1 = d * (float)(int8_t)((ex >> 8) & 0xFFu);
  float v[32];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const unsigned c = ((ql[k] >> sl) & 0x0F0F0F0Fu) | (((qh[k] >> sh) & 0x03030303u) << 4);
    const float ds = k < 4 ? ds0 : ds1;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * k + e] = ds * (float)((int)((c >> (8 * e)) & 0xFFu) - 32);
  }
  float4 *dst = reinterpret_cast<float4 *>(out + i * 32);
#pragma unroll
  for (int k = 0; k < 8; ++k) dst[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
}

// dequantize_q8 (quantize.js:170-181): out[i] = q[i] * scales[i/32].
extern "C" __global__ void __launch_bounds__(256)
pbx_dequant_q8ref(const int8_t *q, const float *scales, float *out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (float)q[i] * scales[i / 32];
}

// Plain 16-byte copy (pbx_dev_copy): a kernel of known traffic, n16 * 16 bytes
// read and written, used to calibrate hardware byte counters.
extern "C" __global__ void __launch_bounds__(256)
pbx_copy16(const uint4 *src, uint4 *dst, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}
