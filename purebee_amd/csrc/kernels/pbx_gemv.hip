// pbx_gemv.hip -- gfx950 kernels for PureBee's quantized matvec instruction:
// weight repack, exact dequantisation and the M=1 GEMV family.
//
// Built with `hipcc --genco --offload-arch=gfx950` into pbx_kernels.hsaco and
// loaded by the runtime with hipModuleLoad; every kernel is extern "C" so the
// runtime can look it up by name with hipModuleGetFunction.
//
// Device layout of a resident weight (N rows, K columns, B = K/32 blocks/row,
// Npad = N rounded up to 64 so row tiles never need a load guard):
//   Q4_0 : qs plane  [Npad][B][16] bytes   (the 16 nibble bytes of each block)
//          d  plane  [Npad/8][B][8] fp16   (8 rows' scales of one block are
//                                           contiguous: one 16-B load serves
//                                           an 8-row group)
//   Q8_0 : qs plane  [Npad][B][32] int8, d plane as Q4_0
//   F32  : plane     [Npad][K] float
// The GGUF block formats these come from are gguf.js:36-49 (sizes) and
// gguf.js:239-286 (element order: Q4_0 byte j holds element j in its low
// nibble and element j+16 in its high nibble; value = (nibble - 8) * d).

#include <hip/hip_runtime.h>
#include <stdint.h>

#define PBX_Q4 0
#define PBX_Q8 1
#define PBX_F32 2

namespace {

__device__ __forceinline__ float f16_bits_to_f32(unsigned bits) {
  // IEEE binary16 -> binary32 (v_cvt_f32_f16), the conversion of
  // gguf.js:55-70 including subnormals, +-inf and NaN.
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits & 0xFFFFu));
}

// ---------------------------------------------------------------------------
// Block dot products against 32 activations held in registers.
// ---------------------------------------------------------------------------

// sum_j x[j] * nibble_j over one Q4_0 block (nibbles unsigned, 0..15); the
// caller subtracts 8*sum(x) to obtain sum_j x[j] * (nibble_j - 8).
__device__ __forceinline__ float dot_q4(const uint4 q, const float (&xr)[32]) {
  const unsigned w[4] = {q.x, q.y, q.z, q.w};
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const unsigned lo = w[j] & 0x0F0F0F0Fu;
    const unsigned hi = (w[j] >> 4) & 0x0F0F0F0Fu;
    s0 = fmaf(xr[4 * j + 0], (float)(lo & 0xFFu), s0);
    s0 = fmaf(xr[4 * j + 1], (float)((lo >> 8) & 0xFFu), s0);
    s0 = fmaf(xr[4 * j + 2], (float)((lo >> 16) & 0xFFu), s0);
    s0 = fmaf(xr[4 * j + 3], (float)(lo >> 24), s0);
    s1 = fmaf(xr[16 + 4 * j + 0], (float)(hi & 0xFFu), s1);
    s1 = fmaf(xr[16 + 4 * j + 1], (float)((hi >> 8) & 0xFFu), s1);
    s1 = fmaf(xr[16 + 4 * j + 2], (float)((hi >> 16) & 0xFFu), s1);
    s1 = fmaf(xr[16 + 4 * j + 3], (float)(hi >> 24), s1);
  }
  return s0 + s1;
}

// sum_j x[j] * (q_j + 128) over one Q8_0 block: flipping the sign bit of each
// int8 gives the unsigned byte q+128, which converts in one instruction; the
// caller subtracts 128*sum(x).
__device__ __forceinline__ float dot_q8(const uint4 qa, const uint4 qb,
                                        const float (&xr)[32]) {
  const unsigned w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const unsigned u = w[j] ^ 0x80808080u;
    float &s = (j & 1) ? s1 : s0;
    s = fmaf(xr[4 * j + 0], (float)(u & 0xFFu), s);
    s = fmaf(xr[4 * j + 1], (float)((u >> 8) & 0xFFu), s);
    s = fmaf(xr[4 * j + 2], (float)((u >> 16) & 0xFFu), s);
    s = fmaf(xr[4 * j + 3], (float)(u >> 24), s);
  }
  return s0 + s1;
}

__device__ __forceinline__ float dot_f32(const uint4 (&q)[8],
                                         const float (&xr)[32]) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float &s = (j & 1) ? s1 : s0;
    s = fmaf(xr[4 * j + 0], __uint_as_float(q[j].x), s);
    s = fmaf(xr[4 * j + 1], __uint_as_float(q[j].y), s);
    s = fmaf(xr[4 * j + 2], __uint_as_float(q[j].z), s);
    s = fmaf(xr[4 * j + 3], __uint_as_float(q[j].w), s);
  }
  return s0 + s1;
}

template <int TYPE> struct BlockTraits;
template <> struct BlockTraits<PBX_Q4> { static constexpr int QB = 16; static constexpr float OFF = 8.f; };
template <> struct BlockTraits<PBX_Q8> { static constexpr int QB = 32; static constexpr float OFF = 128.f; };
template <> struct BlockTraits<PBX_F32> { static constexpr int QB = 128; static constexpr float OFF = 0.f; };

__device__ __forceinline__ void load_x_block(const float *__restrict__ x,
                                             int b, bool valid, float (&xr)[32]) {
  if (valid) {
    const float4 *xp = reinterpret_cast<const float4 *>(x + (size_t)b * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = xp[i];
      xr[4 * i + 0] = v.x; xr[4 * i + 1] = v.y;
      xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) xr[i] = 0.f;
  }
}

// One block of one row: qs bytes at p, scale d; returns the block's
// contribution d * sum_j x_j * w_j (F32: just the dot).
template <int TYPE>
__device__ __forceinline__ float block_term(const uint4 (&q)[BlockTraits<TYPE>::QB / 16],
                                            const float (&xr)[32], float corr,
                                            float d) {
  if constexpr (TYPE == PBX_Q4) {
    return (dot_q4(q[0], xr) - corr) * d;
  } else if constexpr (TYPE == PBX_Q8) {
    return (dot_q8(q[0], q[1], xr) - corr) * d;
  } else {
    return dot_f32(q, xr);
  }
}

// Transposed wavefront reduction: v[0..R) are 64-lane partial sums of R rows.
// log2(R) halving stages exchange half of the remaining values with the lane
// `off` away, so every stage moves R/2, R/4, ... values instead of reducing
// each row separately; afterwards lane l holds row l / (64/R) summed over its
// group, and the remaining butterfly stages finish the 64-lane sum.
template <int CNT, int OFF, int R>
__device__ __forceinline__ void transpose_stage(float (&v)[R], int lane) {
  if constexpr (CNT > 1) {
    const bool up = (lane & OFF) != 0;
#pragma unroll
    for (int i = 0; i < CNT / 2; ++i) {
      const float keep = up ? v[i + CNT / 2] : v[i];
      const float send = up ? v[i] : v[i + CNT / 2];
      v[i] = keep + __shfl_xor(send, OFF, 64);
    }
    transpose_stage<CNT / 2, OFF / 2, R>(v, lane);
  }
}

template <int R>
__device__ __forceinline__ float wave_transpose_reduce(float (&v)[R], int lane) {
  transpose_stage<R, 32, R>(v, lane);
  float r = v[0];
#pragma unroll
  for (int off = (64 / R) / 2; off >= 1; off >>= 1) r += __shfl_xor(r, off, 64);
  return r;
}

// ---------------------------------------------------------------------------
// Wide GEMV: B >= 33 blocks per row.  A workgroup has W = ceil(B/64) waves;
// lane l of wave w owns block b = 64w + l of every row, keeps that block's 32
// activations in registers, and accumulates one partial per row of its
// R-row tile.  Weight loads are 16 B per lane and contiguous across the
// wave (one row's 64 blocks = 1 KiB for Q4_0).  blockIdx.y selects the
// activation row m (Y[m,:] = W . X[m,:]).
// ---------------------------------------------------------------------------
template <int TYPE, int R>
__device__ __forceinline__ void gemv_wide(const uint8_t *__restrict__ qs,
                                          const uint16_t *__restrict__ dsc,
                                          const float *__restrict__ X,
                                          const float *__restrict__ bias,
                                          float *__restrict__ Y, int N, int B) {
  constexpr int QB = BlockTraits<TYPE>::QB;
  constexpr int NV = QB / 16;
  constexpr int MAXW = 8;
  __shared__ float red[MAXW][R];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int b = wave * 64 + lane;
  const bool valid = b < B;
  const int K = B * 32;
  const float *x = X + (size_t)blockIdx.y * K;
  float *y = Y + (size_t)blockIdx.y * N;

  float xr[32];
  load_x_block(x, b, valid, xr);
  float xs = 0.f;
  if constexpr (TYPE != PBX_F32) {
#pragma unroll
    for (int i = 0; i < 32; ++i) xs += xr[i];
  }
  const float corr = BlockTraits<TYPE>::OFF * xs;

  const int r0 = blockIdx.x * R;
  uint4 q[R][NV];
  const uint8_t *base = qs + ((size_t)r0 * B + b) * QB;
#pragma unroll
  for (int i = 0; i < R; ++i) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      q[i][v] = valid ? *reinterpret_cast<const uint4 *>(base + (size_t)i * B * QB + v * 16)
                      : make_uint4(0u, 0u, 0u, 0u);
    }
  }

  // Scales of rows r0..r0+R-1 at block b.
  float dsf[R];
  if constexpr (TYPE != PBX_F32) {
    if constexpr (R >= 8) {
#pragma unroll
      for (int g = 0; g < R / 8; ++g) {
        const uint4 dv = valid ? *reinterpret_cast<const uint4 *>(
                                     dsc + ((size_t)(r0 / 8 + g) * B + b) * 8)
                               : make_uint4(0u, 0u, 0u, 0u);
        const unsigned dw[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dsf[g * 8 + 2 * j] = f16_bits_to_f32(dw[j]);
          dsf[g * 8 + 2 * j + 1] = f16_bits_to_f32(dw[j] >> 16);
        }
      }
    } else {
      // R == 2 or 4 rows inside one 8-row group (r0 % R == 0).
      const uint16_t *dp = dsc + ((size_t)(r0 / 8) * B + b) * 8 + (r0 & 7);
#pragma unroll
      for (int i = 0; i < R; ++i) dsf[i] = valid ? f16_bits_to_f32(dp[i]) : 0.f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i) dsf[i] = 1.f;
  }

  float acc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = block_term<TYPE>(q[i], xr, corr, dsf[i]);

  const float tot = wave_transpose_reduce<R>(acc, lane);
  const int lanes_per_row = 64 / R;
  const int row = lane / lanes_per_row;
  if (nwaves == 1) {
    if ((lane % lanes_per_row) == 0) {
      const int n = r0 + row;
      if (n < N) y[n] = tot + (bias ? bias[n] : 0.f);
    }
  } else {
    if ((lane % lanes_per_row) == 0) red[wave][row] = tot;
    __syncthreads();
    if (threadIdx.x < R) {
      float s = 0.f;
      for (int w = 0; w < nwaves; ++w) s += red[w][threadIdx.x];
      const int n = r0 + threadIdx.x;
      if (n < N) y[n] = s + (bias ? bias[n] : 0.f);
    }
  }
}

// ---------------------------------------------------------------------------
// Small-K GEMV: B <= 32 blocks per row (K <= 1024).  Lane l of a wave owns
// (row slot l / B, block l % B); RPW = 64 / B rows are in flight per pass and
// P passes make a tile of P*RPW rows.  Partials go through LDS and one lane
// per row sums its B entries.  Each of the 4 waves of a workgroup runs its own
// tile.
// ---------------------------------------------------------------------------
template <int TYPE, int P>
__device__ __forceinline__ void gemv_small(const uint8_t *__restrict__ qs,
                                           const uint16_t *__restrict__ dsc,
                                           const float *__restrict__ X,
                                           const float *__restrict__ bias,
                                           float *__restrict__ Y, int N, int B) {
  constexpr int QB = BlockTraits<TYPE>::QB;
  constexpr int NV = QB / 16;
  __shared__ float part[4][P][64];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rpw = 64 / B;
  const bool active = lane < rpw * B;
  const int rs = active ? lane / B : 0;
  const int b = active ? lane % B : 0;
  const int K = B * 32;
  const float *x = X + (size_t)blockIdx.y * K;
  float *y = Y + (size_t)blockIdx.y * N;

  const int T = P * rpw;
  const int r0 = (blockIdx.x * 4 + wave) * T;

  float xr[32];
  load_x_block(x, b, active, xr);
  float xs = 0.f;
  if constexpr (TYPE != PBX_F32) {
#pragma unroll
    for (int i = 0; i < 32; ++i) xs += xr[i];
  }
  const float corr = BlockTraits<TYPE>::OFF * xs;

#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int row = r0 + p * rpw + rs;
    const bool ok = active && row < N;
    uint4 q[NV];
    const uint8_t *src = qs + ((size_t)row * B + b) * QB;
#pragma unroll
    for (int v = 0; v < NV; ++v)
      q[v] = ok ? *reinterpret_cast<const uint4 *>(src + v * 16) : make_uint4(0u, 0u, 0u, 0u);
    float d = 1.f;
    if constexpr (TYPE != PBX_F32)
      d = ok ? f16_bits_to_f32(dsc[((size_t)(row >> 3) * B + b) * 8 + (row & 7)]) : 0.f;
    part[wave][p][lane] = ok ? block_term<TYPE>(q, xr, corr, d) : 0.f;
  }
  __syncthreads();
  for (int t = lane; t < T; t += 64) {
    const int p = t / rpw, r = t % rpw;
    float s = 0.f;
    for (int j = 0; j < B; ++j) s += part[wave][p][r * B + j];
    const int n = r0 + t;
    if (n < N) y[n] = s + (bias ? bias[n] : 0.f);
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Exported kernels.
// ---------------------------------------------------------------------------
#define PBX_WIDE(NAME, TYPE, R)                                               \
  extern "C" __global__ void __launch_bounds__(512)                           \
  NAME(const uint8_t *qs, const uint16_t *dsc, const float *X,                \
       const float *bias, float *Y, int N, int B) {                           \
    gemv_wide<TYPE, R>(qs, dsc, X, bias, Y, N, B);                            \
  }
PBX_WIDE(pbx_gemv_q4_0_wide_r4, PBX_Q4, 4)
PBX_WIDE(pbx_gemv_q4_0_wide_r8, PBX_Q4, 8)
PBX_WIDE(pbx_gemv_q4_0_wide_r16, PBX_Q4, 16)
PBX_WIDE(pbx_gemv_q8_0_wide_r4, PBX_Q8, 4)
PBX_WIDE(pbx_gemv_q8_0_wide_r8, PBX_Q8, 8)
PBX_WIDE(pbx_gemv_f32_wide_r2, PBX_F32, 2)
PBX_WIDE(pbx_gemv_f32_wide_r4, PBX_F32, 4)

#define PBX_SMALL(NAME, TYPE, P)                                              \
  extern "C" __global__ void __launch_bounds__(256)                           \
  NAME(const uint8_t *qs, const uint16_t *dsc, const float *X,                \
       const float *bias, float *Y, int N, int B) {                           \
    gemv_small<TYPE, P>(qs, dsc, X, bias, Y, N, B);                           \
  }
PBX_SMALL(pbx_gemv_q4_0_small, PBX_Q4, 8)
PBX_SMALL(pbx_gemv_q8_0_small, PBX_Q8, 4)
PBX_SMALL(pbx_gemv_f32_small, PBX_F32, 2)

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
  dsc[((size_t)(n >> 3) * B + b) * 8 + (n & 7)] = src[0];
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
  dsc[((size_t)(n >> 3) * B + b) * 8 + (n & 7)] = src[0];
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
  const float d = f16_bits_to_f32(dsc[((size_t)(n >> 3) * B + b) * 8 + (n & 7)]);
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
  const float d = f16_bits_to_f32(dsc[((size_t)(n >> 3) * B + b) * 8 + (n & 7)]);
  float4 *dst = reinterpret_cast<float4 *>(out + i * 32);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    dst[j] = make_float4((float)q[4 * j] * d, (float)q[4 * j + 1] * d,
                         (float)q[4 * j + 2] * d, (float)q[4 * j + 3] * d);
}

// dequantize_q8 (quantize.js:170-181): out[i] = q[i] * scales[i/32].
extern "C" __global__ void __launch_bounds__(256)
pbx_dequant_q8ref(const int8_t *q, const float *scales, float *out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (float)q[i] * scales[i / 32];
}
