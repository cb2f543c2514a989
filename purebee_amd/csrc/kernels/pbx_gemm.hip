// pbx_gemm.hip -- gfx950 MFMA GEMM for the M >= 4 instruction
// (batched prefill, speculative verify): Y[M,N] = X[M,K] . W[N,K]^T with W
// in Q4_0 / Q8_0 planes.
//
// One v_mfma_f32_16x16x32_f16 consumes exactly one 32-wide quantisation
// block: the A operand is 16 activation rows x 32 k (fp16), the B operand is
// 16 weight rows x 32 k dequantised on the fly, the 16x16 fp32 accumulator
// sums over blocks.  Operand lane layout (checked on the device):
//   A: lane l holds A[l%16][8*(l/16) + e], e = 0..7
//   B: lane l holds B[8*(l/16) + e][l%16]
//   D: lane l holds D[4*(l/16) + r][l%16], r = 0..3
// For Q4_0 lane group g = l/16 takes k = 8g..8g+7 of the block: low nibbles
// of bytes 0..7 (g=0), of bytes 8..15 (g=1), high nibbles of bytes 0..7
// (g=2) and of bytes 8..15 (g=3), the element order of gguf.js:259-286.
//
// Precision: activations are scaled per row by a power of two so the row's
// largest magnitude sits just below 2^15, then rounded to fp16 (relative
// error <= 2^-11); weights are (q - 8) * d rounded once to fp16 (the product
// is exact in fp32).  Accumulation is fp32; the power of two is undone
// exactly in the epilogue.

#include "pbx_gemv_impl.h"

using namespace pbx;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
  const uint8_t *qs;    // weight plane
  const uint16_t *dsc;  // fp16 scale plane (4-row groups)
  const _Float16 *X16;  // [Mpad][K] scaled fp16 activations
  const float *inv;     // [Mpad] power of two undoing the row scale
  const float *bias;    // [N] or null (single split only)
  float *Y;             // KS == 1: [M][N]; else partials [KS][M][N]
  int M, N, Npad, B, KS;
  int accumulate;       // 1: Y[m][n] += result (residual), single split only
};

namespace {

template <int TYPE>
__device__ __forceinline__ half8 weight_operand(const GemmArgs &a, int n, int b, int g) {
  half8 v;
  if (n >= a.Npad) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (_Float16)0.f;
    return v;
  }
  const float d = f16_bits_to_f32(a.dsc[dsc_index(n, b, a.B)]);
  if constexpr (TYPE == PBX_Q4) {
    const uint2 w = *reinterpret_cast<const uint2 *>(a.qs + ((size_t)n * a.B + b) * 16 + (g & 1) * 8);
    const unsigned sh = (g >> 1) * 4;  // low nibbles for g < 2, high for g >= 2
    const unsigned lo = (w.x >> sh) & 0x0F0F0F0Fu, hi = (w.y >> sh) & 0x0F0F0F0Fu;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = (_Float16)((float)((int)((lo >> (8 * e)) & 0xFu) - 8) * d);
      v[e + 4] = (_Float16)((float)((int)((hi >> (8 * e)) & 0xFu) - 8) * d);
    }
  } else {
    const uint2 w = *reinterpret_cast<const uint2 *>(a.qs + ((size_t)n * a.B + b) * 32 + g * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = (_Float16)((float)(int8_t)((w.x >> (8 * e)) & 0xFFu) * d);
      v[e + 4] = (_Float16)((float)(int8_t)((w.y >> (8 * e)) & 0xFFu) * d);
    }
  }
  return v;
}

// Workgroup = 4 waves side by side along n.  Wave tile: 16*MT rows of X by
// 16*NT rows of W; blockIdx.z splits the K blocks.
template <int TYPE, int MT, int NT>
__device__ __forceinline__ void gemm_tile(const GemmArgs &a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.x * 4 + wave) * (16 * NT);
  const int m0 = blockIdx.y * (16 * MT);
  const int K = a.B * 32;
  const int per = (a.B + a.KS - 1) / a.KS;
  const int b0 = blockIdx.z * per;
  const int b1 = min(a.B, b0 + per);

  floatx4 acc[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NT; ++u) acc[t][u] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int b = b0; b < b1; ++b) {
    half8 A[MT], W[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) W[u] = weight_operand<TYPE>(a, n0 + 16 * u + li, b, g);
#pragma unroll
    for (int t = 0; t < MT; ++t)
      A[t] = *reinterpret_cast<const half8 *>(a.X16 + (size_t)(m0 + 16 * t + li) * K + b * 32 + 8 * g);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int u = 0; u < NT; ++u)
        acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[t], W[u], acc[t][u], 0, 0, 0);
  }

#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NT; ++u) {
      const int n = n0 + 16 * u + li;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * t + 4 * g + r;
        if (m < a.M && n < a.N) {
          const float v = acc[t][u][r] * a.inv[m];
          if (a.KS == 1) {
            float *y = a.Y + (size_t)m * a.N + n;
            if (a.accumulate)
              *y += v;
            else
              *y = v + (a.bias ? a.bias[n] : 0.f);
          } else {
            a.Y[((size_t)blockIdx.z * a.M + m) * a.N + n] = v;
          }
        }
      }
    }
}

}  // namespace

#define GEMM_KERNEL(NAME, TYPE, MT, NT)                                            \
  extern "C" __global__ void __launch_bounds__(256) NAME(GemmArgs a) {             \
    gemm_tile<TYPE, MT, NT>(a);                                                    \
  }
GEMM_KERNEL(pbx_gemm_q4_m1_n1, PBX_Q4, 1, 1)
GEMM_KERNEL(pbx_gemm_q4_m1_n2, PBX_Q4, 1, 2)
GEMM_KERNEL(pbx_gemm_q4_m1_n4, PBX_Q4, 1, 4)
GEMM_KERNEL(pbx_gemm_q4_m2_n2, PBX_Q4, 2, 2)
GEMM_KERNEL(pbx_gemm_q4_m4_n2, PBX_Q4, 4, 2)
GEMM_KERNEL(pbx_gemm_q4_m4_n4, PBX_Q4, 4, 4)
GEMM_KERNEL(pbx_gemm_q8_m1_n1, PBX_Q8, 1, 1)
GEMM_KERNEL(pbx_gemm_q8_m1_n2, PBX_Q8, 1, 2)
GEMM_KERNEL(pbx_gemm_q8_m1_n4, PBX_Q8, 1, 4)
GEMM_KERNEL(pbx_gemm_q8_m2_n2, PBX_Q8, 2, 2)
GEMM_KERNEL(pbx_gemm_q8_m4_n2, PBX_Q8, 4, 2)
GEMM_KERNEL(pbx_gemm_q8_m4_n4, PBX_Q8, 4, 4)

// Row scaling to fp16: one workgroup per (padded) row.  The scale is
// 2^(15 - e) with 2^(e-1) <= max|x| < 2^e, so every scaled value is below
// 2^15 in magnitude (fp16 max 65504); padding rows are zero.
extern "C" __global__ void __launch_bounds__(256)
pbx_gemm_prep_x(const float *X, _Float16 *X16, float *inv, int M, int K) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  _Float16 *dst = X16 + (size_t)m * K;
  if (m >= M) {
    for (int k = threadIdx.x; k < K; k += blockDim.x) dst[k] = (_Float16)0.f;
    if (threadIdx.x == 0) inv[m] = 0.f;
    return;
  }
  const float *src = X + (size_t)m * K;
  float mx = 0.f;
  for (int k = threadIdx.x; k < K; k += blockDim.x) mx = fmaxf(mx, fabsf(src[k]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.f && mx < INFINITY) frexpf(mx, &e);
  const float scale = mx > 0.f ? ldexpf(1.f, 15 - e) : 1.f;
  for (int k = threadIdx.x; k < K; k += blockDim.x) dst[k] = (_Float16)(src[k] * scale);
  if (threadIdx.x == 0) inv[m] = mx > 0.f ? ldexpf(1.f, e - 15) : 1.f;
}

// Sum of the split-K partials (+ bias, or accumulated into Y).
extern "C" __global__ void __launch_bounds__(256)
pbx_gemm_reduce(const float *part, const float *bias, float *Y, int M, int N, int KS,
                int accumulate) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t MN = (int64_t)M * N;
  if (i >= MN) return;
  float s = 0.f;
  for (int k = 0; k < KS; ++k) s += part[k * MN + i];
  if (accumulate)
    Y[i] += s;
  else
    Y[i] = s + (bias ? bias[i % N] : 0.f);
}
