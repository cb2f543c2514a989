// pbx_gemm.hip -- gfx950 MFMA GEMM for the M >= 4 instruction
// (batched prefill, speculative verify, multi-row LINEAR): Y[M,N] =
// X[M,K] . W[N,K]^T (+ bias) with W in Q4_0 / Q8_0 / Q4_1 / F16 planes
// (fp16 MFMA, below) or F32 (fp32 MFMA, gemm_f32 at the end).
//
// One v_mfma_f32_16x16x32_f16 consumes exactly one 32-wide quantisation
// block: the A operand is 16 activation rows x 32 k (fp16), the B operand is
// the 16 x 32 integer codes of 16 weight rows unpacked on the fly, and the
// 16x16 block product, times each row's block scale, is summed over blocks
// in fp32.  Operand lane layout (checked on the device):
//   A: lane l holds A[l%16][8*(l/16) + e], e = 0..7
//   B: lane l holds B[8*(l/16) + e][l%16]
//   D: lane l holds D[4*(l/16) + r][l%16], r = 0..3
// For Q4_0 lane group g = l/16 takes k = 8g..8g+7 of the block: low nibbles
// of bytes 0..7 (g=0), of bytes 8..15 (g=1), high nibbles of bytes 0..7
// (g=2) and of bytes 8..15 (g=3), the element order of gguf.js:259-286.
//
// Precision: weights enter the MFMA as their integer codes (q - 8 for Q4_0,
// q for Q8_0, q for Q4_1) or, for F16, as themselves, which fp16 holds
// exactly; the block scale d multiplies the block's 16x16 partial product in
// fp32 afterwards, so the weight side adds no rounding at all.  Q4_1 adds
// m * (sum of the block's activations) per block; that sum comes from one
// more MFMA pair against an all-ones operand, shared by every weight tile.  Activations are scaled per row by a power of two so
// the row's largest magnitude sits just below 2^15 and split into two fp16
// operands, hi = fp16(x) and lo = fp16(x - hi), each multiplied by the same
// weight codes (two MFMAs per tile and block): ~22 significant bits instead
// of fp16's 11.  A single fp16 (or bf16) activation operand is not accurate
// enough for the end-to-end bar: on the Llama-3.2-1B shape a 512-token
// prefill with fp16 activations ends 6.4e-3 (max-abs) away from the fp32
// decode path's logits, against a 2e-3 tolerance.  Accumulation is fp32;
// the power of two is undone exactly in the epilogue.

#include "pbx_gemv_impl.h"

using namespace pbx;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
  const uint8_t *qs;      // weight plane
  const uint16_t *dsc;    // fp16 scale plane (4-row groups)
  const _Float16 *X16;    // [Mpad][K] scaled fp16 activations
  const _Float16 *X16lo;  // [Mpad][K] rounding residual of X16
  const float *inv;       // [Mpad] power of two undoing the row scale
  const float *bias;      // [N] or null (single split only)
  float *Y;               // KS == 1: [M][N]; else partials [KS][M][N]
  int M, N, Npad, B, KS;
  int accumulate;         // 1: Y[m][n] += result (residual), single split only
  const uint16_t *msc;    // Q4_1 fp16 min plane
};

namespace {

// Two byte-sized codes c0, c1 (< 256, in bits 0-7 and 8-15 of v) as fp16
// 1024 + c (exact: fp16 spacing is 1 on [1024, 2048)), minus `bias`.
__device__ __forceinline__ half2v codes_to_half2(unsigned v, _Float16 bias) {
  const unsigned p = (v & 0xFFu) | ((v & 0xFF00u) << 8) | 0x64006400u;
  return __builtin_bit_cast(half2v, p) - half2v{bias, bias};
}

// Per-lane operand bytes of one block: 8 codes (8 bytes) for the quantised
// types, 8 fp16 weights (16 bytes) for F16.
template <int TYPE> struct RawT { typedef uint2 type; };
template <> struct RawT<PBX_F16> { typedef uint4 type; };

// Raw bytes of lane group g's 8 weights of row n, block b, and the block's
// scale (and Q4_1 min) bits; zero for padding rows.
template <int TYPE>
__device__ __forceinline__ void load_codes(const GemmArgs &a, int n, int b, int g,
                                           typename RawT<TYPE>::type *raw, unsigned *dbits,
                                           unsigned *mbits) {
  if (n >= a.Npad) {
    *raw = {};
    *dbits = 0u;
    *mbits = 0u;
    return;
  }
  if constexpr (TYPE == PBX_F16) {
    *raw = *reinterpret_cast<const uint4 *>(a.qs + (((size_t)n * a.B + b) * 32 + 8 * g) * 2);
    *dbits = 0x3C00u;  // 1.0
    *mbits = 0u;
    return;
  } else {
    const size_t di = dsc_index(n, b, a.B);
    *dbits = a.dsc[di];
    *mbits = TYPE == PBX_Q41 ? a.msc[di] : 0u;
    if constexpr (TYPE == PBX_Q4 || TYPE == PBX_Q41)
      *raw = *reinterpret_cast<const uint2 *>(a.qs + ((size_t)n * a.B + b) * 16 + (g & 1) * 8);
    else
      *raw = *reinterpret_cast<const uint2 *>(a.qs + ((size_t)n * a.B + b) * 32 + g * 8);
  }
}

// The 8 weights as an fp16 MFMA operand: the integer codes q - 8 (Q4_0,
// low nibbles for g < 2, high for g >= 2), q (Q4_1, same nibbles) or q
// (Q8_0), or the F16 weights themselves.  One v_perm_b32 builds the fp16 pair
// [0x64 | byte e, 0x64 | byte e+1] = 1024 + c (exact: fp16 spacing is 1 on
// [1024, 2048)) from the code bytes and the constant 0x64 bytes, and one
// packed-fp16 subtract removes 1024 + bias.  Nibbles are isolated in their
// bytes first; Q8_0 int8 codes are made unsigned (q + 128).
template <int TYPE>
__device__ __forceinline__ half8 codes_operand(typename RawT<TYPE>::type w, int g) {
  if constexpr (TYPE == PBX_F16) {
    return __builtin_bit_cast(half8, w);
  } else {
    unsigned x = w.x, y = w.y;
    _Float16 bias;
    if constexpr (TYPE == PBX_Q4 || TYPE == PBX_Q41) {
      const unsigned sh = (g >> 1) * 4;
      x = (x >> sh) & 0x0F0F0F0Fu;
      y = (y >> sh) & 0x0F0F0F0Fu;
      bias = TYPE == PBX_Q4 ? (_Float16)1032.f : (_Float16)1024.f;  // 1024 (+ 8)
    } else {
      x ^= 0x80808080u;
      y ^= 0x80808080u;
      bias = (_Float16)1152.f;  // 1024 + 128
    }
    auto pair = [&](unsigned v, unsigned sel) -> half2v {
      // selector bytes 0..3 pick v's bytes, 4 picks a 0x64 byte of the constant
      const unsigned h = __builtin_amdgcn_perm(0x64646464u, v, sel);
      return __builtin_bit_cast(half2v, h) - half2v{bias, bias};
    };
    const half2v p0 = pair(x, 0x04010400u), p1 = pair(x, 0x04030402u);
    const half2v p2 = pair(y, 0x04010400u), p3 = pair(y, 0x04030402u);
    half8 v;
    v[0] = p0[0]; v[1] = p0[1]; v[2] = p1[0]; v[3] = p1[1];
    v[4] = p2[0]; v[5] = p2[1]; v[6] = p3[0]; v[7] = p3[1];
    return v;
  }
}

// acc += the block product of activation tile (hi, lo) and weight operand W,
// scaled by d, plus m * xs (Q4_1; xs = the tile's block sums).  F16 has no
// block scale, so its products chain straight into the accumulator.
template <int TYPE>
__device__ __forceinline__ void block_mma(floatx4 &acc, half8 Ah, half8 Al, half8 W, float d,
                                          float m, const floatx4 &xs) {
  if constexpr (TYPE == PBX_F16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, W, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, W, acc, 0, 0, 0);
  } else {
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    floatx4 blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, W, zero, 0, 0, 0);
    blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, W, blk, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc[r] = fmaf(blk[r], d, acc[r]);
      if constexpr (TYPE == PBX_Q41) acc[r] = fmaf(xs[r], m, acc[r]);
    }
  }
}

// Block sums of an activation tile (Q4_1): the product with all-ones weights.
__device__ __forceinline__ floatx4 block_sums(half8 Ah, half8 Al) {
  const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
  half8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (_Float16)1.f;
  floatx4 s = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, ones, zero, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, ones, s, 0, 0, 0);
}

// Workgroup = 4 waves side by side along n.  Wave tile: 16*MT rows of X by
// 16*NT rows of W; blockIdx.z splits the K blocks.  The block loop runs in
// steps of U blocks whose loads are all issued before the first MFMA, so a
// wave keeps U blocks of weights in flight.
template <int TYPE, int MT, int NT, int U>
__device__ __forceinline__ void gemm_tile(const GemmArgs &a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.x * 4 + wave) * (16 * NT);
  const int m0 = blockIdx.y * (16 * MT);
  const int K = a.B * 32;
  const int per = (a.B + a.KS - 1) / a.KS;
  const int b0 = blockIdx.z * per;
  const int b1 = min(a.B, b0 + per);
  const floatx4 zero = {0.f, 0.f, 0.f, 0.f};

  floatx4 acc[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NT; ++u) acc[t][u] = zero;

  for (int b = b0; b < b1; b += U) {
    typename RawT<TYPE>::type raw[U][NT];
    unsigned dbits[U][NT], mbits[U][NT];
    half8 A[U][MT], Alo[U][MT];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int bb = b + j;
      if (bb < b1) {
#pragma unroll
        for (int u = 0; u < NT; ++u)
          load_codes<TYPE>(a, n0 + 16 * u + li, bb, g, &raw[j][u], &dbits[j][u], &mbits[j][u]);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const size_t off = (size_t)(m0 + 16 * t + li) * K + bb * 32 + 8 * g;
          A[j][t] = *reinterpret_cast<const half8 *>(a.X16 + off);
          Alo[j][t] = *reinterpret_cast<const half8 *>(a.X16lo + off);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      if (b + j < b1) {
        floatx4 xs[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t)
          xs[t] = TYPE == PBX_Q41 ? block_sums(A[j][t], Alo[j][t]) : zero;
#pragma unroll
        for (int u = 0; u < NT; ++u) {
          const half8 W = codes_operand<TYPE>(raw[j][u], g);
          const float d = f16_bits_to_f32(dbits[j][u]);
          const float mn = f16_bits_to_f32(mbits[j][u]);
#pragma unroll
          for (int t = 0; t < MT; ++t) block_mma<TYPE>(acc[t][u], A[j][t], Alo[j][t], W, d, mn, xs[t]);
        }
      }
    }
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
    gemm_tile<TYPE, MT, NT, (MT == 1 ? 8 : 2)>(a);                                  \
  }
GEMM_KERNEL(pbx_gemm_q4_m1_n1, PBX_Q4, 1, 1)
GEMM_KERNEL(pbx_gemm_q4_m1_n2, PBX_Q4, 1, 2)
GEMM_KERNEL(pbx_gemm_q4_m1_n4, PBX_Q4, 1, 4)
GEMM_KERNEL(pbx_gemm_q4_m2_n2, PBX_Q4, 2, 2)
GEMM_KERNEL(pbx_gemm_q8_m1_n1, PBX_Q8, 1, 1)
GEMM_KERNEL(pbx_gemm_q8_m1_n2, PBX_Q8, 1, 2)
GEMM_KERNEL(pbx_gemm_q8_m1_n4, PBX_Q8, 1, 4)
GEMM_KERNEL(pbx_gemm_q8_m2_n2, PBX_Q8, 2, 2)
GEMM_KERNEL(pbx_gemm_q41_m1_n1, PBX_Q41, 1, 1)
GEMM_KERNEL(pbx_gemm_q41_m1_n2, PBX_Q41, 1, 2)
GEMM_KERNEL(pbx_gemm_q41_m1_n4, PBX_Q41, 1, 4)
GEMM_KERNEL(pbx_gemm_q41_m2_n2, PBX_Q41, 2, 2)
GEMM_KERNEL(pbx_gemm_f16_m1_n1, PBX_F16, 1, 1)
GEMM_KERNEL(pbx_gemm_f16_m1_n2, PBX_F16, 1, 2)
GEMM_KERNEL(pbx_gemm_f16_m1_n4, PBX_F16, 1, 4)
GEMM_KERNEL(pbx_gemm_f16_m2_n2, PBX_F16, 2, 2)

// ---------------------------------------------------------------------------
// Large-M kernel (M > 32): workgroup tile 128 (M) x 128 (N), four waves in
// a 2 x 2 arrangement, each wave 64 x 64 (4 x 4 MFMA tiles).  The activation
// tile of a block (128 rows x 32 k, hi and lo, 16 KB) is loaded once per
// workgroup into LDS (double buffered: block b+1 is read from global while
// block b is multiplied) and read by the two waves that share it; each wave
// reads its 64 weight rows' codes one block ahead.  LDS rows are padded to
// 48 halves (measured against 32, 36 and 40).
// Needs X16 / X16lo padded to a multiple of 128 rows.
// ---------------------------------------------------------------------------
#define BIG_TM 128
#define BIG_LDSR 48  // halves per LDS row (32 + 16 padding: fewest bank conflicts measured)

// WN waves along N: 2 (128 x 128 tile, 256 threads).  A 128 x 256 tile
// (WN = 4, 512 threads) measured 35% slower at M = 512 and is not built.
template <int TYPE, int WN>
__device__ __forceinline__ void gemm_big(const GemmArgs &a) {
  constexpr int NTH = 128 * WN;  // threads
  __shared__ __attribute__((aligned(16))) _Float16 As[2][2][BIG_TM * BIG_LDSR];  // [buf][hi/lo]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int wm = wave / WN, wn = wave % WN;
  const int n0 = blockIdx.x * (64 * WN) + wn * 64;
  const int mblk = blockIdx.y * BIG_TM;
  const int m0 = wm * 64;  // within the workgroup tile
  const int K = a.B * 32;
  const int per = (a.B + a.KS - 1) / a.KS;
  const int b0 = blockIdx.z * per;
  const int b1 = min(a.B, b0 + per);
  const floatx4 zero = {0.f, 0.f, 0.f, 0.f};

  // global -> LDS staging: 1024 16-byte chunks per block (2 planes x 128
  // rows x 4 chunks), CH = 1024 / NTH per thread: chunk c = tid + NTH i is
  // plane c / 512, row (c & 511) / 4, 8-half quarter c & 3
  // Thread tid stages chunks c = tid + NTH * i (i < 1024 / NTH): plane c / 512,
  // row (c & 511) / 4, quarter c & 3.  With NTH = 256 the four chunks are
  // (hi, row r), (hi, r + 64), (lo, r), (lo, r + 64); with 512 they are
  // (hi, r) and (lo, r), r = tid / 4.
  const int sq = tid & 3, sr = (tid & 511) >> 2;
  const _Float16 *ghi = a.X16 + (size_t)(mblk + sr) * K + sq * 8;
  const _Float16 *glo = a.X16lo + (size_t)(mblk + sr) * K + sq * 8;
  const size_t g64 = (size_t)64 * K;  // 64 rows further down
  const int lofs = sr * BIG_LDSR + sq * 8, l64 = 64 * BIG_LDSR;
  uint4 st0, st1, st2, st3;
#define BIG_LOAD_A(b)                                                              \
  do {                                                                             \
    st0 = *reinterpret_cast<const uint4 *>(ghi + (b) * 32);                        \
    st2 = *reinterpret_cast<const uint4 *>(glo + (b) * 32);                        \
    if constexpr (NTH == 256) {                                                    \
      st1 = *reinterpret_cast<const uint4 *>(ghi + g64 + (b) * 32);                \
      st3 = *reinterpret_cast<const uint4 *>(glo + g64 + (b) * 32);                \
    }                                                                              \
  } while (0)
#define BIG_STORE_A(buf)                                                           \
  do {                                                                             \
    *reinterpret_cast<uint4 *>(&As[buf][0][lofs]) = st0;                           \
    *reinterpret_cast<uint4 *>(&As[buf][1][lofs]) = st2;                           \
    if constexpr (NTH == 256) {                                                    \
      *reinterpret_cast<uint4 *>(&As[buf][0][lofs + l64]) = st1;                   \
      *reinterpret_cast<uint4 *>(&As[buf][1][lofs + l64]) = st3;                   \
    }                                                                              \
  } while (0)

  floatx4 acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = zero;

  typename RawT<TYPE>::type raw[4];
  unsigned dbits[4], mbits[4];
  if (b0 < b1) {
    BIG_LOAD_A(b0);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      load_codes<TYPE>(a, n0 + 16 * u + li, b0, g, &raw[u], &dbits[u], &mbits[u]);
    BIG_STORE_A(0);
  }
  __syncthreads();
  for (int b = b0; b < b1; ++b) {
    const int buf = (b - b0) & 1;
    const bool more = b + 1 < b1;
    if (more) BIG_LOAD_A(b + 1);
    half8 W[4];
    float d[4], mn[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      W[u] = codes_operand<TYPE>(raw[u], g);
      d[u] = f16_bits_to_f32(dbits[u]);
      mn[u] = f16_bits_to_f32(mbits[u]);
    }
    if (more) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        load_codes<TYPE>(a, n0 + 16 * u + li, b + 1, g, &raw[u], &dbits[u], &mbits[u]);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = m0 + 16 * t + li;
      const half8 Ah = *reinterpret_cast<const half8 *>(&As[buf][0][r * BIG_LDSR + 8 * g]);
      const half8 Al = *reinterpret_cast<const half8 *>(&As[buf][1][r * BIG_LDSR + 8 * g]);
      const floatx4 xs = TYPE == PBX_Q41 ? block_sums(Ah, Al) : zero;
#pragma unroll
      for (int u = 0; u < 4; ++u) block_mma<TYPE>(acc[t][u], Ah, Al, W[u], d[u], mn[u], xs);
    }
    if (more) BIG_STORE_A(buf ^ 1);
    __syncthreads();
  }
#undef BIG_LOAD_A
#undef BIG_STORE_A

#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int n = n0 + 16 * u + li;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int m = mblk + m0 + 16 * t + 4 * g + rr;
        if (m < a.M && n < a.N) {
          const float v = acc[t][u][rr] * a.inv[m];
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

extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q4_big(GemmArgs a) { gemm_big<PBX_Q4, 2>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q8_big(GemmArgs a) { gemm_big<PBX_Q8, 2>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q41_big(GemmArgs a) { gemm_big<PBX_Q41, 2>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_f16_big(GemmArgs a) { gemm_big<PBX_F16, 2>(a); }

// Row scaling to fp16: one workgroup per (padded) row.  The scale is
// 2^(15 - e) with 2^(e-1) <= max|x| < 2^e, so every scaled value is below
// 2^15 in magnitude (fp16 max 65504); padding rows are zero.  X16lo gets
// the residual x*scale - X16 rounded to fp16.
extern "C" __global__ void __launch_bounds__(256)
pbx_gemm_prep_x(const float *X, _Float16 *X16, _Float16 *X16lo, float *inv, int M, int K) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  _Float16 *dst = X16 + (size_t)m * K;
  _Float16 *lo = X16lo + (size_t)m * K;
  if (m >= M) {
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
      dst[k] = (_Float16)0.f;
      lo[k] = (_Float16)0.f;
    }
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
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const float v = src[k] * scale;  // exact: scale is a power of two
    const _Float16 h = (_Float16)v;
    dst[k] = h;
    lo[k] = (_Float16)(v - (float)h);
  }
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

// ---------------------------------------------------------------------------
// F32 weights (engine.js:180-244 tensorMulAdd, wasm-simd.js:94-329 matmul,
// F32 GGUF tensors): v_mfma_f32_16x16x4_f32, exact fp32 products and fp32
// accumulation, no activation preparation.  For a 32-wide k block lane
// (li, g) holds 8 consecutive k (8g .. 8g+7) of activation row li and of
// weight row li; MFMA step j pairs k = 8g + j on both sides, so the eight
// steps cover the block's 32 k (summed in another order, the same sum).
// Operand layout of the 16x16x4 form: A lane l holds A[l%16][l/16], B lane
// l holds B[l/16][l%16], D as the fp16 form.  Workgroup = 4 waves along n,
// wave tile 16*MT x 16*NT, blockIdx.z splits the K blocks.
// ---------------------------------------------------------------------------
struct GemmF32Args {
  const float *W;     // [Npad][K]
  const float *X;     // [M][K]
  const float *bias;  // [N] or null (single split only)
  float *Y;           // KS == 1: [M][N]; else partials [KS][M][N]
  int M, N, Npad, B, KS;
  int accumulate;
};

template <int MT, int NT, int U>
__device__ __forceinline__ void gemm_f32(const GemmF32Args &a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int n0 = (blockIdx.x * 4 + wave) * (16 * NT);
  const int m0 = blockIdx.y * (16 * MT);
  const int K = a.B * 32;
  const int per = (a.B + a.KS - 1) / a.KS;
  const int b0 = blockIdx.z * per;
  const int b1 = min(a.B, b0 + per);
  const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);

  floatx4 acc[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NT; ++u) acc[t][u] = zero;

  for (int b = b0; b < b1; b += U) {
    float4 w[U][NT][2], x[U][MT][2];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const bool blk_ok = b + j < b1;
      const size_t kofs = (size_t)(b + j) * 32 + 8 * g;
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        const int n = n0 + 16 * u + li;
        const float4 *p = reinterpret_cast<const float4 *>(a.W + (size_t)n * K + kofs);
        const bool ok = blk_ok && n < a.Npad;
        w[j][u][0] = ok ? p[0] : z4;
        w[j][u][1] = ok ? p[1] : z4;
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int m = m0 + 16 * t + li;
        const float4 *p = reinterpret_cast<const float4 *>(a.X + (size_t)m * K + kofs);
        const bool ok = blk_ok && m < a.M;
        x[j][t][0] = ok ? p[0] : z4;
        x[j][t][1] = ok ? p[1] : z4;
      }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const float4 &xv = x[j][t][s >> 2];
          const float xs = (s & 3) == 0 ? xv.x : (s & 3) == 1 ? xv.y : (s & 3) == 2 ? xv.z : xv.w;
#pragma unroll
          for (int u = 0; u < NT; ++u) {
            const float4 &wv = w[j][u][s >> 2];
            const float ws = (s & 3) == 0 ? wv.x : (s & 3) == 1 ? wv.y : (s & 3) == 2 ? wv.z : wv.w;
            acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs, ws, acc[t][u], 0, 0, 0);
          }
        }
      }
    }
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
          const float v = acc[t][u][r];
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

#define GEMM_F32_KERNEL(NAME, MT, NT, U)                                           \
  extern "C" __global__ void __launch_bounds__(256) NAME(GemmF32Args a) {          \
    gemm_f32<MT, NT, U>(a);                                                         \
  }
GEMM_F32_KERNEL(pbx_gemm_f32_m1_n1, 1, 1, 4)
GEMM_F32_KERNEL(pbx_gemm_f32_m1_n2, 1, 2, 2)
GEMM_F32_KERNEL(pbx_gemm_f32_m1_n4, 1, 4, 2)
GEMM_F32_KERNEL(pbx_gemm_f32_m2_n2, 2, 2, 2)
GEMM_F32_KERNEL(pbx_gemm_f32_m4_n4, 4, 4, 1)
