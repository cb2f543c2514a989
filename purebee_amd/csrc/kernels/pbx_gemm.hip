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
// Large-M kernel (M > 32): 32x32x16 MFMAs with every operand moved to LDS
// by DMA.  Operand lane layout of v_mfma_f32_32x32x16_f16 (checked on
// the device): A: lane l holds A[l%32][8*(l/32) + e]; B: lane l holds
// B[8*(l/32) + e][l%32]; D: lane l, register r holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32].  A 32-wide block is two MFMAs per
// operand: j = 0 takes k = 8h + e and j = 1 takes k = 16 + 8h + e
// (h = l/32), which are the low and high nibbles of the Q4_0 / Q4_1 bytes
// 8h..8h+7 (a lane reads its 8 code bytes once), the Q8_0 bytes 8h.. and
// 16+8h.., the F16 halves likewise.  Each lane's 16 outputs share one column
// (weight row), so the block scale is one value per lane.
// Workgroup tile MT (M, 128 or 64) x 128 (N), four waves in 2 x 2, wave tile
// MT / 2 x 64 (MT / 64 x 2 MFMA tiles).  A ring of NS LDS stages, each
// [hi/lo][MT rows][4 chunks of 8 halves] of activations, the 128 weight rows'
// code bytes (or F16 weights) and their scales (and Q4_1 mins).  Per block
// every wave issues the same number of DMA instructions (global_load_lds:
// lane i's bytes land at the instruction's LDS base + size * i): MT / 32
// activation chunks and its share of the weight data (DmaW), so one wait
// count fits every wave;
// the loads are issued from inline assembly with SGPR bases, so
// the compiler adds no waits of its own, and no register load is in flight
// across the block loop.  The chunks of activation row r are stored in the
// order q ^ swz(r), swz(r) = ((r >> 1) ^ (r >> 3)) & 3: the 16-byte reads of
// 16 consecutive rows at one chunk fall in 16 distinct bank groups.  The
// loop is unrolled by NS so every LDS offset is an immediate.
// Needs X16 / X16lo padded to a multiple of 128 rows.
// ---------------------------------------------------------------------------
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int a_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

__device__ __forceinline__ unsigned lds_addr(const void *p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// LDS DMA with a uniform 64-bit base in SGPRs and a per-lane 32-bit offset
// (the saddr form): lane i's SIZE bytes from base + voff land at LDS byte
// address m0 + SIZE * i.  m0 must be wave-uniform.
template <int SIZE>
__device__ __forceinline__ void dma_to_lds_s(const void *base, unsigned voff, unsigned m0) {
  if constexpr (SIZE == 16)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 ::"v"(voff), "s"(base), "s"(m0));
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
                 ::"v"(voff), "s"(base), "s"(m0));
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Weight bytes of one row and block in the stage: Q4_0 / Q4_1 16 code bytes,
// Q8_0 32, F16 64 (the fp16 weights); per-block scales (and Q4_1 mins) follow.
template <int TYPE> struct DmaW {
  static constexpr int CB = TYPE == PBX_F16 ? 64 : TYPE == PBX_Q8 ? 32 : 16;
  static constexpr int CODES = 128 * CB;                  // bytes of a stage
  static constexpr int NSC = TYPE == PBX_F16 ? 0 : TYPE == PBX_Q41 ? 2 : 1;  // 256-byte planes
  static constexpr int WD = TYPE == PBX_Q8 || TYPE == PBX_F16 ? 2 : 1;      // weight DMAs a wave
};

// SW: the gate|up weight of a Llama FFN (N / 2 gate rows, then N / 2 up
// rows), with silu(gate) * up in the epilogue.  Workgroup x takes hidden
// columns [64 x, 64 x + 64): tile rows 0-31 are their first 32 gate rows,
// 32-63 the matching up rows, 64-127 the same for the next 32 columns, so a
// wave's two 32-column subtiles (u = 0, 1) hold a gate and its up for one
// lane's column; Y is [M][N / 2].  Needs N / 2 a multiple of 64 and no K
// split.
template <int TYPE, int NS, int MT = 128, bool SW = false>
__device__ __forceinline__ void gemm_dma(const GemmArgs &a) {
  static_assert(MT == 128 || MT == 64, "M tile");
  typedef DmaW<TYPE> W;
  constexpr int NA = MT / 64;                                     // activation chunks a wave and plane
  constexpr int TT = MT / 64;                                     // 32-row MFMA tiles a wave
  constexpr int PS = MT * 32 * 2;                                 // bytes of a stage's hi (or lo) plane
  constexpr int ASTAGE = 2 * PS;                                  // bytes
  constexpr int STAGE = ASTAGE + W::CODES + 256 * W::NSC;         // bytes
  constexpr int PER = 2 * NA + W::WD;                             // DMA instructions a wave and block
  __shared__ __attribute__((aligned(1024))) uint8_t S[NS * STAGE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: SGPR bases
  const int lr = lane & 31, h = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * 128 + wn * 64;
  const int mblk = blockIdx.y * MT;
  const int m0 = wm * (MT / 2);
  const int K = a.B * 32;
  const int per = (a.B + a.KS - 1) / a.KS;
  const int b0 = blockIdx.z * per;
  const int b1 = min(a.B, b0 + per);
  const floatx16 zero16 = {};

  floatx16 acc[TT][2];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) acc[t][u] = zero16;

  if (b0 < b1) {
    // activation DMA i (i < NA) of this wave and plane: LDS chunks
    // (4 i + wave) * 64 + lane; per-lane byte offset from the plane's tile base
    unsigned avoff[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int c = (4 * i + wave) * 64 + lane;  // plane 0 chunk (same offsets in plane 1)
      const int r = c >> 2, q = (c & 3) ^ a_swz(r);
      avoff[i] = (unsigned)((r * K + q * 8) * 2);
    }
    const uint8_t *xhi = reinterpret_cast<const uint8_t *>(a.X16 + (size_t)mblk * K);
    const uint8_t *xlo = reinterpret_cast<const uint8_t *>(a.X16lo + (size_t)mblk * K);
    // Weight DMAs of this wave (bases at the workgroup's first row, so the
    // per-lane offsets stay small).  Code DMA d moves 1 KB: rows
    // (1024 / CB) d + lane / (CB / 16), 16-byte chunk lane % (CB / 16), into
    // the row-major [128][CB] code area.  A plane DMA moves the 128 rows'
    // fp16 scales (or Q4_1 mins): lane i takes dword i & 1 of four-row group
    // i >> 1.  Q4_0: waves 0, 1 codes, waves 2, 3 scales (the same bytes);
    // Q4_1: waves 0, 1 codes, wave 2 scales, wave 3 mins; Q8_0: codes d = wave
    // and the scales; F16: codes d = 2 wave, 2 wave + 1.
    const uint8_t *wb[2];
    unsigned wv[2], wl[2];
    int wstep[2], wsz[2];
    const size_t rowbytes = (size_t)a.B * W::CB;
    // SW: the weight row of tile row i (the gate or up rows of the
    // workgroup's hidden columns; relative to row 0)
    auto sw_row = [&](int i) -> int {
      const int c = i >> 5;
      return ((c & 1) ? a.N / 2 : 0) + blockIdx.x * 64 + 32 * (c >> 1) + (i & 31);
    };
    auto code_dma = [&](int k, int d) {
      const int per_row = W::CB / 16;
      const int i = (1024 / W::CB) * d + lane / per_row;  // tile row
      if constexpr (SW) {
        wb[k] = a.qs;
        wv[k] = (unsigned)((size_t)sw_row(i) * rowbytes + (lane % per_row) * 16);
      } else {
        const int n = min(blockIdx.x * 128 + i, a.Npad - 1) - blockIdx.x * 128;
        wb[k] = a.qs + (size_t)blockIdx.x * 128 * rowbytes;
        wv[k] = (unsigned)(n * rowbytes + (lane % per_row) * 16);
      }
      wl[k] = ASTAGE + d * 1024;
      wstep[k] = W::CB;
      wsz[k] = 16;
    };
    auto plane_dma = [&](int k, const uint16_t *plane, int which) {
      if constexpr (SW) {
        // four-row group lane >> 1 of the tile: four consecutive weight rows
        wb[k] = reinterpret_cast<const uint8_t *>(plane);
        wv[k] = (unsigned)((size_t)(sw_row(4 * (lane >> 1)) >> 2) * a.B * 8 + (lane & 1) * 4);
      } else {
        const int g = min(blockIdx.x * 32 + (lane >> 1), a.Npad / 4 - 1) - blockIdx.x * 32;
        wb[k] = reinterpret_cast<const uint8_t *>(plane) + (size_t)blockIdx.x * 32 * a.B * 8;
        wv[k] = (unsigned)(g * a.B * 8 + (lane & 1) * 4);
      }
      wl[k] = ASTAGE + W::CODES + 256 * which;
      wstep[k] = 8;
      wsz[k] = 4;
    };
    if constexpr (TYPE == PBX_Q4) {
      if (wave < 2) code_dma(0, wave);
      else plane_dma(0, a.dsc, 0);
    } else if constexpr (TYPE == PBX_Q41) {
      if (wave < 2) code_dma(0, wave);
      else if (wave == 2) plane_dma(0, a.dsc, 0);
      else plane_dma(0, a.msc, 1);
    } else if constexpr (TYPE == PBX_Q8) {
      code_dma(0, wave);
      plane_dma(1, a.dsc, 0);
    } else {
      code_dma(0, 2 * wave);
      code_dma(1, 2 * wave + 1);
    }
    const unsigned lbase = lds_addr(&S[0]);
    const unsigned lds0 = __builtin_amdgcn_readfirstlane(lbase + wave * 1024);
    unsigned ldw[2];
#pragma unroll
    for (int k = 0; k < W::WD; ++k) ldw[k] = __builtin_amdgcn_readfirstlane(lbase + wl[k]);
    auto dma = [&](int b, int stage) {
      const unsigned so = stage * STAGE;
#pragma unroll
      for (int i = 0; i < NA; ++i) dma_to_lds_s<16>(xhi + b * 64, avoff[i], lds0 + so + 4096 * i);
#pragma unroll
      for (int i = 0; i < NA; ++i)
        dma_to_lds_s<16>(xlo + b * 64, avoff[i], lds0 + so + PS + 4096 * i);
#pragma unroll
      for (int k = 0; k < W::WD; ++k) {
        if (wsz[k] == 16)
          dma_to_lds_s<16>(wb[k] + (size_t)b * wstep[k], wv[k], ldw[k] + so);
        else
          dma_to_lds_s<4>(wb[k] + (size_t)b * wstep[k], wv[k], ldw[k] + so);
      }
    };
    // this lane's read offsets in a stage
    const uint8_t *rbase = &S[0];
    int aoff[TT][2];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = m0 + 32 * t + lr;
        aoff[t][j] = (r * 32 + (((2 * j + h) ^ a_swz(r)) * 8)) * 2;
      }
    int sofs[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) sofs[u] = ASTAGE + W::CODES + (wn * 64 + 32 * u + lr) * 2;

#pragma unroll
    for (int s = 0; s < NS - 1; ++s) dma(min(b0 + s, b1 - 1), s);

    for (int kb = b0; kb < b1; kb += NS) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int b = kb + s;
        if (b >= b1) break;
        wait_vm<(NS - 2) * PER>();
        lds_barrier();
        dma(min(b + NS - 1, b1 - 1), s == 0 ? NS - 1 : s - 1);
        const uint8_t *sb = rbase + s * STAGE;
        half8 B0[2], B1[2];
        float d[2], mn[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint8_t *wr = sb + ASTAGE + (wn * 64 + 32 * u + lr) * W::CB;
          if constexpr (TYPE == PBX_F16) {
            B0[u] = *reinterpret_cast<const half8 *>(wr + 16 * h);
            B1[u] = *reinterpret_cast<const half8 *>(wr + 32 + 16 * h);
            d[u] = 1.f;
          } else {
            if constexpr (TYPE == PBX_Q8) {
              B0[u] = codes_operand<PBX_Q8>(*reinterpret_cast<const uint2 *>(wr + 8 * h), 0);
              B1[u] = codes_operand<PBX_Q8>(*reinterpret_cast<const uint2 *>(wr + 16 + 8 * h), 0);
            } else {
              const uint2 raw = *reinterpret_cast<const uint2 *>(wr + 8 * h);
              B0[u] = codes_operand<TYPE>(raw, 0);  // low nibbles
              B1[u] = codes_operand<TYPE>(raw, 2);  // high nibbles
            }
            d[u] = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(sb + sofs[u]));
          }
          mn[u] = TYPE == PBX_Q41 ? f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(sb + sofs[u] + 256))
                                  : 0.f;
        }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          const half8 Ah0 = *reinterpret_cast<const half8 *>(sb + aoff[t][0]);
          const half8 Ah1 = *reinterpret_cast<const half8 *>(sb + aoff[t][1]);
          const half8 Al0 = *reinterpret_cast<const half8 *>(sb + PS + aoff[t][0]);
          const half8 Al1 = *reinterpret_cast<const half8 *>(sb + PS + aoff[t][1]);
          floatx16 xs = zero16;
          if constexpr (TYPE == PBX_Q41) {
            // the block sums of the activation rows: the product with all-ones weights
            half8 ones;
#pragma unroll
            for (int e = 0; e < 8; ++e) ones[e] = (_Float16)1.f;
            xs = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ah0, ones, xs, 0, 0, 0);
            xs = __builtin_amdgcn_mfma_f32_32x32x16_f16(Al0, ones, xs, 0, 0, 0);
            xs = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ah1, ones, xs, 0, 0, 0);
            xs = __builtin_amdgcn_mfma_f32_32x32x16_f16(Al1, ones, xs, 0, 0, 0);
          }
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            if constexpr (TYPE == PBX_F16) {
              acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ah0, B0[u], acc[t][u], 0, 0, 0);
              acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Al0, B0[u], acc[t][u], 0, 0, 0);
              acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ah1, B1[u], acc[t][u], 0, 0, 0);
              acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Al1, B1[u], acc[t][u], 0, 0, 0);
            } else {
              floatx16 blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ah0, B0[u], zero16, 0, 0, 0);
              blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(Al0, B0[u], blk, 0, 0, 0);
              blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ah1, B1[u], blk, 0, 0, 0);
              blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(Al1, B1[u], blk, 0, 0, 0);
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                acc[t][u][r] = fmaf(blk[r], d[u], acc[t][u][r]);
                if constexpr (TYPE == PBX_Q41) acc[t][u][r] = fmaf(xs[r], mn[u], acc[t][u][r]);
              }
            }
          }
        }
      }
    }
    wait_vm<0>();
  }

  if constexpr (SW) {
    const int NO = a.N / 2, c = blockIdx.x * 64 + 32 * wn + lr;  // the lane's hidden column
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mblk + m0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m < a.M) {
          const float iv = a.inv[m];
          a.Y[(size_t)m * NO + c] = silu(acc[t][0][r] * iv) * (acc[t][1][r] * iv);
        }
      }
    return;
  }
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int n = n0 + 32 * u + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mblk + m0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
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

extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q4_big(GemmArgs a) { gemm_dma<PBX_Q4, 3>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q8_big(GemmArgs a) { gemm_dma<PBX_Q8, 3>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q41_big(GemmArgs a) { gemm_dma<PBX_Q41, 3>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_f16_big(GemmArgs a) { gemm_dma<PBX_F16, 3>(a); }
// 64-row M tiles: twice the workgroups of the 128-row tile for the GEMMs
// whose 128 x 128 grid leaves CUs idle (o, q|k|v and down at a 512-token
// prompt), without a deeper K split
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q4_b64(GemmArgs a) { gemm_dma<PBX_Q4, 3, 64>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q8_b64(GemmArgs a) { gemm_dma<PBX_Q8, 3, 64>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q41_b64(GemmArgs a) { gemm_dma<PBX_Q41, 3, 64>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_f16_b64(GemmArgs a) { gemm_dma<PBX_F16, 3, 64>(a); }
// gate|up with silu(gate) * up in the epilogue (no K split; Y is [M][N / 2])
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q4_big_sw(GemmArgs a) { gemm_dma<PBX_Q4, 3, 128, true>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q8_big_sw(GemmArgs a) { gemm_dma<PBX_Q8, 3, 128, true>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q41_big_sw(GemmArgs a) { gemm_dma<PBX_Q41, 3, 128, true>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_f16_big_sw(GemmArgs a) { gemm_dma<PBX_F16, 3, 128, true>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q4_b64_sw(GemmArgs a) { gemm_dma<PBX_Q4, 3, 64, true>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q8_b64_sw(GemmArgs a) { gemm_dma<PBX_Q8, 3, 64, true>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_q41_b64_sw(GemmArgs a) { gemm_dma<PBX_Q41, 3, 64, true>(a); }
extern "C" __global__ void __launch_bounds__(256) pbx_gemm_f16_b64_sw(GemmArgs a) { gemm_dma<PBX_F16, 3, 64, true>(a); }

// Row scaling to fp16: one workgroup per (padded) row.  The scale is
// 2^(15 - e) with 2^(e-1) <= max|x| < 2^e, so every scaled value is below
// 2^15 in magnitude (fp16 max 65504); padding rows are zero.  X16lo gets
// the residual x*scale - X16 rounded to fp16.  The row is held in registers
// (PREP_R float4s a thread, K <= 1024 * PREP_R), so it is read once;
// pbx_gemm_prep_x reads longer rows twice.  The
// variants compute the row first: RMSNorm of a residual row (optionally
// after adding split-K partials into it), or SwiGLU of a gate|up row.
#define PREP_R 8
typedef _Float16 half4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void prep_zero_row(_Float16 *dst, _Float16 *lo, float *inv, int K4) {
  const half4v z = {};
  for (int k = threadIdx.x; k < K4; k += 256) {
    reinterpret_cast<half4v *>(dst)[k] = z;
    reinterpret_cast<half4v *>(lo)[k] = z;
  }
  if (threadIdx.x == 0) *inv = 0.f;
}

__device__ __forceinline__ float block_sum256(float v, float *red) {
  v = wave_sum(v);
  __syncthreads();  // red may still be read from an earlier reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float max4(float4 t) {
  return fmaxf(fmaxf(fabsf(t.x), fabsf(t.y)), fmaxf(fabsf(t.z), fabsf(t.w)));
}

// Scale and split the row v (element 4 (tid + 256 i) + c of float4 i) into
// dst / lo, and write the power of two that undoes the scale.
__device__ __forceinline__ void prep_split_row(const float4 (&v)[PREP_R], int K4, _Float16 *dst,
                                               _Float16 *lo, float *inv, float *red) {
  const int tid = threadIdx.x;
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < PREP_R; ++i) mx = fmaxf(mx, max4(v[i]));  // unused slots hold zeros
  mx = wave_max(mx);
  __syncthreads();
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (mx > 0.f && mx < INFINITY) frexpf(mx, &e);
  const float scale = mx > 0.f ? ldexpf(1.f, 15 - e) : 1.f;
#pragma unroll
  for (int i = 0; i < PREP_R; ++i) {
    const int k = tid + 256 * i;
    if (k < K4) {
      // exact: scale is a power of two
      const float a0 = v[i].x * scale, a1 = v[i].y * scale, a2 = v[i].z * scale, a3 = v[i].w * scale;
      const half4v hv = {(_Float16)a0, (_Float16)a1, (_Float16)a2, (_Float16)a3};
      const half4v lv = {(_Float16)(a0 - (float)hv[0]), (_Float16)(a1 - (float)hv[1]),
                         (_Float16)(a2 - (float)hv[2]), (_Float16)(a3 - (float)hv[3])};
      reinterpret_cast<half4v *>(dst)[k] = hv;
      reinterpret_cast<half4v *>(lo)[k] = lv;
    }
  }
  if (tid == 0) *inv = mx > 0.f ? ldexpf(1.f, e - 15) : 1.f;
}

__device__ __forceinline__ void load_row(const float *x, int K4, float4 (&v)[PREP_R]) {
#pragma unroll
  for (int i = 0; i < PREP_R; ++i) {
    const int k = threadIdx.x + 256 * i;
    v[i] = k < K4 ? reinterpret_cast<const float4 *>(x)[k] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// RMSNorm of v in place (llama.js rmsnorm: x * (1 / sqrt(mean(x^2) + eps)) * w).
__device__ __forceinline__ void rms_row(float4 (&v)[PREP_R], const float *w, int K4, float eps,
                                        float *red) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PREP_R; ++i) {
    ss = fmaf(v[i].x, v[i].x, ss);
    ss = fmaf(v[i].y, v[i].y, ss);
    ss = fmaf(v[i].z, v[i].z, ss);
    ss = fmaf(v[i].w, v[i].w, ss);
  }
  ss = block_sum256(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)(4 * K4) + eps);
#pragma unroll
  for (int i = 0; i < PREP_R; ++i) {
    const int k = threadIdx.x + 256 * i;
    if (k < K4) {
      const float4 g = reinterpret_cast<const float4 *>(w)[k];
      v[i] = make_float4(v[i].x * r * g.x, v[i].y * r * g.y, v[i].z * r * g.z, v[i].w * r * g.w);
    }
  }
}

extern "C" __global__ void __launch_bounds__(256)
pbx_gemm_prep_x(const float *X, _Float16 *X16, _Float16 *X16lo, float *inv, int M, int K) {
  __shared__ float red[4];
  const int m = blockIdx.x, K4 = K / 4;  // K is a multiple of 32, at most 1024 * PREP_R
  _Float16 *dst = X16 + (size_t)m * K, *lo = X16lo + (size_t)m * K;
  if (m >= M) return prep_zero_row(dst, lo, inv + m, K4);
  if (K4 > 256 * PREP_R) {
    // longer rows: read twice
    const float4 *src = reinterpret_cast<const float4 *>(X + (size_t)m * K);
    float mx = 0.f;
    for (int k = threadIdx.x; k < K4; k += 256) mx = fmaxf(mx, max4(src[k]));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.f && mx < INFINITY) frexpf(mx, &e);
    const float scale = mx > 0.f ? ldexpf(1.f, 15 - e) : 1.f;
    for (int k = threadIdx.x; k < K4; k += 256) {
      const float4 t = src[k];
      const float a0 = t.x * scale, a1 = t.y * scale, a2 = t.z * scale, a3 = t.w * scale;
      const half4v hv = {(_Float16)a0, (_Float16)a1, (_Float16)a2, (_Float16)a3};
      const half4v lv = {(_Float16)(a0 - (float)hv[0]), (_Float16)(a1 - (float)hv[1]),
                         (_Float16)(a2 - (float)hv[2]), (_Float16)(a3 - (float)hv[3])};
      reinterpret_cast<half4v *>(dst)[k] = hv;
      reinterpret_cast<half4v *>(lo)[k] = lv;
    }
    if (threadIdx.x == 0) inv[m] = mx > 0.f ? ldexpf(1.f, e - 15) : 1.f;
    return;
  }
  float4 v[PREP_R];
  load_row(X + (size_t)m * K, K4, v);
  prep_split_row(v, K4, dst, lo, inv + m, red);
}

// X16 rows of RMSNorm(x) * w (K <= 1024 * PREP_R).
extern "C" __global__ void __launch_bounds__(256)
pbx_gemm_prep_rms(const float *X, const float *normw, float eps, _Float16 *X16, _Float16 *X16lo,
                  float *inv, int M, int K) {
  __shared__ float red[4];
  const int m = blockIdx.x, K4 = K / 4;
  _Float16 *dst = X16 + (size_t)m * K, *lo = X16lo + (size_t)m * K;
  if (m >= M) return prep_zero_row(dst, lo, inv + m, K4);
  float4 v[PREP_R];
  load_row(X + (size_t)m * K, K4, v);
  rms_row(v, normw, K4, eps, red);
  prep_split_row(v, K4, dst, lo, inv + m, red);
}

// x[m] += the sum of the KS split-K partials of row m (the residual add of a
// split GEMM, summed in split order like pbx_gemm_reduce); then, if normw,
// the X16 row of RMSNorm(x[m]) * normw for the next GEMM.
extern "C" __global__ void __launch_bounds__(256)
pbx_gemm_reduce_rms(const float *part, int KS, float *X, const float *normw, float eps,
                    _Float16 *X16, _Float16 *X16lo, float *inv, int M, int K) {
  __shared__ float red[4];
  const int m = blockIdx.x, K4 = K / 4;
  _Float16 *dst = X16 + (size_t)m * K, *lo = X16lo + (size_t)m * K;
  if (m >= M) {
    if (normw) prep_zero_row(dst, lo, inv + m, K4);
    return;
  }
  float4 v[PREP_R];
  float *x = X + (size_t)m * K;
  const size_t MK = (size_t)M * K;
#pragma unroll
  for (int i = 0; i < PREP_R; ++i) {
    const int k = threadIdx.x + 256 * i;
    if (k < K4) {
      // every partial load issued before the sum (KS <= 8)
      float4 pp[8];
#pragma unroll
      for (int p = 0; p < 8; ++p)
        pp[p] = p < KS ? reinterpret_cast<const float4 *>(part + p * MK + (size_t)m * K)[k]
                       : make_float4(0.f, 0.f, 0.f, 0.f);
      float4 s = pp[0];
#pragma unroll
      for (int p = 1; p < 8; ++p)
        if (p < KS) {
          s.x += pp[p].x; s.y += pp[p].y; s.z += pp[p].z; s.w += pp[p].w;
        }
      float4 r = reinterpret_cast<float4 *>(x)[k];
      r.x += s.x; r.y += s.y; r.z += s.z; r.w += s.w;
      reinterpret_cast<float4 *>(x)[k] = r;
      v[i] = r;
    } else {
      v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  if (!normw) return;
  rms_row(v, normw, K4, eps, red);
  prep_split_row(v, K4, dst, lo, inv + m, red);
}

// X16 rows of silu(gate) * up from gate|up rows [M][2 * hidden] (llama.js:329-333).
extern "C" __global__ void __launch_bounds__(256)
pbx_gemm_prep_swiglu(const float *GU, _Float16 *X16, _Float16 *X16lo, float *inv, int M,
                     int hidden) {
  __shared__ float red[4];
  const int m = blockIdx.x, K4 = hidden / 4;
  _Float16 *dst = X16 + (size_t)m * hidden, *lo = X16lo + (size_t)m * hidden;
  if (m >= M) return prep_zero_row(dst, lo, inv + m, K4);
  const float4 *g4 = reinterpret_cast<const float4 *>(GU + (size_t)m * 2 * hidden);
  const float4 *u4 = g4 + K4;
  float4 v[PREP_R];
#pragma unroll
  for (int i = 0; i < PREP_R; ++i) {
    const int k = threadIdx.x + 256 * i;
    if (k < K4) {
      const float4 g = g4[k], u = u4[k];
      v[i] = make_float4(silu(g.x) * u.x, silu(g.y) * u.y, silu(g.z) * u.z, silu(g.w) * u.w);
    } else {
      v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  prep_split_row(v, K4, dst, lo, inv + m, red);
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

// F32 weights, M > 32: v_mfma_f32_32x32x2f32 (A: lane l holds A[l%32][l/32];
// B: lane l holds B[l/32][l%32]; D as the f16 32x32 form; checked on the
// device) with every operand moved to LDS by DMA, the tiling of gemm_dma.
// A stage covers 16 k: the activation tile [128 rows][4 chunks of 4 floats]
// and the weight tile [128 rows][4 chunks], chunks stored in the order
// q ^ swz(row).  Within a group of 8 k (chunks 2g, 2g + 1) lane (r, h)
// reads chunk 2g + h of its row as one float4 and MFMA i (i < 4) takes its
// element i, i.e. k = 8g + 4h + i: every k of the group is used once per
// output.  Each wave issues four DMA instructions a stage (two activation
// and two weight kilobytes).  Rows past M (activations) or Npad (weights)
// are clamped.
template <int NS>
__device__ __forceinline__ void gemm_f32_dma(const GemmF32Args &a) {
  constexpr int TILE = 128 * 64;      // bytes of one operand tile
  constexpr int STAGE = 2 * TILE;     // activations, weights
  __shared__ __attribute__((aligned(1024))) uint8_t S[NS * STAGE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, h = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * 128 + wn * 64;
  const int mblk = blockIdx.y * 128;
  const int m0 = wm * 64;
  const int K = a.B * 32, steps = 2 * a.B;  // 16 k a step
  const int per = (steps + a.KS - 1) / a.KS;
  const int s0 = blockIdx.z * per;
  const int s1 = min(steps, s0 + per);
  const floatx16 zero16 = {};
  floatx16 acc[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) acc[t][u] = zero16;

  if (s0 < s1) {
    // DMA k (k = 0, 1) of this wave for each tile: rows 16 (2 wave + k) + lane / 4
    const uint8_t *xb = reinterpret_cast<const uint8_t *>(a.X) + (size_t)mblk * K * 4;
    const uint8_t *wb = reinterpret_cast<const uint8_t *>(a.W) + (size_t)blockIdx.x * 128 * K * 4;
    unsigned xv[2], wv[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int row = 16 * (2 * wave + k) + (lane >> 2), q = (lane & 3) ^ a_swz(row);
      const int xr = min(mblk + row, a.M - 1) - mblk;
      const int wr = min(blockIdx.x * 128 + row, a.Npad - 1) - blockIdx.x * 128;
      xv[k] = (unsigned)((xr * K + 4 * q) * 4);
      wv[k] = (unsigned)((wr * K + 4 * q) * 4);
    }
    const unsigned lbase = lds_addr(&S[0]);
    const unsigned ldx = __builtin_amdgcn_readfirstlane(lbase + wave * 2048);
    auto dma = [&](int st, int stage) {
      const unsigned so = stage * STAGE;
      const size_t ko = (size_t)st * 64;  // 16 floats
      dma_to_lds_s<16>(xb + ko, xv[0], ldx + so);
      dma_to_lds_s<16>(xb + ko, xv[1], ldx + so + 1024);
      dma_to_lds_s<16>(wb + ko, wv[0], ldx + so + TILE);
      dma_to_lds_s<16>(wb + ko, wv[1], ldx + so + TILE + 1024);
    };
    int aoff[2][2], boff[2][2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int r = m0 + 32 * t + lr;
        aoff[g][t] = r * 64 + (((2 * g + h) ^ a_swz(r)) * 16);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int r = wn * 64 + 32 * u + lr;
        boff[g][u] = TILE + r * 64 + (((2 * g + h) ^ a_swz(r)) * 16);
      }
    }
    const uint8_t *rbase = &S[0];
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) dma(min(s0 + st, s1 - 1), st);
    for (int kb = s0; kb < s1; kb += NS) {
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const int b = kb + st;
        if (b >= s1) break;
        wait_vm<(NS - 2) * 4>();
        lds_barrier();
        dma(min(b + NS - 1, s1 - 1), st == 0 ? NS - 1 : st - 1);
        const uint8_t *sb = rbase + st * STAGE;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          float4 av[2], bv[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) av[t] = *reinterpret_cast<const float4 *>(sb + aoff[g][t]);
#pragma unroll
          for (int u = 0; u < 2; ++u) bv[u] = *reinterpret_cast<const float4 *>(sb + boff[g][u]);
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[t].x, bv[u].x, acc[t][u], 0, 0, 0);
              acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[t].y, bv[u].y, acc[t][u], 0, 0, 0);
              acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[t].z, bv[u].z, acc[t][u], 0, 0, 0);
              acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[t].w, bv[u].w, acc[t][u], 0, 0, 0);
            }
        }
      }
    }
    wait_vm<0>();
  }

#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int n = n0 + 32 * u + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mblk + m0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
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

extern "C" __global__ void __launch_bounds__(256) pbx_gemm_f32_big(GemmF32Args a) { gemm_f32_dma<3>(a); }

// ---------------------------------------------------------------------------
// Skinny Q4_0 GEMM for 1..8 activation rows (speculative verify, short
// batches): the rows of a layer input are normalised once per workgroup
// (RMSNorm when normw is given), scaled per row by a power of two and held in
// LDS as fp16 pairs (hi, lo) in chunks of SK_KC columns; the weights stream
// through v_mfma_f32_32x32x16_f16 (operand layout of gemm_dma) 32 weight rows
// a tile, the four waves of a workgroup splitting the tile's blocks.  A rows
// 8..31 of the MFMA read an all-zero LDS row, so of a lane's 16 outputs only
// registers 0..3 (activation rows 4h + r) carry results and take the block
// scale.  Epilogues: store, add (residual) or SwiGLU of the gate|up pair
// (a tile holds 16 gate and the matching 16 up rows).  K above SK_KC runs one
// tile per workgroup, the chunks converted in turn.
// ---------------------------------------------------------------------------
#define SK_MR 8
#define SK_KC 2048
#define SK_LD (SK_KC + 8)  // halves per LDS row

struct SkinnyArgs {
  const uint8_t *qs;     // Q4_0 code plane [Npad][B][16]
  const uint16_t *dsc;   // fp16 scales (4-row groups)
  const float *X;        // [M][K]
  const float *normw;    // [K] or null
  float *Y;              // [M][ldy]
  int N, B, M, ldy;
  float eps;
};

enum { SK_STORE = 0, SK_ADD = 1, SK_SWIGLU = 2 };

template <int EPI>
__device__ __forceinline__ void skinny_q4(const SkinnyArgs &a) {
  __shared__ __attribute__((aligned(16))) _Float16 Ah[SK_MR + 1][SK_LD], Al[SK_MR + 1][SK_LD];
  __shared__ float rs_scale[SK_MR], rs_inv[SK_MR], rs_norm[SK_MR];
  __shared__ float wred[4][SK_MR][2];
  __shared__ float tred[3][64][4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, h = lane >> 5;
  const int M = a.M, B = a.B, K = B * 32, K4 = K / 4;
  const bool norm = a.normw != nullptr;

  // 1. per-row statistics: sum of squares (RMSNorm) and the largest |x w|.
  // Rows of at most SK_KC columns are loaded once into registers (item j of
  // a thread: row j / 2, float4 column tid + 256 (j % 2)) and converted from
  // there; longer rows are read twice (statistics, then chunk by chunk).
  constexpr int IT = SK_MR * SK_KC / 4 / 256;  // 16 float4 items a thread
  const bool one = K <= SK_KC;
  float4 xr[IT], gr[2];
  float ss[SK_MR], mx[SK_MR];
#pragma unroll
  for (int m = 0; m < SK_MR; ++m) {
    ss[m] = 0.f;
    mx[m] = 0.f;
  }
  if (one) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int k4 = tid + 256 * q;
      gr[q] = norm && k4 < K4 ? reinterpret_cast<const float4 *>(a.normw)[k4] : make_float4(1.f, 1.f, 1.f, 1.f);
    }
#pragma unroll
    for (int j = 0; j < IT; ++j) {
      const int m = j >> 1, k4 = tid + 256 * (j & 1);
      xr[j] = m < M && k4 < K4 ? reinterpret_cast<const float4 *>(a.X + (size_t)m * K)[k4]
                              : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < IT; ++j) {
      const int m = j >> 1;
      const float4 x = xr[j], g = gr[j & 1];
      ss[m] = fmaf(x.x, x.x, fmaf(x.y, x.y, fmaf(x.z, x.z, fmaf(x.w, x.w, ss[m]))));
      mx[m] = fmaxf(mx[m], fmaxf(fmaxf(fabsf(x.x * g.x), fabsf(x.y * g.y)),
                                 fmaxf(fabsf(x.z * g.z), fabsf(x.w * g.w))));
    }
  } else {
#pragma unroll 4
    for (int k = tid; k < K4; k += 256) {
      const float4 g = norm ? reinterpret_cast<const float4 *>(a.normw)[k] : make_float4(1.f, 1.f, 1.f, 1.f);
#pragma unroll
      for (int m = 0; m < SK_MR; ++m) {
        if (m < M) {
          const float4 x = reinterpret_cast<const float4 *>(a.X + (size_t)m * K)[k];
          ss[m] = fmaf(x.x, x.x, fmaf(x.y, x.y, fmaf(x.z, x.z, fmaf(x.w, x.w, ss[m]))));
          mx[m] = fmaxf(mx[m], fmaxf(fmaxf(fabsf(x.x * g.x), fabsf(x.y * g.y)),
                                     fmaxf(fabsf(x.z * g.z), fabsf(x.w * g.w))));
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < SK_MR; ++m) {
    const float s = wave_sum(ss[m]), x = wave_max(mx[m]);
    if (lane == 0) {
      wred[wave][m][0] = s;
      wred[wave][m][1] = x;
    }
  }
  __syncthreads();
  if (tid < SK_MR) {
    const int m = tid;
    const float s = (wred[0][m][0] + wred[1][m][0]) + (wred[2][m][0] + wred[3][m][0]);
    const float x = fmaxf(fmaxf(wred[0][m][1], wred[1][m][1]), fmaxf(wred[2][m][1], wred[3][m][1]));
    const float r = norm ? 1.0f / sqrtf(s / (float)K + a.eps) : 1.f;
    const float vmax = x * r;  // the row's largest magnitude after normalisation
    int e = 0;
    if (vmax > 0.f && vmax < INFINITY) frexpf(vmax, &e);
    rs_norm[m] = r;
    rs_scale[m] = vmax > 0.f ? ldexpf(1.f, 15 - e) : 1.f;
    rs_inv[m] = vmax > 0.f ? ldexpf(1.f, e - 15) : 1.f;
  }
  // the zero row that MFMA rows 8..31 (and rows past M) read
  for (int k = tid; k < SK_LD; k += 256) {
    Ah[SK_MR][k] = (_Float16)0.f;
    Al[SK_MR][k] = (_Float16)0.f;
  }

  const int NO = EPI == SK_SWIGLU ? a.N / 2 : a.N;
  const int per_tile = EPI == SK_SWIGLU ? 16 : 32;
  const int ntiles = (NO + per_tile - 1) / per_tile;
  const int nchunks = (K + SK_KC - 1) / SK_KC;
  const int arow = lr < M ? lr : SK_MR;  // LDS row of this lane's A operand
  constexpr int BPW = SK_KC / 32 / 4;     // blocks of a chunk per wave

  // weight row of this lane's column in tile t
  auto tile_row = [&](int t) -> int {
    int n;
    if constexpr (EPI == SK_SWIGLU)
      n = lr < 16 ? per_tile * t + lr : a.N / 2 + per_tile * t + lr - 16;
    else
      n = per_tile * t + lr;
    return min(n, a.N - 1);
  };
  // the wave's blocks cb0 + wave + 4 i of chunk [cb0, cb1) of row n, all
  // requested at once (blocks past cb1 re-read the last one; not used)
  auto load_blocks = [&](int n, int cb0, int cb1, uint2 (&raw)[BPW], unsigned (&db)[BPW]) {
    const uint8_t *wrow = a.qs + (size_t)n * B * 16 + 8 * h;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int b = min(cb0 + wave + 4 * i, cb1 - 1);
      raw[i] = *reinterpret_cast<const uint2 *>(wrow + (size_t)b * 16);
      db[i] = a.dsc[dsc_index(n, b, B)];
    }
  };
  auto mma_blocks = [&](int cb0, int cb1, const uint2 (&raw)[BPW], const unsigned (&db)[BPW],
                        float (&acc)[4]) {
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int b = cb0 + wave + 4 * i;
      if (b < cb1) {
        const half8 B0 = codes_operand<PBX_Q4>(raw[i], 0), B1 = codes_operand<PBX_Q4>(raw[i], 2);
        const int kk = (b - cb0) * 32 + 8 * h;
        const half8 Ah0 = *reinterpret_cast<const half8 *>(&Ah[arow][kk]);
        const half8 Ah1 = *reinterpret_cast<const half8 *>(&Ah[arow][kk + 16]);
        const half8 Al0 = *reinterpret_cast<const half8 *>(&Al[arow][kk]);
        const half8 Al1 = *reinterpret_cast<const half8 *>(&Al[arow][kk + 16]);
        const floatx16 zero16 = {};
        floatx16 blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ah0, B0, zero16, 0, 0, 0);
        blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(Al0, B0, blk, 0, 0, 0);
        blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ah1, B1, blk, 0, 0, 0);
        blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(Al1, B1, blk, 0, 0, 0);
        const float d = f16_bits_to_f32(db[i]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(blk[r], d, acc[r]);
      }
      // one block at a time: unpacking every block's operands up front
      // would need more registers than two waves a SIMD have
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // one float4 item (row m, columns k .. k+3 of the chunk) into LDS:
  // the RMSNorm product of pbx_rmsnorm_rows, then the exact power-of-two scale
  auto put = [&](int m, int k, float4 x, float4 g) {
    half4v hv = {}, lv = {};
    if (m < M) {
      const float r = rs_norm[m], sc = rs_scale[m];
      const float v0 = (x.x * r) * g.x * sc, v1 = (x.y * r) * g.y * sc;
      const float v2 = (x.z * r) * g.z * sc, v3 = (x.w * r) * g.w * sc;
      hv[0] = (_Float16)v0; hv[1] = (_Float16)v1; hv[2] = (_Float16)v2; hv[3] = (_Float16)v3;
      lv[0] = (_Float16)(v0 - (float)hv[0]); lv[1] = (_Float16)(v1 - (float)hv[1]);
      lv[2] = (_Float16)(v2 - (float)hv[2]); lv[3] = (_Float16)(v3 - (float)hv[3]);
    }
    *reinterpret_cast<half4v *>(&Ah[m][k]) = hv;
    *reinterpret_cast<half4v *>(&Al[m][k]) = lv;
  };
  // chunk c of the activation rows into LDS (a full chunk: the items of
  // xr, from registers for K <= SK_KC, else loaded here in one batch)
  auto convert = [&](int c) {
    const int k0 = c * SK_KC;
    __syncthreads();  // rs_* are written; earlier reads of the chunk buffer are done
    const int kc4 = min(SK_KC, K - k0) / 4;
    if (!one) {
      // a last chunk may be shorter than SK_KC: columns past it are not read
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int k4 = tid + 256 * q;
        gr[q] = norm && k4 < kc4 ? reinterpret_cast<const float4 *>(a.normw + k0)[k4]
                                 : make_float4(1.f, 1.f, 1.f, 1.f);
      }
#pragma unroll
      for (int j = 0; j < IT; ++j) {
        const int m = j >> 1, k4 = tid + 256 * (j & 1);
        xr[j] = m < M && k4 < kc4 ? reinterpret_cast<const float4 *>(a.X + (size_t)m * K + k0)[k4]
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int j = 0; j < IT; ++j) {
      const int m = j >> 1, k4 = tid + 256 * (j & 1);
      if (k4 < kc4) put(m, 4 * k4, xr[j], gr[j & 1]);
    }
    __syncthreads();
  };
  // the four waves' partial sums of tile t; wave 0 applies the epilogue
  auto finish = [&](int t, float (&acc)[4]) {
    if (wave > 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) tred[wave - 1][lane][r] = acc[r];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] += (tred[0][lane][r] + tred[1][lane][r]) + tred[2][lane][r];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * h + r;
        const float v = acc[r] * rs_inv[m];
        const int col = per_tile * t + lr;
        if constexpr (EPI == SK_SWIGLU) {
          const float u = __shfl(v, (lane & 32) | ((lr + 16) & 31), 64);  // the up row of this gate column
          if (lr < 16 && m < M && col < NO) a.Y[(size_t)m * a.ldy + col] = silu(v) * u;
        } else {
          if (m < M && col < NO) {
            float *y = a.Y + (size_t)m * a.ldy + col;
            if constexpr (EPI == SK_ADD)
              *y += v;
            else
              *y = v;
          }
        }
      }
    }
    __syncthreads();  // tred is reused by the next tile
  };

  uint2 rawA[BPW];
  unsigned dA[BPW];
  if (nchunks == 1) {
    // whole rows in LDS once, then tiles t, t + G, ...: all of a tile's
    // blocks requested at once (two workgroups a CU overlap the tiles)
    const int G = gridDim.x, cb1 = B;
    int t = blockIdx.x;
    if (t >= ntiles) return;
    convert(0);
    for (; t < ntiles; t += G) {
      load_blocks(tile_row(t), 0, cb1, rawA, dA);
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      mma_blocks(0, cb1, rawA, dA, acc);
      finish(t, acc);
    }
  } else {
    // one tile a workgroup (grid = tiles), chunk by chunk
    const int t = blockIdx.x;
    if (t >= ntiles) return;
    const int n = tile_row(t);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < nchunks; ++c) {
      const int cb0 = c * (SK_KC / 32), cb1 = min(B, cb0 + SK_KC / 32);
      load_blocks(n, cb0, cb1, rawA, dA);
      convert(c);
      mma_blocks(cb0, cb1, rawA, dA, acc);
    }
    finish(t, acc);
  }
}

extern "C" __global__ void __launch_bounds__(256, 2) pbx_sk_q4_store(SkinnyArgs a) { skinny_q4<SK_STORE>(a); }
extern "C" __global__ void __launch_bounds__(256, 2) pbx_sk_q4_swiglu(SkinnyArgs a) { skinny_q4<SK_SWIGLU>(a); }
