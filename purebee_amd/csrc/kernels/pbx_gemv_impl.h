// pbx_gemv_impl.h -- device implementation of the M=1 GEMV family, shared by
// the plain instruction kernels (pbx_gemv.hip) and the fused decode-step
// kernels (pbx_decode.hip).
//
// A GEMV computes y[n] = sum_k x[k] * W[n,k] for one activation row.  Two
// templates cover every shape:
//   gemv_wide  : B = K/32 >= 33.  W = ceil(B/64) waves per workgroup; lane l
//                of wave w owns block b = 64w + l of every row and keeps that
//                block's 32 activations in registers; R rows per workgroup.
//   gemv_small : B <= 32.  Lane l owns (row slot l/B, block l%B); 64/B rows
//                per pass, P passes per wave, partials summed through LDS.
// Both take a prologue that builds the activation block the lane needs
// (plain load, RMSNorm of x, or SwiGLU of gate/up) and an epilogue that
// consumes each row's sum (store with optional bias, accumulate into y for
// residual connections, or store plus per-tile argmax partials).
#ifndef PBX_GEMV_IMPL_H
#define PBX_GEMV_IMPL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#define PBX_Q4 0
#define PBX_Q8 1
#define PBX_F32 2
#define PBX_Q41 3
#define PBX_F16 4
#define PBX_Q6K 5
#define PBX_Q6KP 6  // Q6_K codes repacked lane-major (integer-limb kernel only)

#define PRO_NONE 0
#define PRO_RMSNORM 1
#define PRO_SWIGLU 2
// RMSNorm of x + acc * 2^-32 (integer-limb kernel, one activation row): the
// residual row plus the pending update the fused attention + o projection
// accumulated as 2^-32 fixed-point integers
#define PRO_RMSACC 3

#define EPI_STORE 0
#define EPI_ADD 1
#define EPI_ARGMAX 2
// Paired rows: the weight holds N/2 gate rows then N/2 up rows; a workgroup
// reads matching gate and up rows and stores silu(gate)*up (N/2 outputs).
#define EPI_SWIGLU 3
// The q|k|v rows of a decode step (integer-limb kernel, one activation row):
// RoPE of the q and k rows at the position state[0] (adjacent row pairs,
// llama.js:163-190), q stored to Y, k and v stored to the cache row of that
// position (the attention then reads every position from the cache).
#define EPI_ROPE 4
// y = (y + acc * 2^-32) + W x, then acc = 0: the residual add that also folds
// the pending update into the residual row (integer-limb kernel)
#define EPI_ADDACC 5

// Everything a fused GEMV launch needs; passed by value.
struct GemvArgs {
  const uint8_t *qs;    // weight plane (nibbles / int8 / f32)
  const uint16_t *dsc;  // fp16 scale plane (quantised types)
  const float *X;       // activation row(s) [M][K]; gate for PRO_SWIGLU
  const float *X2;      // up for PRO_SWIGLU
  const float *normw;   // RMSNorm weight [K] for PRO_RMSNORM
  const float *bias;    // [N] or null (EPI_STORE)
  float *Y;             // [M][N]
  uint64_t *partials;   // EPI_ARGMAX: one key per tile
  int N, B;
  float eps;
  const uint16_t *msc;  // fp16 min plane (Q4_1), same layout as dsc
  int rows;             // gemv_int with MR > 1: valid activation rows
  // EPI_ROPE: position, RoPE table [max_seq][head_dim/2][cos, sin], this
  // layer's caches [max_seq][kvdim], q rows [0, qdim), k rows [qdim,
  // qdim + kvdim), v rows after them
  const int *state;
  const float *rope;
  float *kcache, *vcache;
  int qdim, kvdim, head_dim;
  int pos0;             // EPI_ROPE with several activation rows: row m at pos0 + m
  long long *acc;       // PRO_RMSACC / EPI_ADDACC: pending update [N] (2^-32 units)
  // gemv_mr with the K split over workgroups: one cell per output element
  // [MR][N] (zero between launches).  gemv_int EPI_ROPE: N published rows
  // and the layer's epoch at [N] (the fused q|k|v + attention kernel);
  // EPI_ADDACC: that epoch, advanced once per launch.  EPI_SWIGLU: N / 2
  // published outputs and their epoch at [N / 2] (the joined FFN launch)
  unsigned long long *xcell;
  // builder waves (BW > 0): clr_n 64-bit words of clr zeroed by the grid's
  // builder threads after their build; adv: an epoch that thread 0 of
  // workgroup 0 advances (both only for buffers no one else touches in the
  // launch)
  long long *clr;
  int clr_n;
  unsigned long long *adv;
};

namespace pbx {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef long long i64x2_t __attribute__((ext_vector_type(2)));

// 16-byte streaming load of weight bytes that are read once per matvec
// (nontemporal: they should not displace the activations in the caches).
__device__ __forceinline__ uint4 ld_stream(const void *p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// A pointer the compiler cannot place (one read from memory, not a kernel
// argument) as a global-memory pointer: loads through it are global loads.
// Through the generic pointer they are flat loads, which also count against
// the LDS wait counter, so every LDS wait after them waits for their data.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T *gmem(const T *p) {
  return (const __attribute__((address_space(1))) T *)p;
}

__device__ __forceinline__ uint4 ld_stream_g(const void *p) {
  const u32x4_t v = __builtin_nontemporal_load(gmem(reinterpret_cast<const u32x4_t *>(p)));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Scale plane: 4-row groups, [Npad/4][B][4] fp16, so the scales of 4
// consecutive rows at one block are one 8-byte load and a tile of >= 4 rows
// uses whole cache lines.
__device__ __forceinline__ size_t dsc_index(int n, int b, int B) {
  return ((size_t)(n >> 2) * B + b) * 4 + (n & 3);
}

__device__ __forceinline__ float f16_bits_to_f32(unsigned bits) {
  // IEEE binary16 -> binary32 (v_cvt_f32_f16): the conversion of
  // gguf.js:55-70 including subnormals, +-inf and NaN.
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits & 0xFFFFu));
}

// sum_j x[j] * nibble_j over one Q4_0 block (nibbles unsigned, 0..15); the
// caller subtracts 8*sum(x) to obtain sum_j x[j] * (nibble_j - 8).  Byte j
// holds element j (low nibble) and element j+16 (high nibble).
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

// sum_j x[j] * w[j] over 32 fp16 weights (exact conversions).
__device__ __forceinline__ float dot_f16(const uint4 (&q)[4], const float (&xr)[32]) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const unsigned w[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float &s = (k & 1) ? s1 : s0;
      s = fmaf(xr[8 * j + 2 * k], f16_bits_to_f32(w[k]), s);
      s = fmaf(xr[8 * j + 2 * k + 1], f16_bits_to_f32(w[k] >> 16), s);
    }
  }
  return s0 + s1;
}

// One lane's Q6_K term: d * (sc0 * sum_{l<16} x_l (q_l - 32) +
// sc1 * sum_{l>=16} x_l (q_l - 32)); the unsigned 6-bit codes are assembled
// four at a time, the offset folded into 32 * (sum of x) per half-block.
__device__ __forceinline__ float dot_q6k(const uint4 (&q)[4], unsigned ex, int g,
                                         const float (&xr)[32], float xs, float xlo, float d) {
  const unsigned ql[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
  const unsigned qh[8] = {q[2].x, q[2].y, q[2].z, q[2].w, q[3].x, q[3].y, q[3].z, q[3].w};
  const int sl = (g >> 1) * 4, sh = g * 2;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const unsigned v = ((ql[k] >> sl) & 0x0F0F0F0Fu) | (((qh[k] >> sh) & 0x03030303u) << 4);
    float &s = k < 4 ? s0 : s1;
    s = fmaf(xr[4 * k + 0], (float)(v & 0xFFu), s);
    s = fmaf(xr[4 * k + 1], (float)((v >> 8) & 0xFFu), s);
    s = fmaf(xr[4 * k + 2], (float)((v >> 16) & 0xFFu), s);
    s = fmaf(xr[4 * k + 3], (float)(v >> 24), s);
  }
  const float sc0 = (float)(int8_t)(ex & 0xFFu), sc1 = (float)(int8_t)((ex >> 8) & 0xFFu);
  return d * (sc0 * (s0 - 32.f * xlo) + sc1 * (s1 - 32.f * (xs - xlo)));
}

__device__ __forceinline__ float dot_f32(const uint4 (&q)[8], const float (&xr)[32]) {
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
template <> struct BlockTraits<PBX_Q41> { static constexpr int QB = 16; static constexpr float OFF = 0.f; };
// F16: 32 halves.  Q6_K: the lane's 32 ql bytes then its 32 qh bytes (see
// load_lane); the 6-bit codes carry an offset of 32.
template <> struct BlockTraits<PBX_F16> { static constexpr int QB = 64; static constexpr float OFF = 0.f; };
template <> struct BlockTraits<PBX_Q6K> { static constexpr int QB = 64; static constexpr float OFF = 32.f; };
// Q6_K lane-packed: the 16 low-nibble bytes then the 8 high-field bytes of
// the lane's 32 codes (see load_lane), in two 16-byte registers.
template <> struct BlockTraits<PBX_Q6KP> { static constexpr int QB = 32; static constexpr float OFF = 32.f; };
template <int TYPE> constexpr bool is_q6k() { return TYPE == PBX_Q6K || TYPE == PBX_Q6KP; }

// Types with an fp16 scale plane (d per 32-block, or per 256-block for Q6_K).
template <int TYPE> constexpr bool has_scale() {
  return TYPE == PBX_Q4 || TYPE == PBX_Q8 || TYPE == PBX_Q41 || is_q6k<TYPE>();
}
// Q6_K keeps one d per 256-element super-block: block index and blocks per
// row of the scale plane for the lane's 32-block b.
template <int TYPE> __device__ __forceinline__ int scale_block(int b) {
  return is_q6k<TYPE>() ? b >> 3 : b;
}

// Q6_K super-block as resident (gguf.js:317-364 minus d, which moves to the
// scale plane): ql[128] low nibbles, qh[64] high 2-bit pairs, 16 int8
// sub-block scales; 208 bytes, 16-byte aligned.
#define PBX_Q6K_BYTES 208

// Q6_K lane-packed copy (PBX_Q6KP), 26 bytes per 32-block, row by row:
// [B][16] bytes whose byte j holds code j's low nibble (bits 0-3) and code
// j+16's (bits 4-7); [B][8] bytes whose byte 4u+t holds the 2-bit high
// fields of codes 16u+4s+t at bits 2s, s < 4; [B][2] the int8 scales of the
// two 16-code halves.  Codes are those of the Q6_K layout above, so the
// integer dots of both layouts are the same sums.  A lane's block is one
// 16-byte, one 8-byte and one 2-byte load (the Q6_K layout needs 64 bytes).
#define PBX_Q6KP_ROW 26

// The weight bytes lane-block b (elements 32b .. 32b+31) of row n needs.
// Q6_K: element e = 256*sb + 128*half + 32*g + l (l < 32) is
//   ((ql[64*half + 32*(g&1) + l] >> 4*(g>>1)) & 15)
//   | ((qh[32*half + l] >> 2*g) & 3) << 4,  minus 32,
// times d * scales[8*half + 2*g + l/16] (gguf.js:317-364); with b = 8*sb +
// 4*half + g the lane reads 32 contiguous ql bytes, 32 contiguous qh bytes
// and the two int8 scales of its half-blocks (returned in ex).
//
// The loads are unconditional: a lane that is not `ok` reads block 0 of row
// n (always in the plane), and its value is cancelled later (zero scales,
// zero activations; F32 / F16 bytes are masked here).  A load under a
// branch would make the compiler wait for it at the branch's join, which
// serialises the row loads of a tile into separate memory round trips.
template <int TYPE>
__device__ __forceinline__ void load_lane(const uint8_t *qs, int n, int b, int B, bool ok,
                                          uint4 (&q)[BlockTraits<TYPE>::QB / 16],
                                          unsigned &ex) {
  constexpr int QB = BlockTraits<TYPE>::QB;
  const int bb = ok ? b : 0;
  ex = 0u;
  if constexpr (TYPE == PBX_Q6K) {
    const uint8_t *blk = qs + ((size_t)n * (B >> 3) + (bb >> 3)) * PBX_Q6K_BYTES;
    const int half = (bb >> 2) & 1, g = bb & 3;
    const uint8_t *ql = blk + half * 64 + (g & 1) * 32;
    const uint8_t *qh = blk + 128 + half * 32;
    q[0] = ld_stream(ql);
    q[1] = ld_stream(ql + 16);
    q[2] = ld_stream(qh);
    q[3] = ld_stream(qh + 16);
    ex = *reinterpret_cast<const uint16_t *>(blk + 192 + half * 8 + 2 * g) & (ok ? 0xFFFFu : 0u);
  } else if constexpr (TYPE == PBX_Q6KP) {
    // row n: [B][16] low nibbles, [B][8] high fields, [B][2] int8 scales
    const uint8_t *row = qs + (size_t)n * (B * PBX_Q6KP_ROW);
    q[0] = ld_stream(row + (size_t)bb * 16);
    const uint2 h = *reinterpret_cast<const uint2 *>(row + (size_t)B * 16 + (size_t)bb * 8);
    q[1] = make_uint4(h.x, h.y, 0u, 0u);
    ex = *reinterpret_cast<const uint16_t *>(row + (size_t)B * 24 + (size_t)bb * 2) &
         (ok ? 0xFFFFu : 0u);
  } else {
    const uint8_t *src = qs + ((size_t)n * B + bb) * QB;
#pragma unroll
    for (int v = 0; v < QB / 16; ++v) q[v] = ld_stream(src + v * 16);
    if constexpr (TYPE == PBX_F32 || TYPE == PBX_F16) {
      const unsigned m = ok ? ~0u : 0u;
#pragma unroll
      for (int v = 0; v < QB / 16; ++v) {
        q[v].x &= m; q[v].y &= m; q[v].z &= m; q[v].w &= m;
      }
    }
  }
}


// Element i of row `tok` of a resident [rows][dim] weight, dequantised
// exactly as gguf.js:231-364 (F16, Q8_0, Q4_0, Q4_1, Q6_K) or read (F32).
__device__ __forceinline__ float row_value(const uint8_t *qs, const uint16_t *dsc,
                                          const uint16_t *msc, int type, int tok, int i,
                                          int dim) {
  if (type == PBX_F32) return reinterpret_cast<const float *>(qs)[(size_t)tok * dim + i];
  if (type == PBX_F16)
    return f16_bits_to_f32(reinterpret_cast<const uint16_t *>(qs)[(size_t)tok * dim + i]);
  if (type == PBX_Q6K) {
    // gguf.js:317-364; (d * sc) * (q - 32) is exact in fp32 (11 + 7 + 5
    // significant bits), so this equals the reference's double product
    // rounded once.
    const int SB = dim / 256, sb = i / 256, r = i % 256;
    const int half = r >> 7, g = (r >> 5) & 3, l = r & 31;
    const uint8_t *blk = qs + ((size_t)tok * SB + sb) * PBX_Q6K_BYTES;
    const int lo = (blk[half * 64 + (g & 1) * 32 + l] >> (4 * (g >> 1))) & 15;
    const int hi = (blk[128 + half * 32 + l] >> (2 * g)) & 3;
    const float sc = (float)(int8_t)blk[192 + half * 8 + 2 * g + (l >> 4)];
    const float d = f16_bits_to_f32(dsc[dsc_index(tok, sb, SB)]);
    return (d * sc) * (float)((lo | (hi << 4)) - 32);
  }
  const int B = dim / 32, b = i / 32, j = i % 32;
  const size_t di = dsc_index(tok, b, B);
  const float d = f16_bits_to_f32(dsc[di]);
  if (type == PBX_Q8) return (float)(int8_t)qs[((size_t)tok * B + b) * 32 + j] * d;
  const unsigned byte = qs[((size_t)tok * B + b) * 16 + (j & 15)];
  const int nib = j < 16 ? (int)(byte & 15u) : (int)(byte >> 4);
  if (type == PBX_Q41) return fmaf((float)nib, d, f16_bits_to_f32(msc[di]));
  return (float)(nib - 8) * d;
}

// Block b (32 floats) of base, read unconditionally (block 0 when !valid;
// the caller zeroes such lanes' values), so the loads issue back to back.
__device__ __forceinline__ void load_block_nb(const float *__restrict__ base, int b, bool valid,
                                              float (&v)[32]) {
  const float4 *xp = reinterpret_cast<const float4 *>(base + (size_t)(valid ? b : 0) * 32);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 t = xp[i];
    v[4 * i + 0] = t.x; v[4 * i + 1] = t.y;
    v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
  }
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// Workgroup barrier for LDS hand-offs: waits for this wave's LDS operations
// only.  __syncthreads also drains the wave's outstanding global loads
// (its workgroup-scope fence), which would stall a kernel that has weight
// bytes in flight across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Distances 16 and 32 by gfx950's lane swaps (VALU, no LDS round trip):
// v_permlane32_swap of (v, v) leaves the lower half of v in both halves of
// the first result and the upper half in both halves of the second;
// v_permlane16_swap does the same for the even and odd 16-lane rows.  So
// the first result holds v on lanes with bit OFF clear and the partner's
// value on the others, the second the reverse.
template <int OFF>
__device__ __forceinline__ void lane_swap(float v, float &lo, float &hi) {
  static_assert(OFF == 16 || OFF == 32, "row or half swap");
  const unsigned b = __float_as_uint(v);
  if constexpr (OFF == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
  }
}

// The value the butterfly partner at distance OFF holds.  Distances inside
// a 16-lane row use DPP (a VALU operand modifier: no LDS round trip), with a
// partner that differs in bit OFF and agrees in the bits above it:
//   8 -> row_ror:8 (lane ^ 8), 4 -> row_half_mirror (lane ^ 7),
//   2 -> quad_perm 3,2,1,0 (lane ^ 3), 1 -> quad_perm 1,0,3,2 (lane ^ 1).
// 16 and 32 use the lane swaps above (lane ^ 16, lane ^ 32).  The masks 32,
// 16, 8, 7, 3, 1 are independent, so a butterfly over them sums all 64
// lanes, and each stage's partner agrees on the bits earlier stages split
// on, which the transposed reductions rely on.  All 64 lanes must be active.
template <int OFF>
__device__ __forceinline__ float lane_partner(float v) {
  if constexpr (OFF >= 16) {
    float lo, hi;
    lane_swap<OFF>(v, lo, hi);
    return (__lane_id() & OFF) ? lo : hi;
  } else {
    constexpr int ctrl = OFF == 8 ? 0x128 : OFF == 4 ? 0x141 : OFF == 2 ? 0x1B : 0xB1;
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false));
  }
}

// v + partner and max(v, partner) at distance OFF.  For 16 and 32 the two
// swap results are v and the partner in some order on every lane: the sum
// and the maximum are the same either way.
template <int OFF>
__device__ __forceinline__ float pair_sum(float v) {
  if constexpr (OFF >= 16) {
    float lo, hi;
    lane_swap<OFF>(v, lo, hi);
    return lo + hi;
  } else {
    return v + lane_partner<OFF>(v);
  }
}

template <int OFF>
__device__ __forceinline__ float pair_max(float v) {
  if constexpr (OFF >= 16) {
    float lo, hi;
    lane_swap<OFF>(v, lo, hi);
    return fmaxf(lo, hi);
  } else {
    return fmaxf(v, lane_partner<OFF>(v));
  }
}

template <int OFF = 32>
__device__ __forceinline__ float wave_sum(float v) {
  if constexpr (OFF >= 1) {
    return wave_sum<OFF / 2>(pair_sum<OFF>(v));
  } else {
    return v;
  }
}

template <int OFF = 32>
__device__ __forceinline__ float wave_max(float v) {
  if constexpr (OFF >= 1) {
    return wave_max<OFF / 2>(pair_max<OFF>(v));
  } else {
    return v;
  }
}

// The partner's 64-bit value: both halves moved as bits (the lane moves
// apply no arithmetic).
template <int OFF>
__device__ __forceinline__ uint64_t lane_partner_u64(uint64_t v) {
  const unsigned lo = __float_as_uint(lane_partner<OFF>(__uint_as_float((unsigned)v)));
  const unsigned hi = __float_as_uint(lane_partner<OFF>(__uint_as_float((unsigned)(v >> 32))));
  return (uint64_t)hi << 32 | lo;
}

template <int OFF = 32>
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  if constexpr (OFF >= 1) {
    const uint64_t o = lane_partner_u64<OFF>(v);
    return wave_max_u64<OFF / 2>(o > v ? o : v);
  } else {
    return v;
  }
}

// Order-preserving key for argmax: larger value -> larger key; equal values
// -> the smaller index wins (the first maximum, as llama.js:432-442 keeps
// the first index on ties with its strict `>`).  NaN never wins.
__device__ __forceinline__ uint64_t argmax_key(float v, unsigned idx) {
  if (v != v) return 0;
  unsigned b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

// One block-row term of the lane's 32-block b.  xs = sum of the lane's 32
// activations, xlo = sum of the first 16.  OFF * xs removes the code offset
// (Q4_0, Q8_0); Q4_1 (gguf.js:288-314: value = nibble * d + m) adds m * xs,
// the split of llama-streaming.js:138-145.
template <int TYPE>
__device__ __forceinline__ float block_term(const uint4 (&q)[BlockTraits<TYPE>::QB / 16],
                                            unsigned ex, int b, const float (&xr)[32],
                                            float xs, float xlo, float d, float mn) {
  if constexpr (TYPE == PBX_Q4) {
    return (dot_q4(q[0], xr) - 8.f * xs) * d;
  } else if constexpr (TYPE == PBX_Q41) {
    return fmaf(dot_q4(q[0], xr), d, mn * xs);
  } else if constexpr (TYPE == PBX_Q8) {
    return (dot_q8(q[0], q[1], xr) - 128.f * xs) * d;
  } else if constexpr (TYPE == PBX_F16) {
    return dot_f16(q, xr);
  } else if constexpr (TYPE == PBX_Q6K) {
    return dot_q6k(q, ex, b & 3, xr, xs, xlo, d);
  } else {
    return dot_f32(q, xr);
  }
}

// fp16 scales (or Q4_1 minima) of tile rows 0..R) at block b.  SEG is the
// number of rows of the tile that are consecutive in the plane (R, or R/2
// for paired gate/up tiles); 4-row groups are one 8-byte load.
// Loaded unconditionally (block 0 when !valid) and masked to +0.
template <int R, int SEG, typename RowFn>
__device__ __forceinline__ void load_scale_bits(const uint16_t *plane, RowFn tile_row, int b,
                                                int B, bool valid, unsigned (&out)[R]) {
  const int bb = valid ? b : 0;
  const unsigned m = valid ? ~0u : 0u;
  if constexpr (SEG >= 4) {
#pragma unroll
    for (int g = 0; g < R / 4; ++g) {
      const uint2 dv = *reinterpret_cast<const uint2 *>(plane + dsc_index(tile_row(g * 4), bb, B));
      out[g * 4 + 0] = dv.x & m;
      out[g * 4 + 1] = (dv.x >> 16) & m;
      out[g * 4 + 2] = dv.y & m;
      out[g * 4 + 3] = (dv.y >> 16) & m;
    }
  } else {
    // segments of 1 or 2 rows inside one 4-row group
#pragma unroll
    for (int i = 0; i < R; ++i) out[i] = plane[dsc_index(tile_row(i), bb, B)] & m;
  }
}

// Transposed wavefront reduction: v[0..R) are 64-lane partial sums of R rows.
// Each halving stage exchanges half of the remaining values with the lane
// OFF away, so the stages move R/2, R/4, ... values instead of reducing each
// row separately; lane l ends with row l / (64/R) summed over its group and
// the remaining butterfly stages complete the 64-lane sum.
template <int CNT, int OFF, int R>
__device__ __forceinline__ void transpose_stage(float (&v)[R], int lane) {
  if constexpr (CNT > 1) {
    const bool up = (lane & OFF) != 0;
#pragma unroll
    for (int i = 0; i < CNT / 2; ++i) {
      const float keep = up ? v[i + CNT / 2] : v[i];
      const float send = up ? v[i] : v[i + CNT / 2];
      v[i] = keep + lane_partner<OFF>(send);
    }
    transpose_stage<CNT / 2, OFF / 2, R>(v, lane);
  }
}

template <int R>
__device__ __forceinline__ float wave_transpose_reduce(float (&v)[R], int lane) {
  transpose_stage<R, 32, R>(v, lane);
  return wave_sum<(64 / R) / 2>(v[0]);
}

// The tag that a launch of epoch e publishes its cells with: never 0 (the
// tag of cleared cells), and next_epoch skips the epoch whose tag would wrap
// to 0, so consecutive launches always publish different tags.
__device__ __forceinline__ unsigned cell_tag(unsigned long long e) { return (unsigned)e + 1u; }
__device__ __forceinline__ unsigned long long next_epoch(unsigned long long e) {
  const unsigned long long n = e + 1;
  return cell_tag(n) == 0u ? n + 1 : n;
}

// x + q * 2^-32 rounded once: the residual row with its pending
// fixed-point update (PRO_RMSACC and EPI_ADDACC form the same value).
__device__ __forceinline__ float residual_acc(float x, long long q) {
  return (float)fma((double)q, 0x1p-32, (double)x);
}

// Store of output row n; `res` is the residual y[n] read at kernel start
// (EPI_ADD), so the epilogue does not wait on a second round trip;
// EPI_ADDACC: `racc` its pending update, cleared here.
template <int EPI>
__device__ __forceinline__ void epilogue_row(const GemvArgs &a, float *y, int n, float s, float res,
                                             long long racc = 0) {
  if constexpr (EPI == EPI_ADD) {
    y[n] = res + s;
  } else if constexpr (EPI == EPI_ADDACC) {
    y[n] = residual_acc(res, racc) + s;
    a.acc[n] = 0;
  } else {
    y[n] = s + (a.bias ? a.bias[n] : 0.f);
  }
}

// ---------------------------------------------------------------------------
template <int TYPE, int R, int PRO, int EPI>
__device__ __forceinline__ void gemv_wide(const GemvArgs &a) {
  constexpr int QB = BlockTraits<TYPE>::QB;
  constexpr int NV = QB / 16;
  constexpr int MAXW = 8;
  __shared__ float red[MAXW][R];
  __shared__ float ssw[MAXW];

  const int N = a.N, B = a.B;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int b = wave * 64 + lane;
  const bool valid = b < B;
  const int K = B * 32;
  const float *x = a.X + (size_t)blockIdx.y * K;
  const float *x2 = a.X2 ? a.X2 + (size_t)blockIdx.y * K : nullptr;
  constexpr bool PAIR = EPI == EPI_SWIGLU;
  const int NO = PAIR ? N / 2 : N;  // output rows
  float *y = a.Y + (size_t)blockIdx.y * NO;
  // Row i of the tile: R consecutive rows, or (PAIR) R/2 gate rows starting
  // at r0 and the matching R/2 up rows starting at N/2 + r0.
  const int r0 = blockIdx.x * (PAIR ? R / 2 : R);
  auto tile_row = [&](int i) -> int {
    return PAIR ? (i < R / 2 ? r0 + i : N / 2 + r0 + i - R / 2) : r0 + i;
  };

  // Rows past N (the last tile of a paired matrix) are read as row N - 1;
  // their sums are never stored.
  auto load_row = [&](int i) -> int { return min(tile_row(i), N - 1); };

  // 1. Activation inputs first (x; x2 for SwiGLU; the RMSNorm weights): a CU
  //    returns loads in issue order, so inputs requested behind the weight
  //    stream would arrive only with it.  Then the residual (EPI_ADD).
  const int lanes_per_row = 64 / R;
  float xa[32], xb[32];
  load_block_nb(x, b, valid, xa);
  if constexpr (PRO == PRO_SWIGLU) load_block_nb(x2, b, valid, xb);
  if constexpr (PRO == PRO_RMSNORM) load_block_nb(a.normw, b, valid, xb);
  float res = 0.f;
  if constexpr (EPI == EPI_ADD) {
    const int rr = nwaves == 1 ? ((lane % lanes_per_row) == 0 ? lane / lanes_per_row : R)
                               : (int)threadIdx.x;
    if (rr < R && r0 + rr < N) res = y[r0 + rr];
  }
  // 2. Scale bits, then the weight bytes, all issued before any use.
  unsigned dbits[R], mbits[R];
  if constexpr (has_scale<TYPE>()) {
    constexpr int SEG = PAIR ? R / 2 : R;  // rows contiguous in the scale plane
    const int sb = scale_block<TYPE>(b), SB = scale_block<TYPE>(B);
    load_scale_bits<R, SEG>(a.dsc, load_row, sb, SB, valid, dbits);
    if constexpr (TYPE == PBX_Q41) load_scale_bits<R, SEG>(a.msc, load_row, sb, SB, valid, mbits);
  }
  __builtin_amdgcn_sched_barrier(0);
  uint4 q[R][NV];
  unsigned ex[R];
#pragma unroll
  for (int i = 0; i < R; ++i) load_lane<TYPE>(a.qs, load_row(i), b, B, valid, q[i], ex[i]);
  __builtin_amdgcn_sched_barrier(0);

  // 3. The activation block after the prologue (zero for lanes past B).
  float xr[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    float v = xa[j];
    if constexpr (PRO == PRO_SWIGLU) v = silu(v) * xb[j];
    xr[j] = valid ? v : 0.f;
  }
  if constexpr (PRO == PRO_RMSNORM) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) ss = fmaf(xr[j], xr[j], ss);
    ss = wave_sum(ss);
    if (nwaves > 1) {
      if (lane == 0) ssw[wave] = ss;
      lds_barrier();
      ss = 0.f;
      for (int w = 0; w < nwaves; ++w) ss += ssw[w];
    }
    // RMSNorm (engine.js:429-449): x * (1/rms) * w
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
    for (int j = 0; j < 32; ++j) xr[j] = xr[j] * inv * xb[j];
  }
  float dsf[R], msf[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    dsf[i] = has_scale<TYPE>() ? f16_bits_to_f32(dbits[i]) : 1.f;
    msf[i] = TYPE == PBX_Q41 ? f16_bits_to_f32(mbits[i]) : 0.f;
  }
  float xs = 0.f, xlo = 0.f;
  if constexpr (TYPE != PBX_F32 && TYPE != PBX_F16) {
#pragma unroll
    for (int i = 0; i < 16; ++i) xlo += xr[i];
    xs = xlo;
#pragma unroll
    for (int i = 16; i < 32; ++i) xs += xr[i];
  }

  float acc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = block_term<TYPE>(q[i], ex[i], b, xr, xs, xlo, dsf[i], msf[i]);

  const float tot = wave_transpose_reduce<R>(acc, lane);
  const int row = lane / lanes_per_row;
  uint64_t key = 0;
  if constexpr (PAIR) {
    // gate row i sits in lane i*lpr, its up row in lane i*lpr + 32
    if (nwaves == 1) {
      const float up = lane_partner<32>(tot);
      if (lane < 32 && (lane % lanes_per_row) == 0) {
        const int n = r0 + row;
        if (n < NO) y[n] = silu(tot) * up;
      }
    } else {
      if ((lane % lanes_per_row) == 0) red[wave][row] = tot;
      __syncthreads();
      if (threadIdx.x < R / 2) {
        float g = 0.f, u = 0.f;
        for (int w = 0; w < nwaves; ++w) {
          g += red[w][threadIdx.x];
          u += red[w][threadIdx.x + R / 2];
        }
        const int n = r0 + threadIdx.x;
        if (n < NO) y[n] = silu(g) * u;
      }
    }
    return;
  }
  if (nwaves == 1) {
    if ((lane % lanes_per_row) == 0) {
      const int n = r0 + row;
      if (n < N) {
        epilogue_row<EPI>(a, y, n, tot, res);
        if constexpr (EPI == EPI_ARGMAX) key = argmax_key(tot, (unsigned)n);
      }
    }
  } else {
    if ((lane % lanes_per_row) == 0) red[wave][row] = tot;
    __syncthreads();
    if (threadIdx.x < R) {
      float s = 0.f;
      for (int w = 0; w < nwaves; ++w) s += red[w][threadIdx.x];
      const int n = r0 + threadIdx.x;
      if (n < N) {
        epilogue_row<EPI>(a, y, n, s, res);
        if constexpr (EPI == EPI_ARGMAX) key = argmax_key(s, (unsigned)n);
      }
    }
  }
  if constexpr (EPI == EPI_ARGMAX) {
    if (wave == 0) {
      key = wave_max_u64(key);
      if (lane == 0) a.partials[blockIdx.x] = key;
    }
  }
}

// ---------------------------------------------------------------------------
template <int TYPE, int P, int PRO, int EPI>
__device__ __forceinline__ void gemv_small(const GemvArgs &a) {
  constexpr int QB = BlockTraits<TYPE>::QB;
  constexpr int NV = QB / 16;
  __shared__ float part[4][P][64];

  const int N = a.N, B = a.B;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rpw = 64 / B;
  const bool active = lane < rpw * B;
  const int rs = active ? lane / B : 0;
  const int b = active ? lane % B : 0;
  const int K = B * 32;
  const float *x = a.X + (size_t)blockIdx.y * K;
  const float *x2 = a.X2 ? a.X2 + (size_t)blockIdx.y * K : nullptr;
  float *y = a.Y + (size_t)blockIdx.y * N;

  constexpr bool PAIR = EPI == EPI_SWIGLU;
  const int NO = PAIR ? N / 2 : N;
  float *yo = a.Y + (size_t)blockIdx.y * NO;
  const int T = P * rpw;  // tile rows (PAIR: T/2 gate + T/2 up, T is even)
  const int r0 = (blockIdx.x * 4 + wave) * (PAIR ? T / 2 : T);
  auto tile_row = [&](int t) -> int {
    return PAIR ? (t < T / 2 ? r0 + t : N / 2 + r0 + t - T / 2) : r0 + t;
  };
  auto row_ok = [&](int t) -> bool {
    return PAIR ? (r0 + (t < T / 2 ? t : t - T / 2)) < NO : (r0 + t) < N;
  };

  // Activation inputs first, then the residual, the scales and the weight
  // bytes (the order and branch-free loads of gemv_wide).
  float xa[32], xb[32];
  load_block_nb(x, b, active, xa);
  if constexpr (PRO == PRO_SWIGLU) load_block_nb(x2, b, active, xb);
  if constexpr (PRO == PRO_RMSNORM) load_block_nb(a.normw, b, active, xb);
  // residual of the first row this lane stores (EPI_ADD)
  float res = 0.f;
  if constexpr (EPI == EPI_ADD)
    if (lane < T && r0 + lane < N) res = y[r0 + lane];

  uint4 q[P][NV];
  unsigned ex[P], dbits[P], mbits[P];
  const int sb = scale_block<TYPE>(b), SB = scale_block<TYPE>(B);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const bool ok = active && row_ok(p * rpw + rs);
    const int rw = ok ? tile_row(p * rpw + rs) : 0;
    const unsigned m = ok ? 0xFFFFu : 0u;
    dbits[p] = has_scale<TYPE>() ? a.dsc[dsc_index(rw, sb, SB)] & m : 0u;
    mbits[p] = TYPE == PBX_Q41 ? a.msc[dsc_index(rw, sb, SB)] & m : 0u;
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const bool ok = active && row_ok(p * rpw + rs);
    load_lane<TYPE>(a.qs, ok ? tile_row(p * rpw + rs) : 0, b, B, ok, q[p], ex[p]);
  }
  __builtin_amdgcn_sched_barrier(0);
  float d[P], mn[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    d[p] = has_scale<TYPE>() ? f16_bits_to_f32(dbits[p]) : 1.f;
    mn[p] = TYPE == PBX_Q41 ? f16_bits_to_f32(mbits[p]) : 0.f;
  }

  float xr[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    float v = xa[j];
    if constexpr (PRO == PRO_SWIGLU) v = silu(v) * xb[j];
    xr[j] = active ? v : 0.f;
  }
  if constexpr (PRO == PRO_RMSNORM) {
    float ss = 0.f;
    if (rs == 0) {  // each block counted once
#pragma unroll
      for (int j = 0; j < 32; ++j) ss = fmaf(xr[j], xr[j], ss);
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
    for (int j = 0; j < 32; ++j) xr[j] = xr[j] * inv * xb[j];
  }
  float xs = 0.f, xlo = 0.f;
  if constexpr (TYPE != PBX_F32 && TYPE != PBX_F16) {
#pragma unroll
    for (int i = 0; i < 16; ++i) xlo += xr[i];
    xs = xlo;
#pragma unroll
    for (int i = 16; i < 32; ++i) xs += xr[i];
  }

#pragma unroll
  for (int p = 0; p < P; ++p) {
    const bool ok = active && row_ok(p * rpw + rs);
    part[wave][p][lane] = ok ? block_term<TYPE>(q[p], ex[p], b, xr, xs, xlo, d[p], mn[p]) : 0.f;
  }
  __syncthreads();
  if constexpr (PAIR) {
    for (int t = lane; t < T / 2; t += 64) {
      const int tu = t + T / 2;
      float g = 0.f, u = 0.f;
      for (int j = 0; j < B; ++j) {
        g += part[wave][t / rpw][(t % rpw) * B + j];
        u += part[wave][tu / rpw][(tu % rpw) * B + j];
      }
      const int n = r0 + t;
      if (n < NO) yo[n] = silu(g) * u;
    }
    return;
  }
  uint64_t key = 0;
  for (int t = lane; t < T; t += 64) {
    const int p = t / rpw, r = t % rpw;
    float s = 0.f;
    for (int j = 0; j < B; ++j) s += part[wave][p][r * B + j];
    const int n = r0 + t;
    if (n < N) {
      epilogue_row<EPI>(a, y, n, s, t == lane ? res : y[n]);
      if constexpr (EPI == EPI_ARGMAX) {
        const uint64_t k = argmax_key(s, (unsigned)n);
        key = k > key ? k : key;
      }
    }
  }
  if constexpr (EPI == EPI_ARGMAX) {
    key = wave_max_u64(key);
    if (lane == 0) a.partials[blockIdx.x * 4 + wave] = key;
  }
}

// ---------------------------------------------------------------------------
// RMSNorm + f32 LM head with K = 32 BT (BT <= 16 blocks, the stories15M
// head: 32000 x 288 f32, llama.js:353-367) and argmax partials.  Eight
// lanes a row: lane (r, q) of a wave takes float4 columns q + 8 i (i < BT)
// of row r of each of P passes of 8 rows, so one load instruction of a wave
// reads eight whole 128-byte row segments (gemv_small's lane-per-block
// mapping touches 64 lines an instruction: 1.2 TB/s on this head).  The
// lane's 4 BT activations, normalised, stay in registers for every row.
// Workgroup: 4 waves x 8 P rows; one argmax key per wave.
// ---------------------------------------------------------------------------
template <int BT, int P>
__device__ __forceinline__ void gemv_tall_f32_lmh(const GemvArgs &a) {
  static_assert(BT >= 1 && BT <= 16, "K <= 512");
  const int N = a.N, K = BT * 32, F = K / 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r8 = lane >> 3, q = lane & 7;
  const float4 *X4 = reinterpret_cast<const float4 *>(a.X);
  const float4 *W4 = reinterpret_cast<const float4 *>(a.normw);
  const float4 *M4 = reinterpret_cast<const float4 *>(a.qs);
  float4 xv[BT], wv[BT];
#pragma unroll
  for (int i = 0; i < BT; ++i) {
    xv[i] = X4[q + 8 * i];
    wv[i] = W4[q + 8 * i];
  }
  const int r0 = ((int)blockIdx.x * 4 + wave) * 8 * P;
  float4 m[P][BT];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int row = r0 + 8 * p + r8;
    const size_t base = (size_t)(row < N ? row : 0) * F + q;
#pragma unroll
    for (int i = 0; i < BT; ++i) {
      const uint4 u = ld_stream(M4 + base + 8 * i);
      m[p][i] = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                            __uint_as_float(u.w));
    }
  }
  // RMSNorm: the lanes of row slot 0 hold every column once
  float ss = 0.f;
  if (r8 == 0) {
#pragma unroll
    for (int i = 0; i < BT; ++i)
      ss = fmaf(xv[i].x, xv[i].x, fmaf(xv[i].y, xv[i].y, fmaf(xv[i].z, xv[i].z, fmaf(xv[i].w, xv[i].w, ss))));
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
#pragma unroll
  for (int i = 0; i < BT; ++i)
    xv[i] = make_float4(xv[i].x * inv * wv[i].x, xv[i].y * inv * wv[i].y, xv[i].z * inv * wv[i].z,
                        xv[i].w * inv * wv[i].w);
  uint64_t key = 0;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < BT; ++i) {
      float &s = (i & 1) ? s1 : s0;
      s = fmaf(xv[i].x, m[p][i].x, fmaf(xv[i].y, m[p][i].y, fmaf(xv[i].z, m[p][i].z, fmaf(xv[i].w, m[p][i].w, s))));
    }
    const float t = wave_sum<4>(s0 + s1);  // the row's 8 lanes
    const int row = r0 + 8 * p + r8;
    if (q == 0 && row < N) {
      a.Y[row] = t;
      const uint64_t k = argmax_key(t, (unsigned)row);
      key = k > key ? k : key;
    }
  }
  key = wave_max_u64(key);
  if (lane == 0) a.partials[blockIdx.x * 4 + wave] = key;
}

// ---------------------------------------------------------------------------
// RMSNorm + Q8_0 LM head with K = 32 BT (BT <= 24 blocks: SmolLM2-135M's
// tied 49152 x 576 head) and argmax partials.  A row's codes are 2 BT
// 16-byte chunks (half a block each); eight lanes a row, lane (r, q)
// taking chunks q + 8 i, so a wave's load instruction reads eight 128-byte
// row segments.  The normalised activations are built once per workgroup
// in LDS; a lane keeps the 16 values of each of its chunks in registers and
// their sum (the codes enter as unsigned bytes, code + 128, and 128 sum(x)
// comes off).  Workgroup: 4 waves x 8 P rows; one argmax key per wave.
// ---------------------------------------------------------------------------
template <int BT, int P>
__device__ __forceinline__ void gemv_tall_q8_lmh(const GemvArgs &a) {
  static_assert(BT >= 1 && BT <= 24, "K <= 768");
  constexpr int K = BT * 32, NCH = 2 * BT, NC = (NCH + 7) / 8;
  __shared__ __attribute__((aligned(16))) float xs_l[K];
  __shared__ float red[4];
  const int N = a.N, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r8 = lane >> 3, q = lane & 7;
  const int r0 = ((int)blockIdx.x * 4 + wave) * 8 * P;
  // codes and scales first (clamped: rows past N read row 0, chunks past
  // the row read chunk q and get a zero scale)
  uint4 m[P][NC];
  unsigned dbits[P][NC];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int row = r0 + 8 * p + r8, rr = row < N ? row : 0;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = q + 8 * i, cc = c < NCH ? c : q;
      dbits[p][i] = a.dsc[dsc_index(rr, cc >> 1, BT)] & (c < NCH ? 0xFFFFu : 0u);
    }
  }
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int row = r0 + 8 * p + r8, rr = row < N ? row : 0;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = q + 8 * i, cc = c < NCH ? c : q;
      m[p][i] = ld_stream(a.qs + ((size_t)rr * NCH + cc) * 16);
    }
  }
  // RMSNorm of the activation row into LDS
  float ss = 0.f;
  for (int k = tid; k < K; k += 256) ss = fmaf(a.X[k], a.X[k], ss);
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + a.eps);
  for (int k = tid; k < K; k += 256) xs_l[k] = a.X[k] * inv * a.normw[k];
  __syncthreads();
  float xr[NC][16], xsum[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = q + 8 * i, cc = c < NCH ? c : q;
    xsum[i] = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 f = *reinterpret_cast<const float4 *>(&xs_l[16 * cc + 4 * v]);
      xr[i][4 * v] = f.x;
      xr[i][4 * v + 1] = f.y;
      xr[i][4 * v + 2] = f.z;
      xr[i][4 * v + 3] = f.w;
      xsum[i] += (f.x + f.y) + (f.z + f.w);
    }
  }
  uint64_t key = 0;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const unsigned w[4] = {m[p][i].x ^ 0x80808080u, m[p][i].y ^ 0x80808080u,
                             m[p][i].z ^ 0x80808080u, m[p][i].w ^ 0x80808080u};
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s = fmaf(xr[i][4 * j + 0], (float)(w[j] & 0xFFu), s);
        s = fmaf(xr[i][4 * j + 1], (float)((w[j] >> 8) & 0xFFu), s);
        s = fmaf(xr[i][4 * j + 2], (float)((w[j] >> 16) & 0xFFu), s);
        s = fmaf(xr[i][4 * j + 3], (float)(w[j] >> 24), s);
      }
      acc = fmaf(fmaf(-128.f, xsum[i], s), f16_bits_to_f32(dbits[p][i]), acc);
    }
    const float t = wave_sum<4>(acc);  // the row's 8 lanes
    const int row = r0 + 8 * p + r8;
    if (q == 0 && row < N) {
      a.Y[row] = t;
      const uint64_t k = argmax_key(t, (unsigned)row);
      key = k > key ? k : key;
    }
  }
  key = wave_max_u64(key);
  if (lane == 0) a.partials[blockIdx.x * 4 + wave] = key;
}

// ---------------------------------------------------------------------------
// Integer-limb GEMV for Q4_0 / Q8_0 (and Q6_K heads) with K >= 2048 (decode).
// The workgroup first turns the activation row(s) into fixed point, one
// power-of-two scale per 32-element block:
//   x_q = rint(x * w * 2^(21 - e_b)),  2^(e_b-1) <= max_b |x * w| < 2^e_b,
// (w: the RMSNorm weights, or 1) held in LDS as three signed-byte limbs
// x_q = x2*65536 + x1*256 + x0 plus the exact block sums of x_q and the
// block's 2^(e_b-21).  A block-row dot is then 8 v_dot4_i32_i8 per limb,
// exact in int32, combined once in fp32 with the block's scale and d.
// RMSNorm's 1/rms multiplies the finished sums (the dot is linear in x), so
// only the blocks' own maxima are needed before the limbs can be built.
// Rounding costs at most 2^-22 of the block's max |x * w| per element, against
// the ~75 VALU operations per block-row of the float unpack.
// Q = 1..4 consecutive lanes share a block (8/Q float4s each), so the block
// reductions are 0..2 DPP steps and no builder waits for another before the
// one barrier that publishes the limbs.
// Workgroup: WV waves x RT rows each (PAIR: RT/2 gate + RT/2 up rows); lane
// l owns blocks l, l+64, ... (IB of them) in the dots.
// ---------------------------------------------------------------------------
#define PBX_INT_MAXK 8192

__device__ __forceinline__ int sdot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Sum / max over aligned groups of Q consecutive lanes (Q = 1, 2, 4, 8:
// partners lane^1, lane^3, lane^7 stay inside the group).
template <int Q>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (Q >= 2) v += lane_partner<1>(v);
  if constexpr (Q >= 4) v += lane_partner<2>(v);
  if constexpr (Q >= 8) v += lane_partner<4>(v);
  return v;
}
template <int Q>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (Q >= 2) v = fmaxf(v, lane_partner<1>(v));
  if constexpr (Q >= 4) v = fmaxf(v, lane_partner<2>(v));
  if constexpr (Q >= 8) v = fmaxf(v, lane_partner<4>(v));
  return v;
}
template <int Q>
__device__ __forceinline__ int group_isum(int v) {
  if constexpr (Q >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  if constexpr (Q >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x1B, 0xF, 0xF, false);
  if constexpr (Q >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  return v;
}

// Fixed point of four products p (|p * scale| < 2^21): the float
// p * scale + 1.5 * 2^23 + 0x8080 holds rint(p * scale) + 0x8080 in its low
// 22 bits, so its bytes 0 and 1 are x0 + 128 and x1 + 128 and byte 2 is
// x2 + 64 (x_q = x0 + 256 x1 + 65536 x2, t = x_q + 0x8080 split by bytes).
// Out: the three limb words of the four elements (element i in byte i) and
// the sum of their x_q.
__device__ __forceinline__ void limb_words(float4 p, float scale, int &w0, int &w1, int &w2,
                                           int &sum) {
  constexpr float MAGIC = 12615808.0f;  // 1.5 * 2^23 + 0x8080
  const unsigned a = __float_as_uint(fmaf(p.x, scale, MAGIC));
  const unsigned b = __float_as_uint(fmaf(p.y, scale, MAGIC));
  const unsigned c = __float_as_uint(fmaf(p.z, scale, MAGIC));
  const unsigned d = __float_as_uint(fmaf(p.w, scale, MAGIC));
  // bits = 0x4B408080 + x_q
  sum = (int)(a + b + c + d - 4u * 0x4B408080u);
  const unsigned ab01 = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
  const unsigned cd01 = __builtin_amdgcn_perm(d, c, 0x05010400u);  // c0 d0 c1 d1
  const unsigned ab2 = __builtin_amdgcn_perm(b, a, 0x07030602u);   // a2 b2 . .
  const unsigned cd2 = __builtin_amdgcn_perm(d, c, 0x07030602u);   // c2 d2 . .
  w0 = (int)(__builtin_amdgcn_perm(cd01, ab01, 0x05040100u) ^ 0x80808080u);
  w1 = (int)(__builtin_amdgcn_perm(cd01, ab01, 0x07060302u) ^ 0x80808080u);
  // bytes x2 + 64 in [0x20, 0x60]: + 0x40 (no carries) then ^ 0x80 is x2 mod 256
  w2 = (int)((__builtin_amdgcn_perm(cd2, ab2, 0x05040100u) + 0x40404040u) ^ 0x80808080u);
}

// Schedules for one activation row without the tile loop:
//  * BW > 0: the first BW waves of the workgroup only build the limbs and
//    the WV waves after them only stream rows.  A builder reads the
//    activations in contiguous 1 KB chunks (lane l: float4 l % 8 of block
//    8 * chunk + l / 8) and writes the limb words of its blocks to LDS.  A
//    wave that builds and also streams rows can start its build only once
//    its weight requests have been accepted, and the CU accepts them about
//    as fast as earlier requests return, so the barrier would wait for
//    most of the weight stream (measured on the K = 8192 down GEMV: limbs
//    ready 2.0 us after the start with every wave building, 1.7 us with 8
//    builder waves beside the 4 row waves).
//  * PRE < RT: each wave requests rows 0..PRE-1 before the build and
//    barrier and the others after it, so the barrier is not held behind
//    the issue of the whole tile (16 x 4 gate|up: limbs ready 1.4 us after
//    the start instead of 2.1 us; the dots then overlap the stream).
// LOOP (lm heads, tall matrices): a workgroup takes tiles blockIdx.x,
// blockIdx.x + G, ... (G = gridDim.x) with the next tile's bytes in flight
// while a tile is reduced and builds the activation limbs once; EPI_ARGMAX
// writes one key per workgroup, EPI_STORE stores without a bias.
// MR > 1: MR activation rows (the first a.rows of them valid; row stride K
// in, N out) against one pass over the weight bytes -- the speculative
// verify and short prompts.  MR = 1: activation row blockIdx.y (the plain
// instruction's M < 4 rows).
template <int TYPE, int WV, int RT, int IB, int PRO, int EPI, bool LOOP = false, int MR = 1,
          int BW = 0, int PRE = RT>
__device__ __forceinline__ void gemv_int(const GemvArgs &a) {
  static_assert(TYPE == PBX_Q4 || TYPE == PBX_Q8 || is_q6k<TYPE>(), "quantised weights only");
  static_assert(BW == 0 || (MR == 1 && !LOOP && EPI != EPI_ARGMAX && (IB * 8) % BW == 0),
                "builder waves: one activation row, no tile loop, whole chunks per builder");
  static_assert(PRE >= 1 && (PRE >= RT || (MR == 1 && !LOOP)), "split issue: one row, no loop");
  static_assert(!LOOP || EPI == EPI_ARGMAX || EPI == EPI_STORE, "tile loop epilogues");
  static_assert(MR == 1 || EPI != EPI_ARGMAX, "argmax keys for one row");
  static_assert(EPI != EPI_ROPE || (MR == 1 && !LOOP && RT % 2 == 0), "RoPE rows in pairs");
  static_assert(PRO != PRO_RMSACC || (MR == 1 && !LOOP), "pending update: one activation row");
  static_assert(EPI != EPI_ADDACC || (MR == 1 && !LOOP), "pending update: one activation row");
  constexpr bool RMS = PRO == PRO_RMSNORM || PRO == PRO_RMSACC;
  constexpr int QB = BlockTraits<TYPE>::QB;
  constexpr int NV = QB / 16;
  constexpr bool PAIR = EPI == EPI_SWIGLU;
  static_assert(IB * 64 * 32 <= PBX_INT_MAXK, "K limit");
  constexpr int T = WV * 64;        // threads of the row waves
  constexpr int NB = MR * IB * 64;  // activation blocks (past B: unused)
  // lanes per block in the build, float4s a builder lane covers, and the
  // blocks a lane builds one after another (Q = 1 only).  With more than
  // four waves the blocks are not split: only wave 0 builds (MR = 1), its
  // activations requested first, while the others stream weight bytes.
  // PRO_RMSACC also loads 8 bytes of pending update per element, so four
  // waves share the build there (wave 0 alone would spill).
  constexpr int TB = T <= 256 ? T : PRO == PRO_RMSACC ? 256 : 64;
  constexpr int Q = TB >= 8 * NB ? 8 : TB >= 4 * NB ? 4 : TB >= 2 * NB ? 2 : 1;
  constexpr int FPL = 8 / Q;
  constexpr int IT = (NB * Q + T - 1) / T;
  // limb words 4q..4q+3 of block b at limb[m][L][q][b]: lane l's 16-byte
  // reads of block l are contiguous across the wave (no bank conflicts)
  __shared__ int4 limb[MR][3][2][IB * 64];
  // exact sums of a block's x_q ([0]; Q6_K: its two 16-element halves)
  __shared__ int bsum[MR][2][IB * 64];
  // the block's 2^(e_b - 21) (NaN: the block holds a non-finite x * w)
  __shared__ float bscale[MR][IB * 64];
  // RMSNorm: sums of x^2 of each 16-lane row of the builder waves, SSP per
  // activation row (a builder wave covers 64 / Q blocks of one row)
  constexpr int SSP = IB * Q * 4;
  __shared__ float4 ssq[RMS ? MR : 1][SSP / 4];
  __shared__ uint64_t kred[WV];
  __shared__ float ssqb[BW > 0 ? BW : 1];  // BW > 0: sum of x^2 of each builder wave

  const int N = a.N, B = a.B, K = B * 32;
  const int lane = threadIdx.x & 63, tid = threadIdx.x;
  // wave-uniform (SGPR): row bases and weight addresses are scalar arithmetic;
  // with builder waves, `wave` numbers the row waves (builders: negative)
  const int wave_hw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wave = wave_hw - BW;
  const int NO = PAIR ? N / 2 : N;
  const int rows = MR == 1 ? 1 : a.rows;  // valid activation rows
  constexpr int RTO = PAIR ? RT / 2 : RT;  // output rows a wave
  const int n_tiles = (NO + WV * RTO - 1) / (WV * RTO);
  // first output row of the wave in tile t
  auto rbase = [&](int t) -> int { return (t * WV + wave) * RTO; };
  auto tile_row = [&](int r0, int i) -> int {
    return PAIR ? (i < RT / 2 ? r0 + i : N / 2 + r0 + i - RT / 2) : r0 + i;
  };
  auto row_ok = [&](int r0, int i) -> bool {
    return PAIR ? (r0 + (i < RT / 2 ? i : i - RT / 2)) < NO : (r0 + i) < N;
  };
  constexpr int LPR = 64 / RT;  // lanes per row after the transposed reduction
  const float *X = a.X + (size_t)blockIdx.y * MR * K;
  float *y = a.Y + (size_t)blockIdx.y * MR * NO;
  const int pos = EPI == EPI_ROPE ? a.state[0] : 0;
  // EPI_ROPE with a.xcell: every output row is also published as a 64-bit
  // cell, (epoch + 1) << 32 | value bits, by a relaxed device-scope store,
  // for the attention workgroups of the same launch (no fence: each cell
  // carries its own epoch, so no ordering between cells is needed)
  unsigned pub_tag = 0;
  if constexpr (EPI == EPI_ROPE)
    if (a.xcell) pub_tag = cell_tag(a.xcell[N]);
  if constexpr (EPI == EPI_SWIGLU)
    if (a.xcell) pub_tag = cell_tag(a.xcell[N / 2]);
  if constexpr (BW > 0)
    if (a.adv && blockIdx.x == 0 && threadIdx.x == 0) *a.adv = next_epoch(*a.adv);
  if constexpr (EPI == EPI_ADDACC)
    if (a.xcell && blockIdx.x == 0 && threadIdx.x == 0) a.xcell[0] = next_epoch(a.xcell[0]);

  if constexpr (BW > 0) {
    if (wave < 0) {
      // builder wave wave_hw: chunks wave_hw, wave_hw + BW, ... of 256
      // activations (8 blocks), all requested before any arithmetic
      constexpr int CPB = IB * 8 / BW;
      const int qd = lane & 7;
      float4 xv[CPB], nv[CPB];
      i64x2_t qv[PRO == PRO_RMSACC ? CPB : 1][2];  // PRO_RMSACC: the pending update
#pragma unroll
      for (int c = 0; c < CPB; ++c) {
        const int e0 = (wave_hw + BW * c) * 256 + lane * 4;
        const int ec = e0 < K ? e0 : 0;
        xv[c] = *reinterpret_cast<const float4 *>(X + ec);
        nv[c] = make_float4(1.f, 1.f, 1.f, 1.f);
        if constexpr (RMS) nv[c] = *reinterpret_cast<const float4 *>(a.normw + ec);
        if constexpr (PRO == PRO_RMSACC) {
          qv[c][0] = *reinterpret_cast<const i64x2_t *>(a.acc + ec);
          qv[c][1] = *reinterpret_cast<const i64x2_t *>(a.acc + ec + 2);
        }
      }
      float sq = 0.f;
#pragma unroll
      for (int c = 0; c < CPB; ++c) {
        const int b = (wave_hw + BW * c) * 8 + (lane >> 3);
        const bool ok = b < B;
        float4 t = ok ? xv[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 w = nv[c];
        if constexpr (PRO == PRO_RMSACC)
          t = make_float4(residual_acc(t.x, qv[c][0].x), residual_acc(t.y, qv[c][0].y),
                          residual_acc(t.z, qv[c][1].x), residual_acc(t.w, qv[c][1].y));
        if constexpr (RMS)
          sq = fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, fmaf(t.w, t.w, sq))));
        const float4 p = make_float4(t.x * w.x, t.y * w.y, t.z * w.z, t.w * w.w);
        float mx = fmaxf(fmaxf(fabsf(p.x), fabsf(p.y)), fmaxf(fabsf(p.z), fabsf(p.w)));
        float nf = fmaf(p.x, 0.f, fmaf(p.y, 0.f, fmaf(p.z, 0.f, p.w * 0.f)));
        mx = group_max<8>(mx);
        nf = group_sum<8>(nf);
        int e = 0;
        if (mx > 0.f && mx < INFINITY) frexpf(mx, &e);
        e = max(e, -100);
        int w0, w1, w2, sv;
        limb_words(p, ldexpf(1.f, 21 - e), w0, w1, w2, sv);
        // float4s 0..3 of a block are its elements 0..15
        const int slo = group_isum<8>(qd < 4 ? sv : 0), shi = group_isum<8>(qd < 4 ? 0 : sv);
        if (ok) {
          reinterpret_cast<int *>(&limb[0][0][qd >> 2][b])[qd & 3] = w0;
          reinterpret_cast<int *>(&limb[0][1][qd >> 2][b])[qd & 3] = w1;
          reinterpret_cast<int *>(&limb[0][2][qd >> 2][b])[qd & 3] = w2;
          if (qd == 0) {
            bsum[0][0][b] = is_q6k<TYPE>() ? slo : slo + shi;
            bsum[0][1][b] = shi;
            bscale[0][b] = ldexpf(1.f, e - 21) + nf;
          }
        }
      }
      if constexpr (RMS) {
        sq = wave_sum(sq);
        if (lane == 0) ssqb[wave_hw] = sq;
      }
      lds_barrier();
      if (a.clr) {
        const int gi = (int)blockIdx.x * (BW * 64) + tid;
        if (2 * gi < a.clr_n) reinterpret_cast<i64x2_t *>(a.clr)[gi] = i64x2_t{0, 0};
      }
      return;
    }
  }

  // 1. Builder segments (segment s = L + T * it: block s / Q of the rows,
  //    its float4s FPL*(s % Q) ..) request their activations and RMSNorm
  //    weights before any wave requests weight bytes: a CU returns loads in
  //    issue order, so activations requested behind the weight stream would
  //    arrive only with it.  Loads are unconditional from clamped addresses.
  float4 xv[IT][FPL], nv[IT][FPL];
  i64x2_t qv[PRO == PRO_RMSACC ? IT : 1][PRO == PRO_RMSACC ? 2 * FPL : 1];  // pending updates
  // whole waves hold segments or none (NB * Q is a multiple of 64); the
  // others skip the build: waiting for loads they do not need would hold
  // the barrier behind their weight bytes
  auto builds = [&](int it) -> bool { return BW == 0 && wave * 64 + T * it < NB * Q; };
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if (!builds(it)) continue;
    const int sg = tid + T * it;
    const int gb = sg / Q, m = gb / (IB * 64), b = gb % (IB * 64), qd = sg % Q;
    const bool ok = b < B && m < rows;
    const float *xr = X + (ok ? (size_t)m * K + (size_t)b * 32 + qd * FPL * 4 : 0);
    const float *wr = a.normw + (ok ? (size_t)b * 32 + qd * FPL * 4 : 0);
#pragma unroll
    for (int v = 0; v < FPL; ++v) {
      xv[it][v] = *reinterpret_cast<const float4 *>(xr + 4 * v);
      nv[it][v] = make_float4(1.f, 1.f, 1.f, 1.f);
      if constexpr (RMS) nv[it][v] = *reinterpret_cast<const float4 *>(wr + 4 * v);
    }
    if constexpr (PRO == PRO_RMSACC) {
      const long long *qr = a.acc + (ok ? (size_t)b * 32 + qd * FPL * 4 : 0);
#pragma unroll
      for (int v = 0; v < 2 * FPL; ++v) qv[it][v] = *reinterpret_cast<const i64x2_t *>(qr + 2 * v);
    }
  }

  // 2. Every wave: the residuals it will add (EPI_ADD), the block scales,
  //    then the weight bytes.  Loads are unconditional from clamped
  //    addresses (rows past N read row 0 and are never stored, blocks past B
  //    read block 0 and get a zero scale where the dots use it) so the
  //    compiler issues them back to back; nothing is computed from a loaded
  //    value before the weight bytes are requested.
  float res[MR];
  long long racc = 0;  // EPI_ADDACC: the row's pending update
#pragma unroll
  for (int m = 0; m < MR; ++m) res[m] = 0.f;
  if constexpr (EPI == EPI_ADD || EPI == EPI_ADDACC) {
    const int r0 = rbase(blockIdx.x);
    const int rr = (lane % LPR) == 0 ? lane / LPR : RT;
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (rr < RT && r0 + rr < N) res[m] = y[(size_t)(m < rows ? m : 0) * NO + r0 + rr];
    if constexpr (EPI == EPI_ADDACC)
      if (rr < RT && r0 + rr < N) racc = a.acc[r0 + rr];
  }
  // Q6_K: db holds the super-block's d, ex the lane's two int8 sub-block
  // scales (load_lane); both are used only in the dots.
  // rows i0..i1-1 of tile t (constants after inlining)
  auto load_rows = [&](int t, int i0, int i1, unsigned (&db)[RT][IB], uint4 (&qq)[RT][IB][NV],
                       unsigned (&ex)[RT][IB]) {
    const int r0 = rbase(t);
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      if (i < i0 || i >= i1) continue;
      const int rw = row_ok(r0, i) ? tile_row(r0, i) : 0;
#pragma unroll
      for (int j = 0; j < IB; ++j) {
        const int b = lane + 64 * j, bb = b < B ? b : 0;
        db[i][j] = a.dsc[is_q6k<TYPE>() ? dsc_index(rw, bb >> 3, B >> 3) : dsc_index(rw, bb, B)];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      if (i < i0 || i >= i1) continue;
      const int rw = row_ok(r0, i) ? tile_row(r0, i) : 0;
#pragma unroll
      for (int j = 0; j < IB; ++j) {
        const int b = lane + 64 * j;
        ex[i][j] = 0u;
        if constexpr (is_q6k<TYPE>()) {
          load_lane<TYPE>(a.qs, rw, b, B, b < B, qq[i][j], ex[i][j]);
        } else {
          const uint8_t *src = a.qs + ((size_t)rw * B + (b < B ? b : 0)) * QB;
#pragma unroll
          for (int v = 0; v < NV; ++v) qq[i][j][v] = ld_stream(src + v * 16);
        }
      }
    }
  };
  auto load_tile = [&](int t, unsigned (&db)[RT][IB], uint4 (&qq)[RT][IB][NV],
                       unsigned (&ex)[RT][IB]) { load_rows(t, 0, RT, db, qq, ex); };
  constexpr int PRE_R = PRE < RT ? PRE : RT;  // rows requested before the barrier
  unsigned dbA[RT][IB], dbB[RT][IB], exA[RT][IB], exB[RT][IB];
  uint4 qA[RT][IB][NV], qB[RT][IB][NV];
  // LOOP: the workgroup's tiles are blockIdx.x + k*G, k < TW.  Loads are
  // issued without branches (the second from a clamped index when TW = 1):
  // behind a branch, the wait for an earlier load would also wait for
  // everything the branch may have issued.
  const int G = gridDim.x;
  const int TW = LOOP ? (n_tiles - (int)blockIdx.x + G - 1) / G : 1;
  load_rows(blockIdx.x, 0, PRE_R, dbA, qA, exA);
  if constexpr (LOOP) load_tile(blockIdx.x + (TW > 1 ? G : 0), dbB, qB, exB);
  __builtin_amdgcn_sched_barrier(0);

  // 3. Build: each segment's products x * w, their block's max |x * w| and
  //    exponent (over the Q lanes of the block), the fixed point as limb
  //    words, the block sums; then one barrier publishes them.  nf = sum of
  //    (x * w) * 0 is NaN exactly when a product is infinite or NaN (which
  //    fmaxf would drop); it makes the block's scale NaN, so every output
  //    of the row becomes NaN (the reference's sums are then NaN or +-inf).
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if (!builds(it)) continue;
    const int sg = tid + T * it;
    const int gb = sg / Q, m = gb / (IB * 64), b = gb % (IB * 64), qd = sg % Q;
    const bool ok = b < B && m < rows;
    float4 p[FPL];
    float mx = 0.f, nf = 0.f, sq = 0.f;
#pragma unroll
    for (int v = 0; v < FPL; ++v) {
      float4 t = ok ? xv[it][v] : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 w = nv[it][v];
      if constexpr (PRO == PRO_RMSACC) {
        const i64x2_t q0 = qv[it][2 * v], q1 = qv[it][2 * v + 1];
        t = make_float4(residual_acc(t.x, q0.x), residual_acc(t.y, q0.y), residual_acc(t.z, q1.x),
                        residual_acc(t.w, q1.y));
      }
      if constexpr (RMS)
        sq = fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, fmaf(t.w, t.w, sq))));
      p[v] = make_float4(t.x * w.x, t.y * w.y, t.z * w.z, t.w * w.w);
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(p[v].x), fabsf(p[v].y)), fmaxf(fabsf(p[v].z), fabsf(p[v].w))));
      nf = fmaf(p[v].x, 0.f, fmaf(p[v].y, 0.f, fmaf(p[v].z, 0.f, fmaf(p[v].w, 0.f, nf))));
    }
    if constexpr (Q > 1) {
      mx = group_max<Q>(mx);
      nf = group_sum<Q>(nf);
    }
    if constexpr (RMS) {
      // sum over the 16-lane row (DPP only); lane 16r of the wave writes it
      sq = wave_sum<8>(ok ? sq : 0.f);
      if ((lane & 15) == 0) {
        const int chunk = (wave * 64 + T * it) / Q - m * IB * 64;  // first block of the wave
        reinterpret_cast<float *>(&ssq[m][0])[chunk * Q / 64 * 4 + (lane >> 4)] = sq;
      }
    }
    int e = 0;
    if (mx > 0.f && mx < INFINITY) frexpf(mx, &e);
    e = max(e, -100);  // the scale stays finite; such blocks round to 0
    const float scale = ldexpf(1.f, 21 - e);
    int wl[3][FPL], slo = 0, shi = 0;
#pragma unroll
    for (int v = 0; v < FPL; ++v) {
      int sv;
      limb_words(p[v], scale, wl[0][v], wl[1][v], wl[2][v], sv);
      // float4 qd*FPL + v of the block: elements 0..15 are float4s 0..3
      if (qd * FPL + v < 4) slo += sv; else shi += sv;
    }
    if constexpr (Q > 1) {
      slo = group_isum<Q>(slo);
      shi = group_isum<Q>(shi);
    }
    if (ok) {
#pragma unroll
      for (int L = 0; L < 3; ++L) {
        const int f0 = qd * FPL;  // first word; words 4.. sit in the q = 1 plane
        if constexpr (FPL == 1) {
          reinterpret_cast<int *>(&limb[m][L][f0 >> 2][b])[f0 & 3] = wl[L][0];
        } else if constexpr (FPL == 2) {
          reinterpret_cast<int2 *>(&limb[m][L][f0 >> 2][b])[(f0 & 3) >> 1] =
              make_int2(wl[L][0], wl[L][1]);
        } else if constexpr (FPL == 4) {
          limb[m][L][f0 >> 2][b] = make_int4(wl[L][0], wl[L][1], wl[L][2], wl[L][3]);
        } else {
          limb[m][L][0][b] = make_int4(wl[L][0], wl[L][1], wl[L][2], wl[L][3]);
          limb[m][L][1][b] = make_int4(wl[L][4], wl[L][5], wl[L][6], wl[L][7]);
        }
      }
      if (qd == 0) {
        bsum[m][0][b] = is_q6k<TYPE>() ? slo : slo + shi;
        bsum[m][1][b] = shi;
        bscale[m][b] = ldexpf(1.f, e - 21) + nf;
      }
    }
  }
  lds_barrier();
  if constexpr (PRE_R < RT) load_rows(blockIdx.x, PRE_R, RT, dbA, qA, exA);
  // EPI_ROPE: cos and sin of the lane's row (its pair index inside the head)
  float2 rp = make_float2(1.f, 0.f);
  if constexpr (EPI == EPI_ROPE) {
    const int n = rbase(blockIdx.x) + lane / (64 / RT);
    const int i = ((n < a.qdim + a.kvdim ? n : 0) % a.head_dim) >> 1;
    rp = *reinterpret_cast<const float2 *>(a.rope + (size_t)pos * a.head_dim + 2 * i);
  }
  // RMSNorm's 1/rms of each activation row from the builders' row sums
  // (broadcast LDS reads, while the weight bytes are still arriving); it
  // multiplies the blocks' scales, so the dots need it and no wave
  // computes it at its tail
  float inv[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    inv[m] = 1.f;
    if constexpr (RMS) {
      float sm = 0.f;
      if constexpr (BW > 0) {
#pragma unroll
        for (int c = 0; c < BW; ++c) sm += ssqb[c];
      } else {
#pragma unroll
        for (int c = 0; c < SSP / 4; ++c) {
          const float4 v = ssq[m][c];
          sm += (v.x + v.y) + (v.z + v.w);
        }
      }
      inv[m] = 1.0f / sqrtf(sm / (float)K + a.eps);
    }
  }

  // 4. Dot products as the weight rows arrive; each row's sum after the
  //    transposed reduction, per activation row.
  auto dots = [&](const unsigned (&db)[RT][IB], const uint4 (&qq)[RT][IB][NV],
                  const unsigned (&ex)[RT][IB], float (&tot)[MR]) {
    float acc[MR][RT];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int i = 0; i < RT; ++i) acc[m][i] = 0.f;
#pragma unroll
    for (int j = 0; j < IB; ++j) {
      const int b = lane + 64 * j;
      const bool bok = b < B;
      const int bl = bok ? b : 0;  // lanes past B: zero scales cancel them
      const unsigned bmask = bok ? 0xFFFFu : 0u;
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (MR > 1 && m >= rows) break;  // uniform: rows past the batch
        int xl[3][8];
#pragma unroll
        for (int L = 0; L < 3; ++L) {
          const int4 t0 = limb[m][L][0][bl];
          const int4 t1 = limb[m][L][1][bl];
          xl[L][0] = t0.x; xl[L][1] = t0.y; xl[L][2] = t0.z; xl[L][3] = t0.w;
          xl[L][4] = t1.x; xl[L][5] = t1.y; xl[L][6] = t1.z; xl[L][7] = t1.w;
        }
        // the block's scale (times 1/rms) folded into the limb weights
        const float c0 = bok ? bscale[m][bl] * inv[m] : 0.f;
        const float C1 = 256.f * c0, C2 = 65536.f * c0;
        const float corr = TYPE == PBX_Q4 ? 8.f * (float)bsum[m][0][bl] * c0 : 0.f;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          int s0 = 0, s1 = 0, s2 = 0;
          if constexpr (TYPE == PBX_Q4) {
            // byte t holds element t (low nibble) and t+16 (high): word k
            // covers elements 4k..4k+3 (limb word k) and 16+4k.. (word 4+k)
            const unsigned w[4] = {qq[i][j][0].x, qq[i][j][0].y, qq[i][j][0].z, qq[i][j][0].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const int lo = (int)(w[k] & 0x0F0F0F0Fu), hi = (int)((w[k] >> 4) & 0x0F0F0F0Fu);
              s0 = sdot4(lo, xl[0][k], s0); s0 = sdot4(hi, xl[0][4 + k], s0);
              s1 = sdot4(lo, xl[1][k], s1); s1 = sdot4(hi, xl[1][4 + k], s1);
              s2 = sdot4(lo, xl[2][k], s2); s2 = sdot4(hi, xl[2][4 + k], s2);
            }
          } else if constexpr (is_q6k<TYPE>()) {
            // 6-bit codes of elements 4k..4k+3: low nibbles | 2-bit high
            // fields << 4; the two 16-element halves carry their own int8
            // scales.  Q6_K: the lane's ql bytes (high nibbles for groups 2,
            // 3) and qh bytes; lane-packed: nibble bytes (high nibbles for
            // codes 16..31) and one 2-bit field a byte per group of four.
            unsigned cw[8];
            if constexpr (TYPE == PBX_Q6K) {
              const unsigned shl = 4 * ((b & 3) >> 1), shh = 2 * (b & 3);
              const unsigned wl[8] = {qq[i][j][0].x, qq[i][j][0].y, qq[i][j][0].z, qq[i][j][0].w,
                                      qq[i][j][1].x, qq[i][j][1].y, qq[i][j][1].z, qq[i][j][1].w};
              const unsigned wh[8] = {qq[i][j][2].x, qq[i][j][2].y, qq[i][j][2].z, qq[i][j][2].w,
                                      qq[i][j][3].x, qq[i][j][3].y, qq[i][j][3].z, qq[i][j][3].w};
#pragma unroll
              for (int k = 0; k < 8; ++k)
                cw[k] = ((wl[k] >> shl) & 0x0F0F0F0Fu) | (((wh[k] >> shh) & 0x03030303u) << 4);
            } else {
              const unsigned wl[4] = {qq[i][j][0].x, qq[i][j][0].y, qq[i][j][0].z, qq[i][j][0].w};
              const unsigned wh[2] = {qq[i][j][1].x, qq[i][j][1].y};
#pragma unroll
              for (int k = 0; k < 8; ++k)
                cw[k] = ((wl[k & 3] >> (k < 4 ? 0 : 4)) & 0x0F0F0F0Fu) |
                        (((wh[k >> 2] >> (2 * (k & 3))) & 0x03030303u) << 4);
            }
            int h0 = 0, h1 = 0, h2 = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const int c = (int)cw[k];
              if (k < 4) {
                s0 = sdot4(c, xl[0][k], s0); s1 = sdot4(c, xl[1][k], s1); s2 = sdot4(c, xl[2][k], s2);
              } else {
                h0 = sdot4(c, xl[0][k], h0); h1 = sdot4(c, xl[1][k], h1); h2 = sdot4(c, xl[2][k], h2);
              }
            }
            const float flo = fmaf((float)s2, C2, fmaf((float)s1, C1, fmaf((float)s0, c0,
                              -32.f * (float)bsum[m][0][bl] * c0)));
            const float fhi = fmaf((float)h2, C2, fmaf((float)h1, C1, fmaf((float)h0, c0,
                              -32.f * (float)bsum[m][1][bl] * c0)));
            const float sc0 = (float)(int8_t)(ex[i][j] & 0xFFu);
            const float sc1 = (float)(int8_t)((ex[i][j] >> 8) & 0xFFu);
            acc[m][i] = fmaf(fmaf(sc0, flo, sc1 * fhi), f16_bits_to_f32(db[i][j] & bmask),
                             acc[m][i]);
            continue;
          } else {
            const unsigned w[8] = {qq[i][j][0].x, qq[i][j][0].y, qq[i][j][0].z, qq[i][j][0].w,
                                   qq[i][j][1].x, qq[i][j][1].y, qq[i][j][1].z, qq[i][j][1].w};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              s0 = sdot4((int)w[k], xl[0][k], s0);
              s1 = sdot4((int)w[k], xl[1][k], s1);
              s2 = sdot4((int)w[k], xl[2][k], s2);
            }
          }
          const float f = fmaf((float)s2, C2, fmaf((float)s1, C1, fmaf((float)s0, c0, -corr)));
          acc[m][i] = fmaf(f, f16_bits_to_f32(db[i][j] & bmask), acc[m][i]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) tot[m] = wave_transpose_reduce<RT>(acc[m], lane);
  };
  const int row = lane / LPR;

  if constexpr (LOOP) {
    // tiles k (registers A) and k + 1 (B); each buffer is refilled with the
    // tile two on as soon as it has been reduced.  The steady-state loop
    // issues its loads unconditionally; the last two or three tiles follow.
    uint64_t best = 0;
    auto consume = [&](int k, const float (&tt)[MR]) {
      const int n = rbase(blockIdx.x + k * G) + row;
      if ((lane % LPR) == 0 && n < N) {
#pragma unroll
        for (int m = 0; m < MR; ++m)  // no bias in the loop (a load here would wait)
          if (m < rows) y[(size_t)m * NO + n] = tt[m];
        if constexpr (EPI == EPI_ARGMAX) {
          const uint64_t key = argmax_key(tt[0], (unsigned)n);
          best = key > best ? key : best;
        }
      }
    };
    float tt[MR];
    int k = 0;
    for (; k + 3 < TW; k += 2) {
      dots(dbA, qA, exA, tt);
      load_tile(blockIdx.x + (k + 2) * G, dbA, qA, exA);
      consume(k, tt);
      dots(dbB, qB, exB, tt);
      load_tile(blockIdx.x + (k + 3) * G, dbB, qB, exB);
      consume(k + 1, tt);
    }
    dots(dbA, qA, exA, tt);
    if (k + 2 < TW) load_tile(blockIdx.x + (k + 2) * G, dbA, qA, exA);
    consume(k, tt);
    if (k + 1 < TW) {
      dots(dbB, qB, exB, tt);
      consume(k + 1, tt);
    }
    if (k + 2 < TW) {
      dots(dbA, qA, exA, tt);
      consume(k + 2, tt);
    }
    if constexpr (EPI != EPI_ARGMAX) return;
    best = wave_max_u64(best);
    if (lane == 0) kred[wave] = best;
    __syncthreads();
    if (tid == 0) {
      uint64_t kk = kred[0];
#pragma unroll
      for (int w = 1; w < WV; ++w) kk = kred[w] > kk ? kred[w] : kk;
      a.partials[blockIdx.x] = kk;
    }
    return;
  }

  float tot[MR];
  dots(dbA, qA, exA, tot);
  const int r0 = rbase(blockIdx.x);
  if constexpr (EPI == EPI_ROPE) {
    // rows 2i, 2i+1 sit LPR lanes apart after the transposed reduction
    float pt;
    if constexpr (LPR == 8 || LPR >= 16)
      pt = lane_partner<LPR>(tot[0]);  // exact lane ^ LPR
    else
      pt = __shfl_xor(tot[0], LPR, 64);
    if ((lane % LPR) == 0) {
      const int n = r0 + row;
      const float t = tot[0];
      if (n < a.qdim + a.kvdim) {
        // (x0, x1) -> (x0 c - x1 s, x0 s + x1 c)
        const float o = (n & 1) ? fmaf(pt, rp.y, t * rp.x) : fmaf(t, rp.x, -pt * rp.y);
        if (n < a.qdim) y[n] = o;
        else a.kcache[(size_t)pos * a.kvdim + (n - a.qdim)] = o;
        if (pub_tag)
          __hip_atomic_store(a.xcell + n, (unsigned long long)pub_tag << 32 | __float_as_uint(o),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else if (n < N) {
        a.vcache[(size_t)pos * a.kvdim + (n - a.qdim - a.kvdim)] = t;
        if (pub_tag)
          __hip_atomic_store(a.xcell + n, (unsigned long long)pub_tag << 32 | __float_as_uint(t),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    return;
  }
  if constexpr (PAIR) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float up = lane_partner<32>(tot[m]);
      if (m < rows && lane < 32 && (lane % LPR) == 0) {
        const int n = r0 + row;
        if (n < NO) {
          const float h = silu(tot[m]) * up;
          y[(size_t)m * NO + n] = h;
          if (pub_tag)  // the joined FFN launch: the down slices wait for it
            __hip_atomic_store(a.xcell + n, (unsigned long long)pub_tag << 32 | __float_as_uint(h),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    return;
  }
  uint64_t key = 0;
  if ((lane % LPR) == 0) {
    const int n = r0 + row;
    if (n < N) {
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < rows) epilogue_row<EPI>(a, y + (size_t)m * NO, n, tot[m], res[m], racc);
      if constexpr (EPI == EPI_ARGMAX) key = argmax_key(tot[0], (unsigned)n);
    }
  }
  if constexpr (EPI == EPI_ARGMAX) {
    key = wave_max_u64(key);
    if (lane == 0) kred[wave] = key;
    __syncthreads();
    if (tid == 0) {
      uint64_t best = kred[0];
#pragma unroll
      for (int w = 1; w < WV; ++w) best = kred[w] > best ? kred[w] : best;
      a.partials[blockIdx.x] = best;
    }
  }
}


// The cross-workgroup combine of gemv_mr with XS > 1: every slice adds its
// sum of an output element into the element's 64-bit cell (bits 0..55: the
// sum of the slices' 2^-32 fixed-point values, each biased by 2^51 so the
// field stays non-negative; bits 56..59: slices arrived; bits 60..63:
// slices whose sum was not finite or not below 2^19 in magnitude).  The add
// that brings the count to XS returns the whole sum: that lane stores
// residual + sum (NaN when a slice was poisoned) and clears the cell.  One
// atomic carries value and count, so no fence is needed, and integer
// addition makes the result independent of the arrival order.
template <int XS, int MR>
__device__ __forceinline__ void mr_combine(const GemvArgs &a, bool has, int mcol, int n0,
                                           const float (&acc)[4], const float (&res)[4]) {
  static_assert(XS < 16, "4-bit counts");
  if (!has) return;
  const int N = a.N;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = n0 + i;
    if (n >= N) continue;
    const float p = acc[i];
    const bool bad = !(fabsf(p) < 0x1p19f);
    const unsigned long long c =
        (1ull << 56) + (bad ? (1ull << 60) + (1ull << 51)
                            : (unsigned long long)((1ll << 51) + (long long)rintf(p * 0x1p32f)));
    unsigned long long *cell = a.xcell + (size_t)mcol * N + n;
    const unsigned long long t =
        __hip_atomic_fetch_add(cell, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + c;
    if (((t >> 56) & 15u) != (unsigned)XS) continue;
    __hip_atomic_store(cell, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const long long v = (long long)(t & ((1ull << 56) - 1)) - (long long)XS * (1ll << 51);
    a.Y[(size_t)mcol * N + n] =
        (t >> 60) ? __builtin_nanf("") : (float)fma((double)v, 0x1p-32, (double)res[i]);
  }
}

// ---------------------------------------------------------------------------
// Row-batched GEMV on int8 MFMAs: up to MR = 5 activation rows against one
// pass over Q4_0 weights (K = 2048..8192), for the speculative verify and
// short prompts.  The activations are fixed point as in gemv_int (per row
// and 32-block: x_q = rint(x w 2^(21-e)) in three signed byte limbs), held
// in LDS as the B operand of v_mfma_i32_16x16x32_i8: column c = 3m + L is
// limb L of activation row m (column 15 is zero).  The A operand is the
// codes (0..15) of one block of 16 weight rows.  Operand lanes (checked on
// the device): A lane l holds A[l%16][8(l/16) + j], B lane l holds
// B[8(l/16) + j][l%16], D lane l holds D[4(l/16) + r][l%16].  Element order
// inside a block (the same for A and B): lane group g takes elements
// 4g..4g+3 (low nibbles of bytes 4g..4g+3, limb word g) then 16+4g..16+4g+3
// (their high nibbles, limb word 4+g).  One MFMA a block gives the exact
// integer dots of 16 weight rows with every limb of every row; the lane of
// column (m, L) adds dot * 256^L * 2^(e_mb - 21) / rms_m * d_nb, less
// 8 sum(x_q) on limb 0 (the Q4_0 offset), for its 4 weight rows, and the
// three limb lanes of a row are summed at the end.
// Weight bytes move in 16-byte loads, lane l taking block b + l/16 of row
// l%16 (whole cache-line pieces), and through a 1 KB LDS slot of the wave
// into the A layout (lane l's 16 bytes at 16 l: the A reads of one block hit
// 64 distinct banks); the tile's fp16 row scales likewise in 16-byte loads
// (lane l: row group l/16, two blocks) through a per-wave LDS table.  The B operand of block b lives at slots
// 64 b + ((4c + g) ^ (b & 31)) (int2 each), so the builders' writes of one
// word over 64 blocks spread over the banks and the A-side reads of one
// block stay a permutation of its 64 slots.
// Workgroup: RW x KS waves; wave w computes weight-row tiles (16 rows;
// EPI_SWIGLU: 8 gate rows then their 8 up rows) over the w / RW -th of KS
// slices of the blocks; slices are summed through LDS.  LOOP (KS = 1): the
// workgroup takes tiles blockIdx.x * RW + w % RW + k * gridDim.x * RW, the
// next tile's weights requested while one is multiplied.
// EPI_ROPE: rows of q|k|v at positions pos0 + m (RoPE of q and k, k and v
// written to the cache rows, q to Y).
// XS > 1 (EPI_ADD): the K blocks are split over XS workgroups (blockIdx.y),
// so a workgroup builds and reads only its slice of the activation rows
// (they dominate a CU's bytes at K = 8192); the slices meet in mr_combine.
// ---------------------------------------------------------------------------
typedef int pbx_v4i __attribute__((ext_vector_type(4)));

template <int RW, int KS, int IB, int PRO, int EPI, int MR, bool LOOP = false, int XS = 1>
__device__ __forceinline__ void gemv_mr(const GemvArgs &a) {
  static_assert(MR >= 1 && 3 * MR <= 15, "three limb columns a row, 16 columns");
  static_assert(EPI == EPI_STORE || EPI == EPI_ADD || EPI == EPI_SWIGLU || EPI == EPI_ROPE,
                "epilogues");
  static_assert(!LOOP || (KS == 1 && EPI == EPI_STORE), "tile loop: one slice, stored rows");
  static_assert(XS == 1 || (EPI == EPI_ADD && PRO == PRO_NONE && !LOOP),
                "K split over workgroups: residual add epilogue");
  static_assert((IB * 64) % XS == 0 && (IB * 64 / XS) % (4 * KS) == 0, "whole 4-block steps a slice");
  constexpr int WV = RW * KS, T = WV * 64;
  constexpr int NB = IB * 64 / XS;  // blocks of the workgroup's K slice (past B: unused)
  constexpr bool PAIR = EPI == EPI_SWIGLU;
  // build segments: a block of every activation row, Q lanes each (the
  // block's RMSNorm weights are read once for all rows)
  constexpr int NSEG = NB;
  // 8 lanes a block: each wave reads 1 KB contiguous per activation load
  // (one lane a block reads 64 cache lines per instruction, several times
  // slower for these sizes)
  constexpr int Q = 8;
  constexpr int FPL = 8 / Q;
  constexpr int IT = (NSEG * Q + T - 1) / T;
  constexpr int CH = NB * Q / 64;       // wave-chunks of the blocks
  constexpr int BSM = (NB + KS - 1) / KS;  // blocks a slice at most
  constexpr int NQ = (BSM + 3) / 4;        // 4-block loads a slice
  constexpr int NSC = (BSM + 31) / 32;     // 16-byte scale loads a lane
  __shared__ int2 xb[NB * 64];          // B operand (see the slot rule above)
  __shared__ float2 xsc[NB][MR];        // 2^(e - 21) (NaN: non-finite block), 8 sum(x_q) of it
  __shared__ float ssq[MR][CH];         // RMSNorm: sum of x^2 per wave-chunk
  // a wave's 4 weight blocks (during the dots), then the K-slice partials
  constexpr int RED = (KS > 1 ? KS - 1 : 1) * RW * 64;  // float4s
  constexpr int NSLOT = IB > 2 ? 1 : 2;  // weight slots a wave (LDS budget at K = 8192)
  __shared__ float4 wst_red[WV * 64 * NSLOT > RED ? WV * 64 * NSLOT : RED];
  __shared__ __attribute__((aligned(16))) uint2 wsc[WV][4][NSC * 32];  // row group, block

  // BR blocks a weight row; B blocks (K activations) in this workgroup's
  // K slice, starting at block gb0
  const int N = a.N, BR = a.B, KR = BR * 32, B = BR / XS, K = B * 32;
  const int gb0 = XS > 1 ? (int)blockIdx.y * B : 0;
  const int lane = threadIdx.x & 63, tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rw = wave % RW, ks = wave / RW;
  const int NO = PAIR ? N / 2 : N;
  const int rows = a.rows;
  const int col = lane & 15, g = lane >> 4;
  const int mcol = col / 3, lcol = col - 3 * mcol;  // activation row and limb of the column
  const int n_tiles = (NO + (PAIR ? 7 : 15)) / (PAIR ? 8 : 16);
  auto tile_r0 = [&](int t) -> int { return PAIR ? t * 8 : t * 16; };
  auto wrow = [&](int r0, int i) -> int {  // weight row of tile row i (0..15)
    return PAIR ? (i < 8 ? r0 + i : N / 2 + r0 + i - 8) : r0 + i;
  };
  auto wrow_ok = [&](int r0, int i) -> bool { return (PAIR ? r0 + (i & 7) : r0 + i) < NO; };
  // the wave's K slice
  const int BS = (B + KS - 1) / KS, b0 = ks * BS, b1 = min(B, b0 + BS);

  // 1. activation segments (block b of every row; Q lanes each), requested first
  float4 xv[IT][MR][FPL], nv[IT][FPL];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int sg = tid + T * it;
    const int b = sg / Q, qd = sg % Q;
    if (b >= NB) continue;  // wave-uniform: whole waves hold segments or none
    const bool okb = b < B;
    const float *wr = a.normw + (okb ? (size_t)(gb0 + b) * 32 + qd * FPL * 4 : 0);
#pragma unroll
    for (int v = 0; v < FPL; ++v) {
      nv[it][v] = make_float4(1.f, 1.f, 1.f, 1.f);
      if constexpr (PRO == PRO_RMSNORM) nv[it][v] = *reinterpret_cast<const float4 *>(wr + 4 * v);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const bool ok = m < rows && okb;
      const float *xr = a.X + (ok ? (size_t)m * KR + (size_t)(gb0 + b) * 32 + qd * FPL * 4 : 0);
#pragma unroll
      for (int v = 0; v < FPL; ++v) xv[it][m][v] = *reinterpret_cast<const float4 *>(xr + 4 * v);
    }
  }
  // 2. the first tile's residuals (EPI_ADD), row scales and weights
  const int t0 = blockIdx.x * RW + rw;
  float res[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) res[i] = 0.f;
  if constexpr (EPI == EPI_ADD) {
    const int r0 = tile_r0(t0);
    if (lcol == 0 && mcol < MR) {
      const int mm = mcol < rows ? mcol : 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ti = 4 * g + i;
        res[i] = a.Y[(size_t)mm * NO + (wrow_ok(r0, ti) ? wrow(r0, ti) : 0)];
      }
    }
  }
  // tile t: row scales (lane l: rows 4(l/16)..+3 of the tile, blocks
  // b0 + 32 s + 2(l%16), +1), 16-byte weight pieces (lane l: row l%16,
  // blocks b0 + 4q + l/16)
  auto load_tile = [&](int t, uint4 (&wd)[NSC], uint4 (&wq)[NQ]) {
    const int r0 = tile_r0(t < n_tiles ? t : 0);
    const int rd = wrow_ok(r0, 4 * g) ? wrow(r0, 4 * g) : 0;
#pragma unroll
    for (int sgi = 0; sgi < NSC; ++sgi) {
      const int b = b0 + 32 * sgi + 2 * col;  // even: the pair lies inside B
      // a vector load (a struct copy would go through private memory)
      const u32x4_t v =
          *reinterpret_cast<const u32x4_t *>(a.dsc + dsc_index(rd, gb0 + (b + 1 < b1 ? b : b0), BR));
      wd[sgi] = make_uint4(v.x, v.y, v.z, v.w);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int ra = wrow_ok(r0, col) ? wrow(r0, col) : 0;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int b = b0 + 4 * q + g;
      wq[q] = ld_stream(a.qs + ((size_t)ra * BR + gb0 + (b < b1 ? b : b0)) * 16);
    }
  };
  uint4 wdA[NSC], wdB[NSC];
  uint4 wqA[NQ], wqB[NQ];
  load_tile(t0, wdA, wqA);
  const int G = gridDim.x * RW;  // LOOP: tiles a step
  if constexpr (LOOP) load_tile(t0 + G, wdB, wqB);
  __builtin_amdgcn_sched_barrier(0);

  // 3. build: fixed point of each segment into the B operand slots
#pragma unroll
  for (int it = 0; it < IT; ++it)
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const int sg = tid + T * it;
    const int b = sg / Q, qd = sg % Q;
    if (b >= NB) continue;  // wave-uniform
    const bool ok = m < rows && b < B;
    float4 p[FPL];
    float mx = 0.f, nf = 0.f, sq = 0.f;
#pragma unroll
    for (int v = 0; v < FPL; ++v) {
      const float4 x = ok ? xv[it][m][v] : make_float4(0.f, 0.f, 0.f, 0.f), w = nv[it][v];
      if constexpr (PRO == PRO_RMSNORM)
        sq = fmaf(x.x, x.x, fmaf(x.y, x.y, fmaf(x.z, x.z, fmaf(x.w, x.w, sq))));
      p[v] = make_float4(x.x * w.x, x.y * w.y, x.z * w.z, x.w * w.w);
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(p[v].x), fabsf(p[v].y)), fmaxf(fabsf(p[v].z), fabsf(p[v].w))));
      nf = fmaf(p[v].x, 0.f, fmaf(p[v].y, 0.f, fmaf(p[v].z, 0.f, fmaf(p[v].w, 0.f, nf))));
    }
    if constexpr (Q > 1) {
      mx = group_max<Q>(mx);
      nf = group_sum<Q>(nf);
    }
    if constexpr (PRO == PRO_RMSNORM) {
      sq = wave_sum(sq);  // row m over the wave's 8 blocks
      if (lane == 0) ssq[m][(tid + T * it) / 64] = sq;
    }
    int e = 0;
    if (mx > 0.f && mx < INFINITY) frexpf(mx, &e);
    e = max(e, -100);
    const float scale = ldexpf(1.f, 21 - e);
    int sum = 0;
    int *xbi = reinterpret_cast<int *>(xb);
    const int sw = b & 31;
#pragma unroll
    for (int v = 0; v < FPL; ++v) {
      int w0, w1, w2, sv;
      limb_words(p[v], scale, w0, w1, w2, sv);
      sum += sv;
      // word k = float4 k of the block: lane group k & 3, half k >> 2
      const int k = qd * FPL + v, gg = k & 3, hf = k >> 2;
      const int base = 2 * (64 * b);
      xbi[base + 2 * ((4 * (3 * m) + gg) ^ sw) + hf] = w0;
      xbi[base + 2 * ((4 * (3 * m + 1) + gg) ^ sw) + hf] = w1;
      xbi[base + 2 * ((4 * (3 * m + 2) + gg) ^ sw) + hf] = w2;
      if (m == 0) xbi[base + 2 * ((4 * 15 + gg) ^ sw) + hf] = 0;
    }
    if constexpr (Q > 1) sum = group_isum<Q>(sum);
    if (qd == 0) {
      const float c0 = ldexpf(1.f, e - 21) + nf;
      xsc[b][m] = make_float2(c0, 8.f * (float)sum * c0);
    }
  }
  lds_barrier();

  // 4. dots: one MFMA a block, the lane's column scales, 4 weight rows a lane
  float inv = 1.f;  // 1/rms of the lane's activation row
  if constexpr (PRO == PRO_RMSNORM) {
    if (mcol < MR) {
      float sm = 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c) sm += ssq[mcol][c];
      inv = 1.0f / sqrtf(sm / (float)K + a.eps);
    }
  }
  const float fl = (lcol == 0 ? 1.f : lcol == 1 ? 256.f : 65536.f) * inv;
  const float fk = lcol == 0 ? inv : 0.f;  // the code offset on limb 0 only
  const int mc = mcol < MR ? mcol : 0;
  const int slot = 4 * col + g;
  unsigned *wsl = reinterpret_cast<unsigned *>(wst_red) + 256 * NSLOT * wave;
  auto dots = [&](const uint4 (&wd)[NSC], const uint4 (&wq)[NQ], float (&acc)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = 0.f;
    // the tile's scales into the wave's table: group g, blocks 32 s + 2 col, +1
    // (kept after the weight requests: a store moved above them would wait
    // for the scales before the weights are requested)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int sgi = 0; sgi < NSC; ++sgi) {
      const u32x4_t v = {wd[sgi].x, wd[sgi].y, wd[sgi].z, wd[sgi].w};
      *reinterpret_cast<u32x4_t *>(&wsc[wave][g][32 * sgi + 2 * col]) = v;
    }
    // 4 blocks a step through the wave's LDS slots (two alternate when the
    // budget allows: the next step's weights are stored while this step's
    // operands are read); the step's 4 MFMAs issue back to back and their
    // results are scaled after them.  A wave's LDS operations complete in
    // order, so a slot is rewritten only after the reads issued before.
    auto stage = [&](int q) {
      const u32x4_t wv = {wq[q].x, wq[q].y, wq[q].z, wq[q].w};
      *reinterpret_cast<u32x4_t *>(wsl + 256 * (q % NSLOT) + 4 * lane) = wv;
    };
    if constexpr (NSLOT == 2) stage(0);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if constexpr (NSLOT == 2) {
        if (q + 1 < NQ) stage(q + 1);
      } else {
        stage(q);
      }
      const unsigned *sl = wsl + 256 * (q % NSLOT);
      unsigned w[4];
      int2 bo[4];
      float2 cs[4];
      uint2 dw[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = 4 * q + u, b = b0 + j;
        w[u] = sl[4 * (col + 16 * u) + g];  // row col, block b: dword g
        bo[u] = xb[64 * b + (slot ^ (b & 31))];
        cs[u] = xsc[b][mc];
        dw[u] = wsc[wave][g][j];
      }
      pbx_v4i d[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const long ao =
            (long)(((unsigned long long)((w[u] >> 4) & 0x0F0F0F0Fu) << 32) | (w[u] & 0x0F0F0F0Fu));
        const long bl = (long)(((unsigned long long)(unsigned)bo[u].y << 32) | (unsigned)bo[u].x);
        const pbx_v4i z = {0, 0, 0, 0};
        d[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ao, bl, z, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float c = cs[u].x * fl, kk = cs[u].y * fk;
        acc[0] = fmaf(fmaf((float)d[u][0], c, -kk), f16_bits_to_f32(dw[u].x), acc[0]);
        acc[1] = fmaf(fmaf((float)d[u][1], c, -kk), f16_bits_to_f32(dw[u].x >> 16), acc[1]);
        acc[2] = fmaf(fmaf((float)d[u][2], c, -kk), f16_bits_to_f32(dw[u].y), acc[2]);
        acc[3] = fmaf(fmaf((float)d[u][3], c, -kk), f16_bits_to_f32(dw[u].y >> 16), acc[3]);
      }
    }
    // limbs 0..2 of a row sit in columns 3m..3m+2 (adjacent lanes): DPP
    // row_shl:1 and :2 read lanes +1 and +2 of the 16-lane row (column 3m
    // <= 12 finds both inside it; the other lanes' sums are not used)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = __float_as_int(acc[i]);
      acc[i] += __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x101, 0xF, 0xF, false)) +
                __int_as_float(__builtin_amdgcn_update_dpp(0, v, 0x102, 0xF, 0xF, false));
    }
  };

  float acc[4];
  if constexpr (LOOP) {
    // tiles t0 + k G: registers A, B alternate, each refilled two tiles on
    for (int k = 0;; k += 2) {
      const int ta = t0 + k * G;
      if (ta >= n_tiles) break;
      dots(wdA, wqA, acc);
      load_tile(ta + 2 * G, wdA, wqA);
      if (lcol == 0 && mcol < rows) {
        const int r0 = tile_r0(ta);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = r0 + 4 * g + i;
          if (n < N) a.Y[(size_t)mcol * NO + n] = acc[i];
        }
      }
      const int tb = ta + G;
      if (tb >= n_tiles) break;
      dots(wdB, wqB, acc);
      load_tile(tb + 2 * G, wdB, wqB);
      if (lcol == 0 && mcol < rows) {
        const int r0 = tile_r0(tb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = r0 + 4 * g + i;
          if (n < N) a.Y[(size_t)mcol * NO + n] = acc[i];
        }
      }
    }
    return;
  }

  dots(wdA, wqA, acc);
  // K slices: slices 1.. through LDS (over the weight slots, once every
  // wave is past its dots), slice 0 sums and finishes
  if constexpr (KS > 1) {
    lds_barrier();
    if (ks > 0) wst_red[((ks - 1) * RW + rw) * 64 + lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    lds_barrier();
    if (ks > 0) return;
#pragma unroll
    for (int s = 0; s < KS - 1; ++s) {
      const float4 v = wst_red[(s * RW + rw) * 64 + lane];
      acc[0] += v.x; acc[1] += v.y; acc[2] += v.z; acc[3] += v.w;
    }
  }
  const int r0 = tile_r0(t0);
  if (t0 >= n_tiles) return;
  if constexpr (XS > 1) {
    mr_combine<XS, MR>(a, lcol == 0 && mcol < rows, mcol, r0 + 4 * g, acc, res);
    return;
  }
  if constexpr (PAIR) {
    // tile rows 0..7 (lane groups 0, 1) are gate rows, 8..15 their up rows
    float up[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) up[i] = lane_partner<32>(acc[i]);
    if (lcol == 0 && mcol < rows && g < 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = r0 + 4 * g + i;
        if (n < NO) a.Y[(size_t)mcol * NO + n] = silu(acc[i]) * up[i];
      }
    }
    return;
  }
  if (lcol != 0 || mcol >= rows) return;
  if constexpr (EPI == EPI_ROPE) {
    const int pos = a.pos0 + mcol;
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
      const int n = r0 + 4 * g + i;  // even: rows n, n + 1 are a RoPE pair
      if (n >= N) continue;
      if (n < a.qdim + a.kvdim) {
        const float2 cs = *reinterpret_cast<const float2 *>(
            a.rope + (size_t)pos * a.head_dim + (n % a.head_dim));
        const float o0 = fmaf(acc[i], cs.x, -acc[i + 1] * cs.y);
        const float o1 = fmaf(acc[i], cs.y, acc[i + 1] * cs.x);
        if (n < a.qdim) {
          a.Y[(size_t)mcol * N + n] = o0;
          a.Y[(size_t)mcol * N + n + 1] = o1;
        } else {
          float *kc = a.kcache + (size_t)pos * a.kvdim + (n - a.qdim);
          kc[0] = o0;
          kc[1] = o1;
        }
      } else {
        float *vc = a.vcache + (size_t)pos * a.kvdim + (n - a.qdim - a.kvdim);
        vc[0] = acc[i];
        vc[1] = acc[i + 1];
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = r0 + 4 * g + i;
    if (n < N) a.Y[(size_t)mcol * NO + n] = EPI == EPI_ADD ? res[i] + acc[i] : acc[i];
  }
}


}  // namespace pbx

#endif
