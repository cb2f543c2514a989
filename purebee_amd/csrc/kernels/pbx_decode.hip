// pbx_decode.hip -- gfx950 kernels of the on-GPU Llama decode step.
//
// One decode token (llama.js:204-371 at seqLen 1; llama-streaming.js:505-606)
// runs as, per layer:
//   1. GEMV  x -> [q|k|v]           RMSNorm(x, attn_norm) fused as prologue
//   2. attention                     RoPE, KV-cache append, softmax(q.K)V
//   3. GEMV  attn -> x (+=)          residual add fused as epilogue
//   4. GEMV  x -> silu(gate)*up      RMSNorm(x, ffn_norm) prologue; each
//                                    workgroup pairs gate and up rows
//   5. GEMV  h -> x (+=)             residual epilogue
// then the LM head GEMV (RMSNorm(x, output_norm) prologue, per-tile argmax
// partials epilogue) and a one-workgroup argmax that also advances the
// device-side position, so consecutive steps replay without the host.
// Device state: state[0] = position, state[1] = current token, state[2] =
// step counter (index into the generated-token history).

#include "pbx_gemv_impl.h"

using namespace pbx;

// ---------------------------------------------------------------------------
// Fused GEMV instantiations.  Name: pbx_dk_<type>_<shape>_<mode>
//   shape: w<R> (gemv_wide, R rows per workgroup) or s (gemv_small)
//   mode : qkv = RMSNorm prologue + store      add = plain + accumulate
//          gu  = RMSNorm + paired gate/up rows, stores silu(gate)*up
//          lmh = RMSNorm + argmax partials
// ---------------------------------------------------------------------------
#define DK_WIDE(T, TN, R, PRO, EPI, MN)                                             \
  extern "C" __global__ void __launch_bounds__(512) pbx_dk_##TN##_w##R##_##MN(GemvArgs a) { \
    gemv_wide<T, R, PRO, EPI>(a);                                                   \
  }
#define DK_SMALL(T, TN, P, PRO, EPI, MN)                                            \
  extern "C" __global__ void __launch_bounds__(256) pbx_dk_##TN##_s_##MN(GemvArgs a) { \
    gemv_small<T, P, PRO, EPI>(a);                                                  \
  }
#define DK_MODES_WIDE(T, TN, R)                     \
  DK_WIDE(T, TN, R, PRO_RMSNORM, EPI_STORE, qkv)    \
  DK_WIDE(T, TN, R, PRO_NONE, EPI_ADD, add)         \
  DK_WIDE(T, TN, R, PRO_RMSNORM, EPI_SWIGLU, gu)    \
  DK_WIDE(T, TN, R, PRO_RMSNORM, EPI_ARGMAX, lmh)
#define DK_MODES_SMALL(T, TN, P)                    \
  DK_SMALL(T, TN, P, PRO_RMSNORM, EPI_STORE, qkv)   \
  DK_SMALL(T, TN, P, PRO_NONE, EPI_ADD, add)        \
  DK_SMALL(T, TN, P, PRO_RMSNORM, EPI_SWIGLU, gu)   \
  DK_SMALL(T, TN, P, PRO_RMSNORM, EPI_ARGMAX, lmh)

DK_MODES_WIDE(PBX_Q4, q4, 4)
DK_MODES_WIDE(PBX_Q4, q4, 8)
DK_MODES_WIDE(PBX_Q4, q4, 16)
DK_MODES_SMALL(PBX_Q4, q4, 8)
DK_MODES_WIDE(PBX_Q8, q8, 4)
DK_MODES_WIDE(PBX_Q8, q8, 8)
DK_MODES_SMALL(PBX_Q8, q8, 4)
DK_MODES_WIDE(PBX_Q41, q41, 4)
DK_MODES_WIDE(PBX_Q41, q41, 8)
DK_MODES_WIDE(PBX_Q41, q41, 16)
DK_MODES_SMALL(PBX_Q41, q41, 8)
DK_MODES_WIDE(PBX_F16, f16, 4)
DK_MODES_WIDE(PBX_F16, f16, 8)
DK_MODES_SMALL(PBX_F16, f16, 4)
DK_MODES_WIDE(PBX_Q6K, q6k, 4)
DK_MODES_WIDE(PBX_Q6K, q6k, 8)
DK_MODES_SMALL(PBX_Q6K, q6k, 4)
// Integer-limb kernels (Q4_0 / Q8_0, 2048 <= K <= 8192): gate|up for both
// types, every decode GEMV for Q4_0.
// Name: pbx_dk_<type>_i<WV>x<RT>b<IB>_<mode>.
#define DK_INT(T, TN, WV, RT, IB, PRO, EPI, MN)                                            \
  extern "C" __global__ void __launch_bounds__(WV * 64)                                   \
      pbx_dk_##TN##_i##WV##x##RT##b##IB##_##MN(GemvArgs a) {                              \
    gemv_int<T, WV, RT, IB, PRO, EPI>(a);                                                 \
  }
#define DK_INT_GU(T, TN, WV, RT, IB) DK_INT(T, TN, WV, RT, IB, PRO_RMSNORM, EPI_SWIGLU, gu)
#define DK_INT_QKV(T, TN, WV, RT, IB) DK_INT(T, TN, WV, RT, IB, PRO_RMSNORM, EPI_STORE, qkv)
// q|k|v with RoPE and the cache append (EPI_ROPE): pbx_dk_<type>_i<WV>x<RT>b<IB>_qkvr
#define DK_INT_QKVR(T, TN, WV, RT, IB) DK_INT(T, TN, WV, RT, IB, PRO_RMSNORM, EPI_ROPE, qkvr)
#define DK_INT_ADD(T, TN, WV, RT, IB) DK_INT(T, TN, WV, RT, IB, PRO_NONE, EPI_ADD, add)
#define DK_INT_LMH(T, TN, WV, RT, IB) DK_INT(T, TN, WV, RT, IB, PRO_RMSNORM, EPI_ARGMAX, lmh)
// lm head with a tile loop per workgroup: pbx_dk_<type>_i<WV>x<RT>b<IB>l_lmh
#define DK_INT_LMHL(T, TN, WV, RT, IB)                                                    \
  extern "C" __global__ void __launch_bounds__(WV * 64)                                   \
      pbx_dk_##TN##_i##WV##x##RT##b##IB##l_lmh(GemvArgs a) {                              \
    gemv_int<T, WV, RT, IB, PRO_RMSNORM, EPI_ARGMAX, true>(a);                            \
  }
// Scheduled variants (pbx_gemv_impl.h): w<BW> = BW builder waves beside the
// WV row waves, p<PRE> = rows requested before the limb barrier.
// Name: pbx_dk_<type>_i<WV>x<RT>b<IB>[w<BW>][p<PRE>]_<mode>.
#define DK_INT_S(T, TN, WV, RT, IB, BW, PRE, SUF, PRO, EPI, MN)                               \
  extern "C" __global__ void __launch_bounds__((WV + BW) * 64)                            \
      pbx_dk_##TN##_i##WV##x##RT##b##IB##SUF##_##MN(GemvArgs a) {                         \
    gemv_int<T, WV, RT, IB, PRO, EPI, false, 1, BW, PRE>(a);                              \
  }
// 16-wave workgroups (at most 128 VGPRs a lane) only where the prologue
// wave's activation registers still fit: Q4_0 with one block per lane.
DK_INT_GU(PBX_Q4, q4, 8, 4, 1)
DK_INT_GU(PBX_Q4, q4, 16, 4, 1)
DK_INT_S(PBX_Q4, q4, 16, 4, 1, 0, 2, p2, PRO_RMSNORM, EPI_SWIGLU, gu)
// after pbx_attention_o_*: the input is x + the pending update
DK_INT_S(PBX_Q4, q4, 16, 4, 1, 0, 2, p2, PRO_RMSACC, EPI_SWIGLU, gua)
// the same with 8 builder waves beside 8 row waves of 8 rows (4 requested
// before the limb barrier): the default gate|up after the fused attention
DK_INT_S(PBX_Q4, q4, 8, 8, 1, 8, 4, w8p4, PRO_RMSACC, EPI_SWIGLU, gua)
DK_INT_GU(PBX_Q4, q4, 8, 4, 2)
DK_INT_GU(PBX_Q8, q8, 8, 4, 1)
DK_INT_GU(PBX_Q8, q8, 8, 4, 2)
// Q4_0 decode roles (measured on Llama-3.2-1B shapes): qkv 4 x 4, o and
// down 4 x 2, lm head 4 x 8 with the tile loop (4 x 16 at K = 4096); the
// others are tuning alternatives.
DK_INT_QKV(PBX_Q4, q4, 4, 4, 1)
DK_INT_QKVR(PBX_Q4, q4, 4, 4, 1)
DK_INT_QKV(PBX_Q4, q4, 4, 4, 2)
DK_INT_QKV(PBX_Q4, q4, 8, 2, 1)
DK_INT_ADD(PBX_Q4, q4, 4, 2, 1)
DK_INT_ADD(PBX_Q4, q4, 4, 2, 2)
DK_INT_ADD(PBX_Q4, q4, 4, 2, 4)
DK_INT_S(PBX_Q4, q4, 4, 2, 4, 8, 2, w8, PRO_NONE, EPI_ADD, add)
DK_INT_S(PBX_Q4, q4, 4, 2, 4, 8, 2, w8, PRO_NONE, EPI_ADDACC, adda)  // folds the update in
DK_INT_S(PBX_Q4, q4, 4, 2, 4, 4, 2, w4, PRO_NONE, EPI_ADDACC, adda)
DK_INT_S(PBX_Q4, q4, 4, 2, 4, 4, 2, w4, PRO_NONE, EPI_ADD, add)
DK_INT_ADD(PBX_Q4, q4, 4, 1, 1)
DK_INT_ADD(PBX_Q4, q4, 4, 1, 4)
DK_INT_LMH(PBX_Q4, q4, 4, 16, 1)
DK_INT_LMH(PBX_Q4, q4, 4, 16, 2)
DK_INT_LMH(PBX_Q4, q4, 4, 8, 1)
DK_INT_LMHL(PBX_Q4, q4, 4, 8, 1)
DK_INT_LMHL(PBX_Q4, q4, 4, 4, 1)
// Q6_K lm head (the output matrix of llama.cpp Q4_0 files), K = 2048, on
// the resident Q6_K layout and on the lane-packed copy
DK_INT_LMHL(PBX_Q6K, q6k, 4, 4, 1)
DK_INT_LMHL(PBX_Q6KP, q6kp, 4, 4, 1)

// Lane-packed copy (PBX_Q6KP layout, PBX_Q6KP_ROW bytes per 32-block) of a
// resident Q6_K matrix of N rows x B 32-blocks: one thread per (row, block)
// decodes the block's 32 codes from its super-block and writes them back
// in the lane-major byte order.  d stays in the matrix's scale plane.
extern "C" __global__ void __launch_bounds__(256)
pbx_pack_q6_k_lanes(const uint8_t *qs, uint8_t *dst, int N, int B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)N * B) return;
  const int n = (int)(i / B), b = (int)(i % B);
  const uint8_t *blk = qs + ((size_t)n * (B >> 3) + (b >> 3)) * PBX_Q6K_BYTES;
  const int half = (b >> 2) & 1, g = b & 3;
  const uint8_t *ql = blk + half * 64 + (g & 1) * 32, *qh = blk + 128 + half * 32;
  uint8_t code[32];
#pragma unroll
  for (int l = 0; l < 32; ++l)
    code[l] = (uint8_t)(((ql[l] >> (4 * (g >> 1))) & 15) | (((qh[l] >> (2 * g)) & 3) << 4));
  uint8_t *row = dst + (size_t)n * B * PBX_Q6KP_ROW;
  uint8_t *lo = row + (size_t)b * 16, *hi = row + (size_t)B * 16 + (size_t)b * 8;
#pragma unroll
  for (int j = 0; j < 16; ++j) lo[j] = (uint8_t)((code[j] & 15) | ((code[j + 16] & 15) << 4));
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      unsigned v = 0;
#pragma unroll
      for (int sf = 0; sf < 4; ++sf) v |= (unsigned)((code[16 * u + 4 * sf + t] >> 4) & 3) << (2 * sf);
      hi[4 * u + t] = (uint8_t)v;
    }
  const uint8_t *sc = blk + 192 + half * 8 + 2 * g;
  uint8_t *so = row + (size_t)B * 24 + (size_t)b * 2;
  so[0] = sc[0];
  so[1] = sc[1];
}

// Row-batched integer-limb GEMVs: up to MR activation rows against one pass
// over the weights (speculative verify, prompts of 4..MR tokens), args.rows
// valid.  Name: pbx_dk_<type>_i<WV>x<RT>b<IB>r<MR>[l]_<mode>; mode lmh here
// stores logit rows (no argmax).
#define DK_INT_ROWS(T, TN, WV, RT, IB, MR, LOOP, L, PRO, EPI, MN)                          \
  extern "C" __global__ void __launch_bounds__(WV * 64)                                   \
      pbx_dk_##TN##_i##WV##x##RT##b##IB##r##MR##L##_##MN(GemvArgs a) {                    \
    gemv_int<T, WV, RT, IB, PRO, EPI, LOOP, MR>(a);                                       \
  }
DK_INT_ROWS(PBX_Q4, q4, 8, 2, 1, 8, false, , PRO_RMSNORM, EPI_STORE, qkv)
DK_INT_ROWS(PBX_Q4, q4, 8, 1, 1, 8, false, , PRO_NONE, EPI_ADD, add)
DK_INT_ROWS(PBX_Q4, q4, 8, 1, 4, 5, false, , PRO_NONE, EPI_ADD, add)  // LDS: 5 rows x 24 KB

// Row-batched GEMVs on int8 MFMAs for 1..5 activation rows (gemv_mr):
// pbx_mr_q4_<RW>x<KS>b<IB>_<mode>, RW 16-row tiles x KS K slices a workgroup.
// One workgroup a CU is the plan (LDS), so a lane may hold as many
// registers as the wave count allows: the weight requests then never wait
// for registers that an earlier load still has to fill.  The verify uses
// q|k|v 1x8, o 1x8, gate|up 4x4 and the LM head 8x1; the other shapes are
// tuning options.
#define MR_K(RW, KS, IB, PRO, EPI, MN)                                                       \
  extern "C" __global__ void __launch_bounds__(RW * KS * 64)                                \
      __attribute__((amdgpu_waves_per_eu(1, 1)))                                             \
      pbx_mr_q4_##RW##x##KS##b##IB##_##MN(GemvArgs a) {                                      \
    gemv_mr<RW, KS, IB, PRO, EPI, 5>(a);                                                     \
  }
MR_K(1, 4, 1, PRO_RMSNORM, EPI_ROPE, qkvr)
MR_K(1, 4, 1, PRO_NONE, EPI_ADD, add)
MR_K(4, 1, 1, PRO_RMSNORM, EPI_SWIGLU, gu)
MR_K(4, 2, 1, PRO_RMSNORM, EPI_SWIGLU, gu)
MR_K(1, 8, 1, PRO_RMSNORM, EPI_ROPE, qkvr)
MR_K(1, 8, 1, PRO_NONE, EPI_ADD, add)
MR_K(4, 4, 1, PRO_RMSNORM, EPI_SWIGLU, gu)
MR_K(1, 16, 1, PRO_RMSNORM, EPI_ROPE, qkvr)
MR_K(1, 16, 1, PRO_NONE, EPI_ADD, add)
// the verify's LM head (RMSNorm + logits of every row): 8x1, several workgroups a CU
MR_K(8, 1, 1, PRO_RMSNORM, EPI_STORE, store)
MR_K(4, 2, 1, PRO_RMSNORM, EPI_STORE, store)
// down with the K blocks split over XS workgroups (grid y):
// pbx_mr_q4_<RW>x<KS>b<IB>s<XS>_add (the verify uses 4x4b4s8)
#define MR_KX(RW, KS, IB, XS, PRO, EPI, MN)                                                  \
  extern "C" __global__ void __launch_bounds__(RW * KS * 64)                                \
      __attribute__((amdgpu_waves_per_eu(1, 1)))                                             \
      pbx_mr_q4_##RW##x##KS##b##IB##s##XS##_##MN(GemvArgs a) {                               \
    gemv_mr<RW, KS, IB, PRO, EPI, 5, false, XS>(a);                                          \
  }
MR_KX(4, 1, 4, 8, PRO_NONE, EPI_ADD, add)
MR_KX(4, 2, 4, 8, PRO_NONE, EPI_ADD, add)
MR_KX(4, 4, 4, 8, PRO_NONE, EPI_ADD, add)

DK_MODES_WIDE(PBX_F32, f32, 2)
DK_MODES_WIDE(PBX_F32, f32, 4)
DK_MODES_SMALL(PBX_F32, f32, 2)
// f32 LM heads with K = 32 BT <= 512: pbx_dk_f32_t<BT>_lmh (8 lanes a row)
#define DK_TALL_F32(BT)                                                                     \
  extern "C" __global__ void __launch_bounds__(256) pbx_dk_f32_t##BT##_lmh(GemvArgs a) {    \
    gemv_tall_f32_lmh<BT, 2>(a);                                                           \
  }
DK_TALL_F32(8)
DK_TALL_F32(9)
DK_TALL_F32(12)
DK_TALL_F32(16)
// Q8_0 LM heads with K = 32 BT <= 768: pbx_dk_q8_t<BT>_lmh (8 lanes a row)
#define DK_TALL_Q8(BT)                                                                      \
  extern "C" __global__ void __launch_bounds__(256) pbx_dk_q8_t##BT##_lmh(GemvArgs a) {     \
    gemv_tall_q8_lmh<BT, 2>(a);                                                            \
  }
DK_TALL_Q8(8)
DK_TALL_Q8(9)
DK_TALL_Q8(12)
DK_TALL_Q8(16)
DK_TALL_Q8(18)
DK_TALL_Q8(24)

// ---------------------------------------------------------------------------
// Block reductions for 256-thread workgroups.
// ---------------------------------------------------------------------------
namespace {

__device__ __forceinline__ float block_reduce(float v, bool is_max, float *scratch) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = __shfl_xor(v, off, 64);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();  // scratch may still be read from a previous reduction
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
  for (int w = 1; w < nw; ++w) r = is_max ? fmaxf(r, scratch[w]) : r + scratch[w];
  return r;
}

}  // namespace

#define PBX_ATTN_MAX_SEQ 8192
#define PBX_ATTN_MAX_HD 256

struct AttnArgs {
  const float *qkv;    // [dim | kv_dim | kv_dim] of this token, before RoPE
  float *kcache;       // this layer: [max_seq][kv_dim]
  float *vcache;
  const float *rope;   // [max_seq][head_dim/2][cos, sin]
  float *out;          // [dim]
  const int *state;    // state[0] = position
  int n_heads, n_kv_heads, head_dim;
  float scale;         // 1/sqrt(head_dim)
  int max_seq;         // cache rows (pbx_attention_head_c)
  // pbx_attention_o_*: the layer's o projection (Q4_0 planes: dim rows of
  // dim / 32 blocks), the residual's pending update [dim] (2^-32 units) and
  // the residual row (set to NaN where a head's product is not finite)
  const uint8_t *oqs;
  const uint16_t *odsc;
  long long *oacc;
  float *ox;
  // pbx_qkvr_attn_o_*: the q|k|v rows published by the same launch's GEMV
  // workgroups ([qdim | kv_dim | kv_dim] cells, the epoch at [cell_n])
  const unsigned long long *cells;
  int cell_n, qdim;
  // pbx_qkvr_attn_o_*: the model's device status word (a wait that gives
  // up ORs PBX_DEV_WAIT_TIMEOUT into it), the poll limit (0: PBX_CELL_SPIN)
  // and a tag offset that only a test sets (the cells then never match)
  int *status;
  int spin, skew;
  // the small-model step (pbx_small_step_q8): the tag comes from *epoch
  // instead of cells[cell_n], and the head's output is published as cells
  // (tag << 32 | value bits) at ocells + h * head_dim instead of stored
  const unsigned long long *epoch;
  unsigned long long *ocells;
};

// One workgroup per query head (llama.js:258-301 / llama-streaming.js:543-573):
// rotate q and the new k (adjacent pairs, llama.js:163-190), append k and v
// at `pos` (the first query head of each KV group writes), scores over
// positions 0..pos, max-subtracted softmax, weighted sum of V.
// Loads are arranged for memory-level parallelism: a thread scores whole
// positions (head_dim/4 independent 16-B loads of one K row), and the V sum
// splits the head_dim/4 float4 columns x (256 / (head_dim/4)) position groups
// over the threads, four positions per iteration.
extern "C" __global__ void __launch_bounds__(256) pbx_attention_decode(AttnArgs a) {
  __shared__ float qr[PBX_ATTN_MAX_HD], kn[PBX_ATTN_MAX_HD], vn[PBX_ATTN_MAX_HD];
  __shared__ float sc[PBX_ATTN_MAX_SEQ];
  __shared__ float4 part[256];
  __shared__ float red[8];

  const int h = blockIdx.x, hd = a.head_dim;
  const int group = a.n_heads / a.n_kv_heads, kvh = h / group;
  const int kvdim = a.n_kv_heads * hd, dim = a.n_heads * hd;
  const int pos = a.state[0];
  const float *q = a.qkv + (size_t)h * hd;
  const float *k = a.qkv + dim + (size_t)kvh * hd;
  const float *v = a.qkv + dim + kvdim + (size_t)kvh * hd;
  const float *rp = a.rope + (size_t)pos * hd;

  for (int i = threadIdx.x; i < hd / 2; i += blockDim.x) {
    const float c = rp[2 * i], s = rp[2 * i + 1];
    const float q0 = q[2 * i], q1 = q[2 * i + 1];
    qr[2 * i] = q0 * c - q1 * s;
    qr[2 * i + 1] = q0 * s + q1 * c;
    const float k0 = k[2 * i], k1 = k[2 * i + 1];
    kn[2 * i] = k0 * c - k1 * s;
    kn[2 * i + 1] = k0 * s + k1 * c;
    vn[2 * i] = v[2 * i];
    vn[2 * i + 1] = v[2 * i + 1];
  }
  __syncthreads();
  float *krow = a.kcache + (size_t)kvh * hd;
  float *vrow = a.vcache + (size_t)kvh * hd;
  if (h % group == 0) {
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
      krow[(size_t)pos * kvdim + d] = kn[d];
      vrow[(size_t)pos * kvdim + d] = vn[d];
    }
  }

  // scores: positions < pos from the cache, position pos from LDS
  const int L = pos + 1;
  const int hd4 = hd / 4;
  for (int j = threadIdx.x; j < L; j += blockDim.x) {
    float dot = 0.f;
    if (j < pos) {
      const float4 *kr = reinterpret_cast<const float4 *>(krow + (size_t)j * kvdim);
      float d0 = 0.f, d1 = 0.f;
      for (int d4 = 0; d4 < hd4; d4 += 2) {
        const float4 t = kr[d4];
        d0 = fmaf(qr[4 * d4], t.x, d0);
        d0 = fmaf(qr[4 * d4 + 1], t.y, d0);
        d0 = fmaf(qr[4 * d4 + 2], t.z, d0);
        d0 = fmaf(qr[4 * d4 + 3], t.w, d0);
        if (d4 + 1 < hd4) {
          const float4 u = kr[d4 + 1];
          d1 = fmaf(qr[4 * d4 + 4], u.x, d1);
          d1 = fmaf(qr[4 * d4 + 5], u.y, d1);
          d1 = fmaf(qr[4 * d4 + 6], u.z, d1);
          d1 = fmaf(qr[4 * d4 + 7], u.w, d1);
        }
      }
      dot = d0 + d1;
    } else {
      for (int d = 0; d < hd; ++d) dot = fmaf(qr[d], kn[d], dot);
    }
    sc[j] = dot * a.scale;
  }
  // The first V rows this thread will need do not depend on the softmax:
  // issue their loads before the reductions so the latency overlaps.
  const int G = (int)blockDim.x / hd4;
  const int c = threadIdx.x % hd4, g = threadIdx.x / hd4;
  const float4 *vb = reinterpret_cast<const float4 *>(vrow) + c;
  const size_t stride4 = (size_t)kvdim / 4;
  const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 vp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // unconditional load from a clamped row (row 0 is always in the cache),
    // the zero selected after it: a conditional load becomes a flat load of
    // a selected address
    const int j = g + i * G;
    const bool ok = g < G && j < pos;
    const float4 t = vb[(size_t)(ok ? j : 0) * stride4];
    vp[i] = ok ? t : zero4;
  }
  __syncthreads();
  float m = -INFINITY;
  for (int j = threadIdx.x; j < L; j += blockDim.x) m = fmaxf(m, sc[j]);
  m = block_reduce(m, true, red);
  float sum = 0.f;
  for (int j = threadIdx.x; j < L; j += blockDim.x) {
    const float e = expf(sc[j] - m);
    sc[j] = e;
    sum += e;
  }
  sum = block_reduce(sum, false, red);
  for (int j = threadIdx.x; j < L; j += blockDim.x) sc[j] = sc[j] / sum;
  __syncthreads();

  // out[d] = sum_j p_j V[j][d]: thread = (float4 column c, position group g)
  float4 acc = zero4;
  if (g < G) {
    const float4 vnew = make_float4(vn[4 * c], vn[4 * c + 1], vn[4 * c + 2], vn[4 * c + 3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = g + i * G;
      if (j < L) {
        const float4 vv = j < pos ? vp[i] : vnew;
        const float p = sc[j];
        acc.x = fmaf(p, vv.x, acc.x); acc.y = fmaf(p, vv.y, acc.y);
        acc.z = fmaf(p, vv.z, acc.z); acc.w = fmaf(p, vv.w, acc.w);
      }
    }
    int j = g + 4 * G;
    for (; j + 3 * G < pos; j += 4 * G) {
      const float4 v0 = vb[(size_t)j * stride4];
      const float4 v1 = vb[(size_t)(j + G) * stride4];
      const float4 v2 = vb[(size_t)(j + 2 * G) * stride4];
      const float4 v3 = vb[(size_t)(j + 3 * G) * stride4];
      const float p0 = sc[j], p1 = sc[j + G], p2 = sc[j + 2 * G], p3 = sc[j + 3 * G];
      acc.x = fmaf(p0, v0.x, acc.x); acc.y = fmaf(p0, v0.y, acc.y);
      acc.z = fmaf(p0, v0.z, acc.z); acc.w = fmaf(p0, v0.w, acc.w);
      acc.x = fmaf(p1, v1.x, acc.x); acc.y = fmaf(p1, v1.y, acc.y);
      acc.z = fmaf(p1, v1.z, acc.z); acc.w = fmaf(p1, v1.w, acc.w);
      acc.x = fmaf(p2, v2.x, acc.x); acc.y = fmaf(p2, v2.y, acc.y);
      acc.z = fmaf(p2, v2.z, acc.z); acc.w = fmaf(p2, v2.w, acc.w);
      acc.x = fmaf(p3, v3.x, acc.x); acc.y = fmaf(p3, v3.y, acc.y);
      acc.z = fmaf(p3, v3.z, acc.z); acc.w = fmaf(p3, v3.w, acc.w);
    }
    for (; j < L; j += G) {
      const float4 t = vb[(size_t)(j < pos ? j : 0) * stride4];
      const float4 vv = j < pos ? t : vnew;
      const float p = sc[j];
      acc.x = fmaf(p, vv.x, acc.x); acc.y = fmaf(p, vv.y, acc.y);
      acc.z = fmaf(p, vv.z, acc.z); acc.w = fmaf(p, vv.w, acc.w);
    }
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x < hd4) {
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int gg = 0; gg < G; ++gg) {
      const float4 t = part[gg * hd4 + threadIdx.x];
      s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
    }
    reinterpret_cast<float4 *>(a.out + (size_t)h * hd)[threadIdx.x] = s;
  }
}

// ---------------------------------------------------------------------------
// Split-position attention (flash-decoding) for head_dim <= 128: grid
// (n_kv_heads, S); workgroup (g, s) serves the Gq = n_heads/n_kv_heads query
// heads of KV group g (one wave each) over positions [s*C, (s+1)*C) of
// 0..pos, C = ceil((pos+1)/S).  K/V tiles of up to 32 positions are staged
// once in LDS for all Gq heads; each wave keeps a running max / sum / weighted V sum
// (online softmax) and writes its partial; pbx_attention_combine then merges
// the S partials of every head:
//   out = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s,
// the softmax(q.K)V of llama.js:258-301 evaluated in S pieces.  The split
// holding `pos` rotates the new k, appends k and v to the cache and uses them
// from LDS; no other split reads position pos.
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// Flash decoding in one workgroup per query head (head_dim <= 64): the
// attention of llama.js:258-301 / llama-streaming.js:543-573 at batch 1.
// The positions read from the cache go in chunks of up to 512; a chunk of
// 32J positions (J = 1..16, as many as the context needs) gives every one
// of the eight waves 4J consecutive positions, so all waves carry the same
// short dependency chain whatever the context length.  Lane l holds dims
// 4(l%16)..4(l%16)+3 of q (which it rotates itself, llama.js:163-190) and
// of its row's positions base + 4j + l/16 of K and V, so each 16-byte load
// reads four whole 256-byte cache rows.  A position's dot is summed over
// the 16 lanes of its row by DPP, which leaves it in all 16 lanes: the row
// then runs its own online softmax (running max m, sum l and weighted V
// sum) with no cross-lane traffic at all.  Scores are kept in base-2 units
// (q is pre-scaled by scale * log2 e, so every exponential is one v_exp).
// The 32 row states and the new position (q . rotated new k, weight 1,
// value v) merge once through LDS, in one wave: lane i rescales state i by
// 2^(m_i - M) and every lane then sums its output dim over the states.
// The new position never comes from the cache: the group's first head
// appends k and v at pos after everything has been read, so no workgroup
// depends on another's write.
// ---------------------------------------------------------------------------
#define PBX_HA_MAX_HD 64
#define PBX_HA_WAVES 8
#define PBX_HA_STATES (PBX_HA_WAVES * 4 + 1)  // row states + the new position

// One chunk for the calling wave: positions base + 4j + ps (j < J) of the
// nc cached positions (loads clamped to the last one, scores past it masked
// to -inf), folded into the row's running (m, l, acc).
template <int J>
__device__ __forceinline__ void head_chunk(const float *kb, const float *vb, int kvdim, int dcol,
                                           int base, int nc, int ps, const float4 qq, float &m,
                                           float &l, float4 &acc) {
  float4 k[J], v[J];
#pragma unroll
  for (int j = 0; j < J; ++j)
    k[j] = *reinterpret_cast<const float4 *>(kb + (size_t)min(base + 4 * j + ps, nc - 1) * kvdim + dcol);
#pragma unroll
  for (int j = 0; j < J; ++j)
    v[j] = *reinterpret_cast<const float4 *>(vb + (size_t)min(base + 4 * j + ps, nc - 1) * kvdim + dcol);
  float s[J];
  float mc = -INFINITY;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const float d = wave_sum<8>(fmaf(qq.x, k[j].x, fmaf(qq.y, k[j].y, fmaf(qq.z, k[j].z, qq.w * k[j].w))));
    s[j] = base + 4 * j + ps < nc ? d : -INFINITY;
    mc = fmaxf(mc, s[j]);
  }
  const float mn = fmaxf(m, mc);
  const float ms = mn == -INFINITY ? 0.f : mn;  // a row with no position yet
  const float f = __builtin_amdgcn_exp2f(m - ms);
  float ls = 0.f;
  float4 a = make_float4(acc.x * f, acc.y * f, acc.z * f, acc.w * f);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const float p = __builtin_amdgcn_exp2f(s[j] - ms);
    ls += p;
    a.x = fmaf(p, v[j].x, a.x);
    a.y = fmaf(p, v[j].y, a.y);
    a.z = fmaf(p, v[j].z, a.z);
    a.w = fmaf(p, v[j].w, a.w);
  }
  l = fmaf(l, f, ls);
  acc = a;
  m = mn;
}

__device__ __forceinline__ void attention_head_body(const AttnArgs &a, const int pos) {
  __shared__ float st_m[PBX_HA_STATES], st_l[PBX_HA_STATES], st_e[PBX_HA_STATES];
  __shared__ __attribute__((aligned(16))) float st_acc[PBX_HA_STATES][PBX_HA_MAX_HD];
  const int h = blockIdx.x, hd = a.head_dim, hd4 = hd / 4;
  const int Gq = a.n_heads / a.n_kv_heads, g = h / Gq;
  const int dim = a.n_heads * hd, kvdim = a.n_kv_heads * hd;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int dg = lane & 15, ps = lane >> 4;  // dim group, row (position slot)
  const int dcol = 4 * min(dg, hd4 - 1);     // clamped for head_dim < 64
  float *kb = a.kcache + (size_t)g * hd, *vb = a.vcache + (size_t)g * hd;
  const int nc = pos;  // positions read from the cache

  // the lane's dims of q, the new k and v, and their RoPE pairs
  const float4 cs = *reinterpret_cast<const float4 *>(a.rope + (size_t)pos * hd + dcol);
  const float4 qv = *reinterpret_cast<const float4 *>(a.qkv + (size_t)h * hd + dcol);
  const float4 kv = *reinterpret_cast<const float4 *>(a.qkv + dim + (size_t)g * hd + dcol);
  const float4 vnw = *reinterpret_cast<const float4 *>(a.qkv + dim + kvdim + (size_t)g * hd + dcol);
  const float c = a.scale * 1.44269504088896340736f;  // scale * log2 e
  float4 qq = make_float4(qv.x * cs.x - qv.y * cs.y, qv.x * cs.y + qv.y * cs.x,
                          qv.z * cs.z - qv.w * cs.w, qv.z * cs.w + qv.w * cs.z);
  if (dg >= hd4) qq = make_float4(0.f, 0.f, 0.f, 0.f);  // repeats of the last dims
  qq = make_float4(qq.x * c, qq.y * c, qq.z * c, qq.w * c);

  float m = -INFINITY, l = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int c0 = 0; c0 < nc; c0 += PBX_HA_WAVES * 64) {
    const int J = min(16, (nc - c0 + 4 * PBX_HA_WAVES - 1) / (4 * PBX_HA_WAVES));
    const int base = c0 + 4 * w * J;
    if (base >= nc) continue;  // wave-uniform: nothing of this wave's
    switch (J) {
#define PBX_HEAD_CHUNK(n) \
  case n: head_chunk<n>(kb, vb, kvdim, dcol, base, nc, ps, qq, m, l, acc); break;
      PBX_HEAD_CHUNK(1) PBX_HEAD_CHUNK(2) PBX_HEAD_CHUNK(3) PBX_HEAD_CHUNK(4)
      PBX_HEAD_CHUNK(5) PBX_HEAD_CHUNK(6) PBX_HEAD_CHUNK(7) PBX_HEAD_CHUNK(8)
      PBX_HEAD_CHUNK(9) PBX_HEAD_CHUNK(10) PBX_HEAD_CHUNK(11) PBX_HEAD_CHUNK(12)
      PBX_HEAD_CHUNK(13) PBX_HEAD_CHUNK(14) PBX_HEAD_CHUNK(15) PBX_HEAD_CHUNK(16)
#undef PBX_HEAD_CHUNK
      default: break;
    }
  }

  // state 4w + ps: the row's; state 32: the new position
  const int si = 4 * w + ps;
  if (dg == 0) {
    st_m[si] = m;
    st_l[si] = l;
  }
  *reinterpret_cast<float4 *>(&st_acc[si][4 * dg]) = acc;
  const float4 knw = make_float4(kv.x * cs.x - kv.y * cs.y, kv.x * cs.y + kv.y * cs.x,
                                 kv.z * cs.z - kv.w * cs.w, kv.z * cs.w + kv.w * cs.z);
  if (w == 0 && ps == 0) {
    const float sn = wave_sum<8>(fmaf(qq.x, knw.x, fmaf(qq.y, knw.y, fmaf(qq.z, knw.z, qq.w * knw.w))));
    if (dg == 0) {
      st_m[PBX_HA_STATES - 1] = sn;
      st_l[PBX_HA_STATES - 1] = 1.f;
    }
    *reinterpret_cast<float4 *>(&st_acc[PBX_HA_STATES - 1][4 * dg]) = vnw;
  }
  lds_barrier();

  // merge: M is finite (the new position)
  if (w == 0) {
    constexpr int NS = PBX_HA_STATES;
    const float mi = lane < NS ? st_m[lane] : -INFINITY;
    const float li = lane < NS ? st_l[lane] : 0.f;
    const float M = wave_max(mi);
    const float e = __builtin_amdgcn_exp2f(mi - M);
    const float den = wave_sum(e * li);
    if (lane < NS) st_e[lane] = e;
    // the wave reads what its own lanes wrote: LDS keeps a wave's order
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float num = 0.f;
#pragma unroll
    for (int i = 0; i < NS; ++i) num = fmaf(st_e[i], st_acc[i][lane], num);
    if (lane < hd) a.out[(size_t)h * hd + lane] = num / den;
  }
  // the KV-cache append (the group's first head, lanes 0..hd/4-1), last
  if (h % Gq == 0 && tid < hd4) {
    *reinterpret_cast<float4 *>(kb + (size_t)pos * kvdim + dcol) = knw;
    *reinterpret_cast<float4 *>(vb + (size_t)pos * kvdim + dcol) = vnw;
  }
}

extern "C" __global__ void __launch_bounds__(PBX_HA_WAVES * 64) pbx_attention_head(AttnArgs a) {
  attention_head_body(a, a.state[0]);
}

// ---------------------------------------------------------------------------
// The same attention on a cache that already holds k and v at every position
// 0..pos and a q that is already rotated (the decode step's q|k|v GEMV with
// the RoPE epilogue, or pbx_rope_append_rows for a batch): no RoPE, no
// new-position state and no append here.  Positions are interleaved over
// the lanes: slot i holds positions 32i..32i+31, and the row ps of wave w
// takes position 32i + 4w + ps.  SPEC (decode): the first PBX_HC_SPEC slots
// are requested before the position is known (their rows do not depend on
// it), so the K/V transfer overlaps the load of the position; positions
// past it are masked, their V replaced by zeros (rows never written may
// hold anything).
// ---------------------------------------------------------------------------
#ifndef PBX_HC_SPEC
#define PBX_HC_SPEC 2
#endif

// Folds slots s0..s0+J-1 (K rows k, V rows v of the calling lane's row)
// into the row's running (m, l, acc); positions >= nc are masked.
template <int J, bool MASKV>
__device__ __forceinline__ void head_fold(const float4 (&k)[J], const float4 (&v)[J], int s0,
                                          int pl, int nc, const float4 qq, float &m, float &l,
                                          float4 &acc) {
  float s[J];
  float mc = -INFINITY;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const float d = wave_sum<8>(fmaf(qq.x, k[j].x, fmaf(qq.y, k[j].y, fmaf(qq.z, k[j].z, qq.w * k[j].w))));
    s[j] = 32 * (s0 + j) + pl < nc ? d : -INFINITY;
    mc = fmaxf(mc, s[j]);
  }
  const float mn = fmaxf(m, mc);
  const float ms = mn == -INFINITY ? 0.f : mn;  // a row with no position yet
  const float f = __builtin_amdgcn_exp2f(m - ms);
  float ls = 0.f;
  float4 a = make_float4(acc.x * f, acc.y * f, acc.z * f, acc.w * f);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const float p = __builtin_amdgcn_exp2f(s[j] - ms);
    float4 vv = v[j];
    if (MASKV && !(32 * (s0 + j) + pl < nc)) vv = make_float4(0.f, 0.f, 0.f, 0.f);
    ls += p;
    a.x = fmaf(p, vv.x, a.x);
    a.y = fmaf(p, vv.y, a.y);
    a.z = fmaf(p, vv.z, a.z);
    a.w = fmaf(p, vv.w, a.w);
  }
  l = fmaf(l, f, ls);
  acc = a;
  m = mn;
}

// Slots s0..s0+J-1 from the cache, rows clamped to nc - 1.
template <int J>
__device__ __forceinline__ void head_chunk_c(const float *kb, const float *vb, int kvdim, int dcol,
                                             int s0, int pl, int nc, const float4 qq, float &m,
                                             float &l, float4 &acc) {
  float4 k[J], v[J];
#pragma unroll
  for (int j = 0; j < J; ++j)
    k[j] = *reinterpret_cast<const float4 *>(kb + (size_t)min(32 * (s0 + j) + pl, nc - 1) * kvdim + dcol);
#pragma unroll
  for (int j = 0; j < J; ++j)
    v[j] = *reinterpret_cast<const float4 *>(vb + (size_t)min(32 * (s0 + j) + pl, nc - 1) * kvdim + dcol);
  head_fold<J, false>(k, v, s0, pl, nc, qq, m, l, acc);
}

// The same while the newest position nc - 1 is still being written: its
// cache row is requested like the others, and its k and v (kn, vn: the
// lane's dims) replace the loaded ones.  `ready` runs between the requests
// and the arithmetic (the fused kernel waits there for q, kn and vn).
template <int J, class Ready>
__device__ __forceinline__ void head_chunk_n(const float *kb, const float *vb, int kvdim, int dcol,
                                             int s0, int pl, int nc, Ready &&ready,
                                             const float4 &qq, const float4 &kn, const float4 &vn,
                                             float &m, float &l, float4 &acc) {
  float4 k[J], v[J];
#pragma unroll
  for (int j = 0; j < J; ++j)
    k[j] = *reinterpret_cast<const float4 *>(kb + (size_t)min(32 * (s0 + j) + pl, nc - 1) * kvdim + dcol);
#pragma unroll
  for (int j = 0; j < J; ++j)
    v[j] = *reinterpret_cast<const float4 *>(vb + (size_t)min(32 * (s0 + j) + pl, nc - 1) * kvdim + dcol);
  ready();
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (32 * (s0 + j) + pl == nc - 1) {
      k[j] = kn;
      v[j] = vn;
    }
  head_fold<J, false>(k, v, s0, pl, nc, qq, m, l, acc);
}

// Query head h and part s of workgroup column b (n_heads * parts columns).
// Workgroups go to the 8 XCDs round robin (column b on XCD b % 8 while the
// grid's x extent is a multiple of 8), each XCD with its own L2; with
// n_heads a multiple of 8, XCD x takes the consecutive heads x * n_heads / 8
// .. (all their parts), so the heads of a KV group share an L2 and their K/V
// rows come from HBM once instead of once per head; so do the 128-byte
// lines of the o projection that 4 adjacent heads read.
__device__ __forceinline__ void xcd_head(int b, int n_heads, int &h, int &s) {
  if (n_heads % 8) {
    h = b % n_heads;
    s = b / n_heads;
  } else {
    const int hpx = n_heads / 8, k = b / 8;
    h = (b % 8) * hpx + k % hpx;
    s = k / hpx;
  }
}

// IPT > 0 (pbx_attention_o_*, head_dim 64, Q4_0 o projection): after the
// head's attention output o_h, the workgroup multiplies it by the 64 columns
// of W_o it meets (blocks 2h and 2h + 1 of every row) for its 256 * IPT
// output rows [256 * IPT * s, ..) and adds each row's product into the
// residual's pending update as a 2^-32 fixed-point integer (64-bit atomics:
// integer addition is associative, so the sum of the n_heads products does
// not depend on the order the workgroups reach it).  The gate|up GEMV reads
// x + update as its input and the down GEMV folds the update into x.  A
// product that is not finite or not below 2^26 in magnitude (the sum of 32
// of them would leave the 64-bit range) sets the residual element to NaN.
// The weight bytes are requested right after the first K/V slots, so they
// stream in under the attention.
//
// FUSED (pbx_qkvr_attn_o_*, after the q|k|v GEMV workgroups of the same
// launch, workgroup column bid): q of the head and k, v of the newest
// position are still being computed.  The workgroup requests every cached
// position (the newest row too, whose loaded values it discards) and the o
// projection's bytes, then three waves wait for the 3 x 64 published cells
// (value bits tagged with the layer's epoch + 1; a cell that has not
// arrived after PBX_CELL_SPIN polls gives NaN) and pass them on through LDS.
#define PBX_CELL_SPIN (1 << 16)
// Bit of the model's status word set by a bounded wait that gave up; the
// host reads the word after the call's work and reports a timeout.
#define PBX_DEV_WAIT_TIMEOUT 1
// Polls a published cell until it carries `tag`.  After `spin` polls it
// gives up: the value is NaN and PBX_DEV_WAIT_TIMEOUT goes into the status
// word, so the host reports the call as failed instead of returning the
// NaN results.  One load at a time: three in flight, one every ~200 ns,
// made the decode step slower (353.3 against 349.0 us a token).
__device__ __forceinline__ float poll_cell(const unsigned long long *cp, unsigned tag, int spin,
                                           int *status) {
  unsigned long long v = __hip_atomic_load(cp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int it = 0; (unsigned)(v >> 32) != tag && it < spin; ++it) {
    __builtin_amdgcn_s_sleep(1);
    v = __hip_atomic_load(cp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if ((unsigned)(v >> 32) == tag) return __uint_as_float((unsigned)v);
  __hip_atomic_fetch_or(status, PBX_DEV_WAIT_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_nanf("");
}

// MAXJ: position slots a wave keeps in flight (16 slots of K and V are
// 128 registers a lane; a caller with less room passes fewer).
template <bool SPEC, int IPT = 0, bool FUSED = false, int MAXJ = 16>
__device__ __forceinline__ void attention_cached_body(const AttnArgs &a, const int pos_arg,
                                                      const int bid = -1) {
  static_assert(MAXJ >= 1 && MAXJ <= 16, "1..16 slots");
  static_assert(!FUSED || SPEC, "fused: device position");
  __shared__ float st_m[PBX_HA_WAVES], st_l[PBX_HA_WAVES];
  __shared__ __attribute__((aligned(16))) float st_acc[PBX_HA_WAVES][PBX_HA_MAX_HD];
  __shared__ float o_h[IPT > 0 ? 64 : 1], o_sum[2];
  __shared__ __attribute__((aligned(16))) float nrow[FUSED ? 3 : 1][FUSED ? 64 : 4];
  int h, part;
  xcd_head(bid < 0 ? (int)blockIdx.x : bid, a.n_heads, h, part);
  const int hd = a.head_dim, hd4 = hd / 4;
  const int Gq = a.n_heads / a.n_kv_heads, g = h / Gq;
  const int kvdim = a.n_kv_heads * hd;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int dg = lane & 15, ps = lane >> 4;  // dim group, row
  const int dcol = 4 * min(dg, hd4 - 1);     // clamped for head_dim < 64
  const int pl = 4 * w + ps;                 // the row's position in a slot
  const float *kb = a.kcache + (size_t)g * hd, *vb = a.vcache + (size_t)g * hd;

  float4 k0[SPEC ? PBX_HC_SPEC : 1], v0[SPEC ? PBX_HC_SPEC : 1];
  const int fpos = FUSED ? a.state[0] : 0;  // first: the requests below need it
  if constexpr (SPEC && !FUSED) {
#pragma unroll
    for (int j = 0; j < PBX_HC_SPEC; ++j)
      k0[j] = *reinterpret_cast<const float4 *>(kb + (size_t)min(32 * j + pl, a.max_seq - 1) * kvdim + dcol);
#pragma unroll
    for (int j = 0; j < PBX_HC_SPEC; ++j)
      v0[j] = *reinterpret_cast<const float4 *>(vb + (size_t)min(32 * j + pl, a.max_seq - 1) * kvdim + dcol);
  }
  const float4 qv = FUSED ? make_float4(0.f, 0.f, 0.f, 0.f)
                          : *reinterpret_cast<const float4 *>(a.qkv + (size_t)h * hd + dcol);
  // IPT > 0: the o projection's bytes of the workgroup's items (item j: row
  // 256 * IPT * part + j / 2, block 2h + j % 2; thread t holds items t + 512 i)
  uint4 wq[IPT > 0 ? IPT : 1];
  unsigned wd[IPT > 0 ? IPT : 1];
  if constexpr (IPT > 0) {
    const int B = a.n_heads * 2;
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      const int it = tid + PBX_HA_WAVES * 64 * i;
      const int row = 256 * IPT * part + (it >> 1), blk = 2 * h + (it & 1);
      wq[i] = ld_stream(a.oqs + ((size_t)row * B + blk) * 16);
      wd[i] = a.odsc[dsc_index(row, blk, B)];
    }
  }
  const int nc = (FUSED ? fpos : SPEC ? a.state[0] : pos_arg) + 1;  // positions 0..pos
  const float c = a.scale * 1.44269504088896340736f;  // scale * log2 e
  float4 qq = dg < hd4 ? make_float4(qv.x * c, qv.y * c, qv.z * c, qv.w * c)
                       : make_float4(0.f, 0.f, 0.f, 0.f);  // repeats of the last dims

  float m = -INFINITY, l = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  int s0 = 0;
  unsigned tag = 0;
  if constexpr (FUSED) {
    tag = cell_tag(a.epoch ? *a.epoch : a.cells[a.cell_n]) + (unsigned)a.skew;
    const int spin = a.spin > 0 ? a.spin : PBX_CELL_SPIN;
    float4 kn = make_float4(0.f, 0.f, 0.f, 0.f), vn = kn;
    auto ready = [&]() {
      if (w < 3) {  // wave 0: q of head h; 1, 2: k, v of KV head g
        nrow[w][lane] =
            lane < hd ? poll_cell(a.cells + (w == 0 ? h * hd : a.qdim + (w - 1) * kvdim + g * hd) +
                                      lane,
                                  tag, spin, a.status)
                      : 0.f;
      }
      lds_barrier();
      const float4 q4 = *reinterpret_cast<const float4 *>(&nrow[0][dcol]);
      // lanes past head_dim / 4 repeat the last dims: their q stays 0
      qq = dg < hd4 ? make_float4(q4.x * c, q4.y * c, q4.z * c, q4.w * c)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
      kn = *reinterpret_cast<const float4 *>(&nrow[1][dcol]);
      vn = *reinterpret_cast<const float4 *>(&nrow[2][dcol]);
    };
    auto none = [] {};
    bool first = true;
    while (32 * s0 < nc) {
      const int J = min(MAXJ, (nc - 32 * s0 + 31) / 32);
      switch (J) {
#define PBX_HEAD_CHUNK_N(n)                                                                \
  case n:                                                                                  \
    if constexpr (n <= MAXJ) {                                                             \
      if (first)                                                                           \
        head_chunk_n<n>(kb, vb, kvdim, dcol, s0, pl, nc, ready, qq, kn, vn, m, l, acc);    \
      else                                                                                 \
        head_chunk_n<n>(kb, vb, kvdim, dcol, s0, pl, nc, none, qq, kn, vn, m, l, acc);     \
    }                                                                                      \
    break;
        PBX_HEAD_CHUNK_N(1) PBX_HEAD_CHUNK_N(2) PBX_HEAD_CHUNK_N(3) PBX_HEAD_CHUNK_N(4)
        PBX_HEAD_CHUNK_N(5) PBX_HEAD_CHUNK_N(6) PBX_HEAD_CHUNK_N(7) PBX_HEAD_CHUNK_N(8)
        PBX_HEAD_CHUNK_N(9) PBX_HEAD_CHUNK_N(10) PBX_HEAD_CHUNK_N(11) PBX_HEAD_CHUNK_N(12)
        PBX_HEAD_CHUNK_N(13) PBX_HEAD_CHUNK_N(14) PBX_HEAD_CHUNK_N(15) PBX_HEAD_CHUNK_N(16)
#undef PBX_HEAD_CHUNK_N
        default: break;
      }
      first = false;
      s0 += J;
    }
  } else if constexpr (SPEC) {
    head_fold<PBX_HC_SPEC, true>(k0, v0, 0, pl, nc, qq, m, l, acc);
    s0 = PBX_HC_SPEC;
  }
  while (!FUSED && 32 * s0 < nc) {
    const int J = min(16, (nc - 32 * s0 + 31) / 32);
    switch (J) {
#define PBX_HEAD_CHUNK_C(n) \
  case n: head_chunk_c<n>(kb, vb, kvdim, dcol, s0, pl, nc, qq, m, l, acc); break;
      PBX_HEAD_CHUNK_C(1) PBX_HEAD_CHUNK_C(2) PBX_HEAD_CHUNK_C(3) PBX_HEAD_CHUNK_C(4)
      PBX_HEAD_CHUNK_C(5) PBX_HEAD_CHUNK_C(6) PBX_HEAD_CHUNK_C(7) PBX_HEAD_CHUNK_C(8)
      PBX_HEAD_CHUNK_C(9) PBX_HEAD_CHUNK_C(10) PBX_HEAD_CHUNK_C(11) PBX_HEAD_CHUNK_C(12)
      PBX_HEAD_CHUNK_C(13) PBX_HEAD_CHUNK_C(14) PBX_HEAD_CHUNK_C(15) PBX_HEAD_CHUNK_C(16)
#undef PBX_HEAD_CHUNK_C
      default: break;
    }
    s0 += J;
  }

  // merge in two levels: the wave's 4 rows (same dims, 16 lanes apart) in
  // registers, then the 8 wave states through LDS in one wave
  const float mw = pair_max<32>(pair_max<16>(m));  // finite for wave 0 (position 0)
  const float er = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mw);
  const float lw = pair_sum<32>(pair_sum<16>(l * er));
  const float4 aw = make_float4(pair_sum<32>(pair_sum<16>(acc.x * er)),
                                pair_sum<32>(pair_sum<16>(acc.y * er)),
                                pair_sum<32>(pair_sum<16>(acc.z * er)),
                                pair_sum<32>(pair_sum<16>(acc.w * er)));
  if (lane == 0) {
    st_m[w] = mw;
    st_l[w] = lw;
  }
  if (lane < 16) *reinterpret_cast<float4 *>(&st_acc[w][4 * dg]) = aw;
  lds_barrier();
  if (w == 0) {
    const float mi = lane < PBX_HA_WAVES ? st_m[lane] : -INFINITY;
    const float li = lane < PBX_HA_WAVES ? st_l[lane] : 0.f;
    const float M = wave_max<4>(mi);  // lanes 0..7 hold the states
    const float e = mi == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mi - M);
    const float den = wave_sum<4>(e * li);
    // readlane moves 32-bit integers: the floats travel as their bits
    float num = 0.f;
#pragma unroll
    for (int i = 0; i < PBX_HA_WAVES; ++i)
      num = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), i)), st_acc[i][lane], num);
    const float dn = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(den), 0));
    if constexpr (IPT == 0) {
      if (lane < hd) {
        const float o = num / dn;
        if (FUSED && a.ocells)  // published with the launch's own tag (no test offset)
          __hip_atomic_store(a.ocells + (size_t)h * hd + lane,
                             (unsigned long long)(tag - (unsigned)a.skew) << 32 | __float_as_uint(o),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          a.out[(size_t)h * hd + lane] = o;
      }
    } else {
      const float o = num / dn;  // head_dim 64: every lane
      o_h[lane] = o;
      const float sb = wave_sum<16>(o);  // lanes 0..31 and 32..63: the two blocks
      if ((lane & 31) == 0) o_sum[lane >> 5] = sb;
    }
  }
  if constexpr (IPT > 0) {
    lds_barrier();
    const int B = a.n_heads * 2;
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      const int it = tid + PBX_HA_WAVES * 64 * i;
      const int row = 256 * IPT * part + (it >> 1), hb = it & 1;
      const float *ov = o_h + 32 * hb;
      // sum of q * o over the block (q: codes 0..15), then (sum - 8 sum o) d
      const unsigned w4[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
      float t = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const unsigned lo = w4[j] & 0x0F0F0F0Fu, hi = (w4[j] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          t = fmaf((float)((lo >> (8 * k)) & 0xFFu), ov[4 * j + k], t);
          t = fmaf((float)((hi >> (8 * k)) & 0xFFu), ov[16 + 4 * j + k], t);
        }
      }
      float p = fmaf(-8.f, o_sum[hb], t) * f16_bits_to_f32(wd[i]);
      p += lane_partner<1>(p);  // the row's other block: the adjacent lane
      if (hb == 0) {
        if (fabsf(p) < 0x1p26f)
          atomicAdd(reinterpret_cast<unsigned long long *>(a.oacc) + row,
                    (unsigned long long)(long long)rintf(p * 0x1p32f));
        else
          a.ox[row] = __builtin_nanf("");
      }
    }
  }
}

// Decode step on the cache-complete layout (after pbx_dk_*_qkvr).
extern "C" __global__ void __launch_bounds__(PBX_HA_WAVES * 64) pbx_attention_head_c(AttnArgs a) {
  attention_cached_body<true>(a, 0);
}

// The same with the o projection fused (n_heads * dim / (256 * IPT)
// workgroups; head_dim 64, Q4_0 o projection, dim a multiple of 256 * IPT).
#define PBX_ATTN_O(IPT)                                                                     \
  extern "C" __global__ void __launch_bounds__(PBX_HA_WAVES * 64)                           \
      pbx_attention_o_c##IPT(AttnArgs a) {                                                  \
    attention_cached_body<true, IPT>(a, 0);                                                 \
  }
PBX_ATTN_O(1)
PBX_ATTN_O(2)
PBX_ATTN_O(4)
#undef PBX_ATTN_O

// RMSNorm + q|k|v GEMV + RoPE + cache append (workgroups 0..np-1: 4 row
// waves of RT rows and 4 builder waves, Q4_0, K = 32 * 64) and the attention
// with the o projection (workgroups np.., as pbx_attention_o_c<IPT>) in one
// launch: the GEMV publishes q, k and v row by row, and each attention
// workgroup waits only for the 192 values of its head.  The GEMV
// workgroups come first in the grid, so every XCD dispatches them before
// any attention workgroup and none of them waits: the grid always drains.
// np must be a multiple of 8 (the attention's XCD placement).  A CU holds
// one of these workgroups (their registers), so the attention workgroups
// request their K/V rows while the GEMV runs only where the grid fits the
// CUs: Llama-3.2-1B's 96 GEMV (RT 8) + 128 attention (IPT 2) workgroups.
#define PBX_QKVR_ATTN_O(WV, RT, BW, SUF, IPT)                                               \
  extern "C" __global__ void __launch_bounds__(PBX_HA_WAVES * 64)                           \
      pbx_qkvr_attn_o_r##RT##SUF##c##IPT(GemvArgs g, AttnArgs a, int np) {                  \
    static_assert(WV + BW == PBX_HA_WAVES, "one workgroup size");                           \
    if ((int)blockIdx.x < np)                                                               \
      gemv_int<PBX_Q4, WV, RT, 1, PRO_RMSNORM, EPI_ROPE, false, 1, BW, RT>(g);              \
    else                                                                                    \
      attention_cached_body<true, IPT, true>(a, 0, (int)blockIdx.x - np);                   \
  }
PBX_QKVR_ATTN_O(4, 4, 4, , 1)
PBX_QKVR_ATTN_O(4, 8, 4, , 2)
#undef PBX_QKVR_ATTN_O

// ---------------------------------------------------------------------------
// The FFN of a layer in one launch (llama-streaming.js:583-606: RMSNorm,
// w1/w3, silu(g) * u, w2 and the residual), for dim 2048, hidden 8192 and
// Q4_0 (Llama-3.2-1B): 256 workgroups of 8 builder and 8 row waves.
//
// Gate|up: workgroup j is the integer-limb GEMV of gate rows and up rows
// [32 j, 32 j + 32) (the builders form the limbs of RMSNorm(x + update), the
// row waves stream 8 rows each) and publishes its 32 outputs h as 64-bit
// cells, (epoch + 1) << 32 | value bits, by relaxed device-scope stores.
//
// Down: the 256 blocks of K are split into 8 slices of 32 blocks (1024
// values of h, the outputs of workgroups [32 s, 32 s + 32)), the 2048 rows
// into 32 tiles of 64; workgroup j takes slice s = j / 32 and tile j % 32,
// so the workgroups that produce a slice also consume it.  Builder thread t
// takes row 64 tile + t / 8 and the slice's blocks t % 8 + 8 i (i < 4): it
// requests those W_down bytes as soon as the limbs of gate|up are built (a
// row's 8 lanes read 128 contiguous bytes per block step).  Once the
// workgroup's own outputs are out, 256 builder threads poll 4 consecutive
// cells each until the slice's 1024 values carry the launch's tag, and turn
// them into the same per-block 22-bit fixed point as the GEMV inputs (three
// int8 limbs in LDS, read by 8 lanes at consecutive blocks: no bank
// conflicts); the dots are v_dot4 over the nibble codes (the first form,
// fp32 FMAs with 8 lanes a row at blocks 4 apart, spent 3.6 us in
// conflicted LDS reads).  The 8 slices of a row meet in the row's count
// cell (as the verify's split down projection: value biased by 2^51 in
// 2^-32 units plus a count, no fence, independent of the arrival order),
// and the add that completes the count stores x + update + sum into the
// next residual row and clears the cell.  The cell waits are bounded like
// the attention's: after `spin` polls the values are NaN and the status
// word is marked.
// ---------------------------------------------------------------------------
struct FfnArgs {
  const uint8_t *qs;          // W_down qs plane: 2048 rows of 256 blocks
  const uint16_t *dsc;        // its scale plane
  const float *x;             // the layer's residual row (the gate|up input)
  const long long *acc;       // its pending attention update (2^-32 units)
  unsigned long long *cell;   // [2048] count cells (zero between launches)
  float *xout;                // the next residual row
  unsigned long long *qepoch; // the layer's q|k|v epoch: advanced here
  int *status;
  int spin;
};

#define PBX_FFN_SLICES 8

extern "C" __global__ void __launch_bounds__(1024) pbx_ffn_q4_d2048_h8192(GemvArgs g, FfnArgs f) {
  constexpr int HID = 8192, KB = HID / 32, S = PBX_FFN_SLICES, SB = KB / S;  // 32 blocks a slice
  constexpr int TILES = 256 / S;  // 32 tiles of 64 rows
  // limb words 4q..4q+3 of slice block b at hl[L][q][b]; the block's exact
  // sum of codes and its 2^(e_b - 21) (NaN: a non-finite value)
  __shared__ int4 hl[3][2][SB];
  __shared__ int hsum[SB];
  __shared__ float hscale[SB];
  const int j = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int sl = j / TILES, tile = j % TILES;
  const bool bld = tid < 512;  // the builder waves (gemv_int's first BW = 8 waves)
  // no other workgroup reads the q|k|v epoch in this launch
  if (j == 0 && tid == 0) *f.qepoch = next_epoch(*f.qepoch);
  const unsigned tag = cell_tag(g.xcell[HID]);
  gemv_int<PBX_Q4, 8, 8, 1, PRO_RMSACC, EPI_SWIGLU, false, 1, 8, 4>(g);

  const int row = tile * 64 + ((tid & 511) >> 3), g8 = tid & 7, b0 = sl * SB + g8;
  uint4 wq[4];
  unsigned wd[4];
  float xr = 0.f;
  long long ar = 0;
  if (bld) {
    if (g8 == 0) {
      xr = f.x[row];
      ar = f.acc[row];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) wd[i] = f.dsc[dsc_index(row, b0 + 8 * i, KB)];
#pragma unroll
    for (int i = 0; i < 4; ++i) wq[i] = ld_stream(f.qs + ((size_t)row * KB + b0 + 8 * i) * 16);
  }
  lds_barrier();  // the workgroup's own gate|up outputs are published
  if (tid < 256) {
    // cells 4t .. 4t + 3 of the slice: float4 t % 8 of slice block t / 8
    const unsigned long long *cp = g.xcell + sl * SB * 32 + 4 * tid;
    unsigned long long v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = __hip_atomic_load(cp + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int spin = f.spin > 0 ? f.spin : PBX_CELL_SPIN;
    auto missing = [&]() {
      return (unsigned)(v[0] >> 32) != tag || (unsigned)(v[1] >> 32) != tag ||
             (unsigned)(v[2] >> 32) != tag || (unsigned)(v[3] >> 32) != tag;
    };
    for (int it = 0; missing() && it < spin; ++it) {
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if ((unsigned)(v[k] >> 32) != tag)
          v[k] = __hip_atomic_load(cp + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const bool ok = !missing();
    if (!ok)
      __hip_atomic_fetch_or(f.status, PBX_DEV_WAIT_TIMEOUT, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    const float4 p = ok ? make_float4(__uint_as_float((unsigned)v[0]), __uint_as_float((unsigned)v[1]),
                                      __uint_as_float((unsigned)v[2]), __uint_as_float((unsigned)v[3]))
                        : make_float4(NAN, NAN, NAN, NAN);
    // the block's fixed point, as the GEMV builders form it (no norm weight)
    const int qd = tid & 7, b = tid >> 3;
    float mx = fmaxf(fmaxf(fabsf(p.x), fabsf(p.y)), fmaxf(fabsf(p.z), fabsf(p.w)));
    float nf = fmaf(p.x, 0.f, fmaf(p.y, 0.f, fmaf(p.z, 0.f, p.w * 0.f)));
    mx = group_max<8>(mx);
    nf = group_sum<8>(nf);
    int e = 0;
    if (mx > 0.f && mx < INFINITY) frexpf(mx, &e);
    e = max(e, -100);
    int w0, w1, w2, sv;
    limb_words(p, ldexpf(1.f, 21 - e), w0, w1, w2, sv);
    const int st = group_isum<8>(sv);
    reinterpret_cast<int *>(&hl[0][qd >> 2][b])[qd & 3] = w0;
    reinterpret_cast<int *>(&hl[1][qd >> 2][b])[qd & 3] = w1;
    reinterpret_cast<int *>(&hl[2][qd >> 2][b])[qd & 3] = w2;
    if (qd == 0) {
      hsum[b] = st;
      hscale[b] = ldexpf(1.f, e - 21) + nf;
    }
  }
  lds_barrier();
  if (!bld) return;
  // the row's dots over its 4 blocks: exact int32 per limb, then the block's
  // scale and d (Q4_0's -8 offset: one 8 * sum(x_q) correction)
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int b = g8 + 8 * i;
    int xl[3][8];
#pragma unroll
    for (int L = 0; L < 3; ++L) {
      const int4 t0 = hl[L][0][b], t1 = hl[L][1][b];
      xl[L][0] = t0.x; xl[L][1] = t0.y; xl[L][2] = t0.z; xl[L][3] = t0.w;
      xl[L][4] = t1.x; xl[L][5] = t1.y; xl[L][6] = t1.z; xl[L][7] = t1.w;
    }
    const unsigned w4[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int lo = (int)(w4[k] & 0x0F0F0F0Fu), hi = (int)((w4[k] >> 4) & 0x0F0F0F0Fu);
      s0 = sdot4(lo, xl[0][k], s0); s0 = sdot4(hi, xl[0][4 + k], s0);
      s1 = sdot4(lo, xl[1][k], s1); s1 = sdot4(hi, xl[1][4 + k], s1);
      s2 = sdot4(lo, xl[2][k], s2); s2 = sdot4(hi, xl[2][4 + k], s2);
    }
    const float c0 = hscale[b];
    const float fb = fmaf((float)s2, 65536.f * c0,
                          fmaf((float)s1, 256.f * c0, fmaf((float)s0, c0, -8.f * (float)hsum[b] * c0)));
    acc = fmaf(fb, f16_bits_to_f32(wd[i]), acc);
  }
  acc = group_sum<8>(acc);
  if (g8 != 0) return;
  const bool bad = !(fabsf(acc) < 0x1p19f);
  const unsigned long long c =
      (1ull << 56) + (bad ? (1ull << 60) + (1ull << 51)
                          : (unsigned long long)((1ll << 51) + (long long)rintf(acc * 0x1p32f)));
  const unsigned long long t =
      __hip_atomic_fetch_add(f.cell + row, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + c;
  if (((t >> 56) & 15u) != (unsigned)S) return;
  __hip_atomic_store(f.cell + row, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const long long v = (long long)(t & ((1ull << 56) - 1)) - (long long)S * (1ll << 51);
  f.xout[row] = (t >> 60) ? __builtin_nanf("")
                          : (float)fma((double)v, 0x1p-32, (double)residual_acc(xr, ar));
}

// ---------------------------------------------------------------------------
// Small models: every layer of a decode step in one launch.
//
// For Q8_0 layers with dim <= 1024, hidden <= 4096 and head_dim <= 64
// (stories15M- and SmolLM2-135M-shaped models) each GEMV of a layer moves
// 0.1-2 MB: as separate launches every one of them sits on the ~5 us floor
// of a launch (dispatch, the activation round trip, one weight round trip),
// five a layer.  Here G workgroups of 512 threads (one a CU, all resident:
// the host keeps G <= the CU count) run all the layers of the step; the
// phases of a layer hand their outputs on as 64-bit cells, (tag << 32) |
// value bits, written by relaxed device-scope stores, and the next phase's
// workgroups poll the cells they need (bounded like the joined Llama
// launches: after `spin` polls a value is NaN and the status word is
// marked).  Layer l, workgroup j:
//   1. RMSNorm(x) (x: the step's row for l = 0, else the cells layer l - 1
//      published), the q|k|v rows [rq j, rq j + rq) (even: RoPE pairs), RoPE
//      of q and k, k and v appended at the position, all three published;
//   2. j < n_heads: the attention of query head j (the decode attention
//      body, which waits for q of its head and k, v of its KV head and reads
//      the older positions from the cache), o_h published;
//   3. the o projection's rows [ro j, ..) + the residual, published (x1);
//   4. RMSNorm(x1), the gate|up columns [rg j, ..): silu(g) * u published;
//   5. the down projection's rows [rd j, ..) + x1, published as layer
//      l + 1's input (the last layer stores it to x for the LM head).
// A task is one 32-block of one weight row (32 bytes of codes and its fp16
// scale): thread t takes tasks t, t + 512, ... of a GEMV; the partial dots
// meet in LDS, 8 threads a row.  The q|k|v bytes are requested when the
// layer starts, the others when the attention is done, so they arrive
// under the hand-offs.  Cells are written once a step with the step's tag,
// cell_tag(*epoch); the last workgroup to finish advances *epoch.
// ---------------------------------------------------------------------------
#define PBX_SM_T (PBX_HA_WAVES * 64)  // threads a workgroup (the attention body's)
#define PBX_SM_MAXD 1024
#define PBX_SM_MAXH 4096
#define PBX_SM_SQ 2  // task slots a thread: q|k|v, o, gate|up, down
#define PBX_SM_SO 1
#define PBX_SM_SG 4
#define PBX_SM_SD 2
#define PBX_SM_MAXR 256  // gate|up rows a workgroup (the host keeps them to this)
// GEMV activations in LDS: 32-value block b at 36 b (4 floats of padding):
// the 16-byte reads of 16 lanes at consecutive blocks then cover all 64
// banks once (at 32 floats a block they would meet in 8 of them).
#define PBX_SM_BLK 36
__device__ __forceinline__ int sm_pad(int i) { return (i >> 5) * PBX_SM_BLK + (i & 31); }

struct SmallLayer {
  const uint8_t *qkv_qs, *o_qs, *gu_qs, *d_qs;
  const uint16_t *qkv_d, *o_d, *gu_d, *d_d;
  const float *attn_norm, *ffn_norm;
};

struct SmallArgs {
  const SmallLayer *layers;   // [n_layers] in device memory
  AttnArgs at;                // layer 0's cache rows, the heads, state, status and poll limit
  long long layer_kv;         // cache floats of one layer
  unsigned long long *cells;  // layer l: cell_stride cells [q|k|v | o_h | x1 | h | next x]
  long long cell_stride;
  unsigned long long *epoch;  // the step's tag is cell_tag(*epoch)
  unsigned *done;             // workgroups finished (zero between launches)
  float *x;                   // layer 0's input; the last layer's output
  int n_layers, dim, hidden, qkv_rows;
  float eps;
  int rq, ro, rg, rd;         // rows (rg: gate|up columns) a workgroup
  int test_layer, skew;       // test hook: that layer's waits expect tag + skew
};

// One task slot: 32 codes, the block's scale bits (0 for an empty slot).
struct SmSlot {
  uint4 a, b;
  unsigned d;
};

// Task t of a GEMV with B blocks a row; row_of maps the workgroup's row
// index to the weight row.  Loads are unconditional (an empty slot reads
// the first task's bytes and gets a zero scale).
template <class RowOf>
__device__ __forceinline__ SmSlot sm_load(const uint8_t *qs, const uint16_t *dsc, int B, int ntask,
                                          int t, RowOf row_of) {
  const bool ok = t < ntask;
  const int tt = ok ? t : 0;
  const int r = row_of(tt / B), b = tt % B;
  SmSlot s;
  const uint8_t *src = qs + ((size_t)r * B + b) * 32;  // from the layer table: global loads
  s.a = ld_stream_g(src);
  s.b = ld_stream_g(src + 16);
  s.d = *gmem(dsc + dsc_index(r, b, B)) & (ok ? 0xFFFFu : 0u);
  return s;
}

// The slot's partial dot with the activations of its block (LDS).
__device__ __forceinline__ float sm_dot(const SmSlot &s, const float *xb) {
  float xr[32];
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const float4 f = *reinterpret_cast<const float4 *>(xb + 4 * v);
    xr[4 * v] = f.x;
    xr[4 * v + 1] = f.y;
    xr[4 * v + 2] = f.z;
    xr[4 * v + 3] = f.w;
  }
  float xs = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) xs += xr[i];
  return (dot_q8(s.a, s.b, xr) - 128.f * xs) * f16_bits_to_f32(s.d);
}

// Partial dots of S slots into part[task] (then a barrier); act holds the
// activations in the padded layout (sm_pad).
template <int S>
__device__ __forceinline__ void sm_dots(const SmSlot (&sl)[S], int B, int ntask, const float *act,
                                        float *part) {
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int t = (int)threadIdx.x + PBX_SM_T * i;
    if (t < ntask) part[t] = sm_dot(sl[i], act + (size_t)(t % B) * PBX_SM_BLK);
  }
  __syncthreads();
}

// Sum of row i's B partials (8 threads a row: threads 8i .. 8i + 7 all
// return it).
__device__ __forceinline__ float sm_row(const float *part, int i, int B) {
  const int sub = threadIdx.x & 7;
  float v = 0.f;
  for (int b = sub; b < B; b += 8) v += part[i * B + b];
  return group_sum<8>(v);
}

__device__ __forceinline__ void sm_publish(unsigned long long *cell, unsigned tag, float v) {
  __hip_atomic_store(cell, (unsigned long long)tag << 32 | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// The values of n published cells (n <= P * 512; thread t: cells t,
// t + 512, ...), polled until they carry tag; after `spin` polls the missing
// ones are NaN and the status word is marked.
template <int P>
__device__ __forceinline__ void sm_poll(const unsigned long long *cells, int n, unsigned tag,
                                        int spin, int *status, float (&val)[P]) {
  const int tid = threadIdx.x;
  unsigned long long v[P];
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const int i = tid + PBX_SM_T * k;
    v[k] = i < n ? __hip_atomic_load(cells + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                 : (unsigned long long)tag << 32;
  }
  auto missing = [&]() {
    bool r = false;
#pragma unroll
    for (int k = 0; k < P; ++k) r |= (unsigned)(v[k] >> 32) != tag;
    return r;
  };
  for (int it = 0; missing() && it < spin; ++it) {
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < P; ++k)
      if ((unsigned)(v[k] >> 32) != tag)
        v[k] = __hip_atomic_load(cells + tid + PBX_SM_T * k, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
  }
  if (missing())
    __hip_atomic_fetch_or(status, PBX_DEV_WAIT_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int k = 0; k < P; ++k)
    val[k] = (unsigned)(v[k] >> 32) == tag ? __uint_as_float((unsigned)v[k]) : __builtin_nanf("");
}

// val (thread t: elements t, t + 512, ...) into dst in the padded GEMV
// layout, between two barriers (dst may still be read before).
template <int P>
__device__ __forceinline__ void sm_store(const float (&val)[P], int n, float *dst) {
  __syncthreads();
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const int i = (int)threadIdx.x + PBX_SM_T * k;
    if (i < n) dst[sm_pad(i)] = val[k];
  }
  __syncthreads();
}

// A layer's residual row (val) into xin, x * w into act (padded) and
// 1 / rms(x) returned: llama.js's RMSNorm with 1/rms applied to the finished
// dot products (the dot is linear in x), so one pass and the barriers the
// store needs anyway.
__device__ __forceinline__ float sm_store_norm(const float (&val)[2], const float (&w)[2], int n,
                                               float eps, float *xin, float *act, float *red) {
  const int tid = threadIdx.x;
  __syncthreads();
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = tid + PBX_SM_T * k;
    if (i < n) {
      xin[i] = val[k];
      act[sm_pad(i)] = val[k] * w[k];
      ss = fmaf(val[k], val[k], ss);
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w8 = 0; w8 < PBX_HA_WAVES; ++w8) tot += red[w8];
  return 1.0f / sqrtf(tot / (float)n + eps);
}

extern "C" __global__ void __launch_bounds__(PBX_SM_T) pbx_small_step_q8(SmallArgs a) {
  __shared__ __attribute__((aligned(16))) float xin[PBX_SM_MAXD];  // the layer's residual row
  // a GEMV's activations (padded layout)
  __shared__ __attribute__((aligned(16))) float act[PBX_SM_MAXH / 32 * PBX_SM_BLK];
  __shared__ float part[PBX_SM_T * PBX_SM_SG];                      // partial dots
  __shared__ float red[PBX_HA_WAVES];
  const int j = blockIdx.x, tid = threadIdx.x;
  const int dim = a.dim, hidden = a.hidden, qr = a.qkv_rows;
  const int B = dim / 32, BH = hidden / 32;
  const int kvdim = a.at.n_kv_heads * a.at.head_dim, hd = a.at.head_dim;
  const int pos = a.at.state[0];
  const unsigned tag0 = cell_tag(*a.epoch);
  const int spin = a.at.spin > 0 ? a.at.spin : PBX_CELL_SPIN;
  int *status = a.at.status;
  // the workgroup's rows of each GEMV
  const int q0 = j * a.rq, nq = max(0, min(a.rq, qr - q0));
  const int o0 = j * a.ro, no = max(0, min(a.ro, dim - o0));
  const int c0 = j * a.rg, ng = max(0, min(a.rg, hidden - c0));
  const int d0 = j * a.rd, nd = max(0, min(a.rd, dim - d0));

  for (int l = 0; l < a.n_layers; ++l) {
    const SmallLayer L = a.layers[l];
    unsigned long long *cq = a.cells + (size_t)l * a.cell_stride;
    unsigned long long *co = cq + qr, *cx1 = co + dim, *ch = cx1 + dim, *cn = ch + hidden;
    // cells are published with the step's tag; the test hook's layer waits
    // for another one (its waits give up, every workgroup still finishes)
    const unsigned tag = tag0, want = tag0 + (l == a.test_layer ? (unsigned)a.skew : 0u);
    // 1. the q|k|v bytes and the norm weights, then the layer's input row
    SmSlot sq[PBX_SM_SQ];
#pragma unroll
    for (int i = 0; i < PBX_SM_SQ; ++i)
      sq[i] = sm_load(L.qkv_qs, L.qkv_d, B, nq * B, tid + PBX_SM_T * i,
                      [&](int r) { return min(q0 + r, qr - 1); });
    float nw[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) nw[k] = *gmem(L.attn_norm + min(tid + PBX_SM_T * k, dim - 1));
    float xv[2];
    if (l == 0) {
#pragma unroll
      for (int k = 0; k < 2; ++k) xv[k] = a.x[min(tid + PBX_SM_T * k, dim - 1)];
    } else {
      // the next-x cells of layer l - 1 (its cn)
      sm_poll(cq - a.cell_stride + qr + 2 * dim + hidden, dim, want, spin, status, xv);
    }
    float inv = sm_store_norm(xv, nw, dim, a.eps, xin, act, red);
    sm_dots(sq, B, nq * B, act, part);
    for (int i = tid >> 3; i < ((nq + 7) & ~7); i += PBX_SM_T / 8) {
      // rows 2i', 2i' + 1 sit in adjacent 8-thread groups of one wave
      const float v = (i < nq ? sm_row(part, i, B) : 0.f) * inv;
      const float pv = lane_partner<8>(v);
      if (i < nq && (tid & 7) == 0) {
        const int n = q0 + i;
        float o = v;
        if (n < dim + kvdim) {
          const float2 cs =
              *reinterpret_cast<const float2 *>(a.at.rope + (size_t)pos * hd + ((n & ~1) % hd));
          o = (n & 1) ? fmaf(pv, cs.y, v * cs.x) : fmaf(v, cs.x, -pv * cs.y);
          if (n >= dim) a.at.kcache[(size_t)l * a.layer_kv + (size_t)pos * kvdim + (n - dim)] = o;
        } else {
          a.at.vcache[(size_t)l * a.layer_kv + (size_t)pos * kvdim + (n - dim - kvdim)] = o;
        }
        sm_publish(cq + n, tag, o);
      }
    }
    // 2. attention of query head j
    if (j < a.at.n_heads) {
      AttnArgs at = a.at;
      at.kcache += (size_t)l * a.layer_kv;
      at.vcache += (size_t)l * a.layer_kv;
      at.cells = cq;
      at.qdim = dim;
      at.epoch = a.epoch;
      at.ocells = co;
      at.skew = l == a.test_layer ? a.skew : 0;
      attention_cached_body<true, 0, true, 8>(at, 0, j);
    }
    // 3. o projection + residual
    SmSlot so[PBX_SM_SO];
#pragma unroll
    for (int i = 0; i < PBX_SM_SO; ++i)
      so[i] = sm_load(L.o_qs, L.o_d, B, no * B, tid + PBX_SM_T * i,
                      [&](int r) { return min(o0 + r, dim - 1); });
    // gate|up rows interleaved: local row 2c is gate column c0 + c, 2c + 1 its up row
    SmSlot sg[PBX_SM_SG];
#pragma unroll
    for (int i = 0; i < PBX_SM_SG; ++i)
      sg[i] = sm_load(L.gu_qs, L.gu_d, B, 2 * ng * B, tid + PBX_SM_T * i, [&](int r) {
        return min((r & 1) ? hidden + c0 + (r >> 1) : c0 + (r >> 1), 2 * hidden - 1);
      });
    SmSlot sd[PBX_SM_SD];
#pragma unroll
    for (int i = 0; i < PBX_SM_SD; ++i)
      sd[i] = sm_load(L.d_qs, L.d_d, BH, nd * BH, tid + PBX_SM_T * i,
                      [&](int r) { return min(d0 + r, dim - 1); });
#pragma unroll
    for (int k = 0; k < 2; ++k) nw[k] = *gmem(L.ffn_norm + min(tid + PBX_SM_T * k, dim - 1));
    sm_poll(co, dim, want, spin, status, xv);
    sm_store(xv, dim, act);
    sm_dots(so, B, no * B, act, part);
    for (int i = tid >> 3; i < no; i += PBX_SM_T / 8) {
      const float v = sm_row(part, i, B);
      if ((tid & 7) == 0) sm_publish(cx1 + o0 + i, tag, xin[o0 + i] + v);
    }
    // 4. RMSNorm + gate|up + SwiGLU (gate and up rows in adjacent 8-thread groups)
    sm_poll(cx1, dim, want, spin, status, xv);
    inv = sm_store_norm(xv, nw, dim, a.eps, xin, act, red);
    sm_dots(sg, B, 2 * ng * B, act, part);
    for (int i = tid >> 3; i < ((2 * ng + 7) & ~7); i += PBX_SM_T / 8) {
      const float v = (i < 2 * ng ? sm_row(part, i, B) : 0.f) * inv;
      const float up = lane_partner<8>(v);
      if (i < 2 * ng && (i & 1) == 0 && (tid & 7) == 0)
        sm_publish(ch + c0 + (i >> 1), tag, silu(v) * up);
    }
    // 5. down + residual
    float hv[PBX_SM_MAXH / PBX_SM_T];
    sm_poll(ch, hidden, want, spin, status, hv);
    sm_store(hv, hidden, act);
    sm_dots(sd, BH, nd * BH, act, part);
    for (int i = tid >> 3; i < nd; i += PBX_SM_T / 8) {
      const float v = sm_row(part, i, BH);
      if ((tid & 7) == 0) {
        const float xo = xin[d0 + i] + v;
        if (l + 1 == a.n_layers) a.x[d0 + i] = xo;
        else sm_publish(cn + d0 + i, tag, xo);
      }
    }
  }
  // the last workgroup out advances the step's epoch (every workgroup read
  // it when it started)
  __syncthreads();
  if (tid == 0) {
    const unsigned d = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d + 1 == gridDim.x) {
      __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.epoch, next_epoch(*a.epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Batched rows (speculative verify, short batches; head_dim <= 64): workgroup
// (head, row t) at position start + t, after pbx_rope_append_rows has rotated
// q and k of every row and appended k and v; the arguments of
// pbx_attention_rows.
extern "C" __global__ void __launch_bounds__(PBX_HA_WAVES * 64)
pbx_attention_head_rows(const float *qkv, float *kcache, float *vcache, float *out, int start,
                        int n_heads, int n_kv_heads, int head_dim, float scale) {
  const int t = blockIdx.y, dim = n_heads * head_dim;
  AttnArgs a{qkv + (size_t)t * (dim + 2 * n_kv_heads * head_dim), kcache, vcache, nullptr,
             out + (size_t)t * dim, nullptr, n_heads, n_kv_heads, head_dim, scale, 0};
  attention_cached_body<false>(a, start + t);
}

#define PBX_SPLIT_TILE 32
#define PBX_SPLIT_MAX_HD 128
#define PBX_SPLIT_MAX_GQ 16

struct AttnSplitArgs {
  const float *qkv;    // [dim | kv_dim | kv_dim] of this token, before RoPE
  float *kcache;       // this layer: [max_seq][kv_dim]
  float *vcache;
  const float *rope;   // [max_seq][head_dim/2][cos, sin]
  float *out;          // [dim]
  const int *state;    // state[0] = position
  float *part;         // [n_heads][S][head_dim + 2]: m, l, acc[head_dim]
  int n_heads, n_kv_heads, head_dim, S;
  float scale;         // 1/sqrt(head_dim)
};

extern "C" __global__ void __launch_bounds__(1024) pbx_attention_split(AttnSplitArgs a) {
  __shared__ float qs[PBX_SPLIT_MAX_GQ][PBX_SPLIT_MAX_HD];
  __shared__ float kt[PBX_SPLIT_TILE][PBX_SPLIT_MAX_HD + 1];  // +1: conflict-free column reads
  __shared__ float vt[PBX_SPLIT_TILE][PBX_SPLIT_MAX_HD];
  __shared__ float knew[PBX_SPLIT_MAX_HD], vnew[PBX_SPLIT_MAX_HD];
  const int g = blockIdx.x, s = blockIdx.y;
  const int hd = a.head_dim, Gq = a.n_heads / a.n_kv_heads, half = hd / 2;
  const int dim = a.n_heads * hd, kvdim = a.n_kv_heads * hd;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int pos = a.state[0], L = pos + 1;
  const int C = (L + a.S - 1) / a.S;
  const int p0 = min(s * C, L), p1 = min(p0 + C, L);
  const bool has_pos = p0 <= pos && pos < p1;
  const float *rp = a.rope + (size_t)pos * hd;
  float *kbase = a.kcache + (size_t)g * hd, *vbase = a.vcache + (size_t)g * hd;
  const int hd4 = hd / 4;
  // A tile is T positions such that each thread loads at most TL float4 of
  // K and of V: T = min(32, TL * threads / (head_dim / 4)) >= 8.
  constexpr int TL = 4;
  const int T = min(PBX_SPLIT_TILE, TL * (int)blockDim.x / hd4);
  float4 kreg[TL], vreg[TL];
  // Unconditional loads (slots past the tile read position t0; the row at
  // pos is replaced by the new k, v in store_tile): a load under a branch
  // would wait at the branch's join.
  auto load_tile = [&](int t0, int n) {
#pragma unroll
    for (int r = 0; r < TL; ++r) {
      const int i = threadIdx.x + r * blockDim.x;
      const bool in = i < n * hd4;
      const int j = in ? i / hd4 : 0, c4 = in ? 4 * (i % hd4) : 0, p = min(t0 + j, pos);
      kreg[r] = *reinterpret_cast<const float4 *>(kbase + (size_t)p * kvdim + c4);
      vreg[r] = *reinterpret_cast<const float4 *>(vbase + (size_t)p * kvdim + c4);
    }
  };
  auto store_tile = [&](int t0, int n) {
#pragma unroll
    for (int r = 0; r < TL; ++r) {
      const int i = threadIdx.x + r * blockDim.x;
      const int j = i / hd4, c4 = 4 * (i % hd4), p = t0 + j;
      if (i < n * hd4) {
        float4 kv = kreg[r], vv = vreg[r];
        if (p == pos) {
          kv = make_float4(knew[c4], knew[c4 + 1], knew[c4 + 2], knew[c4 + 3]);
          vv = make_float4(vnew[c4], vnew[c4 + 1], vnew[c4 + 2], vnew[c4 + 3]);
        }
        kt[j][c4] = kv.x; kt[j][c4 + 1] = kv.y; kt[j][c4 + 2] = kv.z; kt[j][c4 + 3] = kv.w;
        *reinterpret_cast<float4 *>(&vt[j][c4]) = vv;
      }
    }
  };
  // q pairs of the group's heads: Gq * hd/2 <= 64 * Gq = threads, so one
  // pair per thread; the new k, v pair (hd/2 <= 64) likewise.  They are
  // needed first, so they are requested before the first K/V tile (a wave's
  // loads complete in issue order).  Unconditional loads from clamped
  // addresses, used only where valid.
  {
    const int i = threadIdx.x;
    const bool qok = i < Gq * half, kok = has_pos && i < half;
    const int hh = qok ? i / half : 0, k = i % half;
    const int ik = i < half ? i : 0;
    const float2 cs = *reinterpret_cast<const float2 *>(rp + 2 * k);
    const float2 qv = *reinterpret_cast<const float2 *>(a.qkv + (size_t)(g * Gq + hh) * hd + 2 * k);
    const float *kp = a.qkv + dim + (size_t)g * hd;
    const float2 kv = *reinterpret_cast<const float2 *>(kp + 2 * ik);
    const float2 vv = *reinterpret_cast<const float2 *>(kp + kvdim + 2 * ik);
    __builtin_amdgcn_sched_barrier(0);
    load_tile(p0, min(T, p1 - p0));  // an empty split reads row pos, unused
    __builtin_amdgcn_sched_barrier(0);
    if (qok) {
      qs[hh][2 * k] = qv.x * cs.x - qv.y * cs.y;
      qs[hh][2 * k + 1] = qv.x * cs.y + qv.y * cs.x;
    }
    if (kok) {
      knew[2 * i] = kv.x * cs.x - kv.y * cs.y;
      knew[2 * i + 1] = kv.x * cs.y + kv.y * cs.x;
      vnew[2 * i] = vv.x;
      vnew[2 * i + 1] = vv.y;
    }
  }
  lds_barrier();  // LDS hand-off only; K/V loads stay in flight
  if (has_pos)
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
      kbase[(size_t)pos * kvdim + d] = knew[d];
      vbase[(size_t)pos * kvdim + d] = vnew[d];
    }

  float m = -INFINITY, l = 0.f, acc0 = 0.f, acc1 = 0.f;
  for (int t0 = p0; t0 < p1; t0 += T) {
    const int n = min(T, p1 - t0);
    if (t0 != p0) load_tile(t0, n);
    store_tile(t0, n);
    lds_barrier();  // LDS hand-off only; K/V loads stay in flight
    if (w < Gq) {
      float sc = -INFINITY;
      if (lane < n) {
        float d0 = 0.f, d1 = 0.f;
        for (int d = 0; d < hd; d += 2) {
          d0 = fmaf(qs[w][d], kt[lane][d], d0);
          d1 = fmaf(qs[w][d + 1], kt[lane][d + 1], d1);
        }
        sc = (d0 + d1) * a.scale;
      }
      float mt = sc;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
      const float mn = fmaxf(m, mt);
      const float f = expf(m - mn);  // 0 on the first tile (m = -inf)
      const float p = lane < n ? expf(sc - mn) : 0.f;
      l = fmaf(l, f, wave_sum(p));
      acc0 *= f;
      acc1 *= f;
      for (int j = 0; j < n; ++j) {
        const float pj = __shfl(p, j, 64);
        if (lane < hd) acc0 = fmaf(pj, vt[j][lane], acc0);
        if (lane + 64 < hd) acc1 = fmaf(pj, vt[j][lane + 64], acc1);
      }
      m = mn;
    }
    lds_barrier();  // LDS hand-off only; K/V loads stay in flight
  }
  if (w < Gq) {
    float *pp = a.part + ((size_t)(g * Gq + w) * a.S + s) * (hd + 2);
    if (lane == 0) {
      pp[0] = m;
      pp[1] = l;
    }
    if (lane < hd) pp[2 + lane] = acc0;
    if (lane + 64 < hd) pp[2 + 64 + lane] = acc1;
  }
}

// One wave per query head: merge the S split partials (m_s, l_s, acc_s),
// S <= 64.  Lane t reads split t's (m, l); the weights e^(m_t - M) are then
// broadcast from lane t while every lane sums its head_dim column over the
// splits, 32 splits' loads in flight at a time.  Empty splits carry m = -inf
// and weigh e^-inf = 0; split 0 always holds position 0, so M is finite.
extern "C" __global__ void __launch_bounds__(64)
pbx_attention_combine(const float *part, float *out, int head_dim, int S) {
  const int h = blockIdx.x, lane = threadIdx.x, hd = head_dim, st = hd + 2;
  const float *pb = part + (size_t)h * S * st;
  // Every load of the first 32 splits is issued before any reduction, from
  // clamped addresses (split 0, column 0) and masked afterwards: loads under
  // a branch would each wait at the branch's join.
  const int c0 = lane < hd ? lane : 0, c1 = lane + 64 < hd ? lane + 64 : 0;
  float v0[32], v1[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int si = i < S ? i : 0;
    v0[i] = pb[(size_t)si * st + 2 + c0];
    v1[i] = pb[(size_t)si * st + 2 + c1];
  }
  const int sl = lane < S ? lane : 0;
  const float mraw = pb[(size_t)sl * st], lraw = pb[(size_t)sl * st + 1];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    v0[i] = (i < S && lane < hd) ? v0[i] : 0.f;
    v1[i] = (i < S && lane + 64 < hd) ? v1[i] : 0.f;
  }
  const float mt = lane < S ? mraw : -INFINITY;
  const float lt = lane < S ? lraw : 0.f;
  float mx = mt;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  const float wt = expf(mt - mx);
  const float lsum = wave_sum(wt * lt);
  float o0 = 0.f, o1 = 0.f;
  for (int t0 = 0; t0 < S; t0 += 32) {
    if (t0 > 0) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int si = t0 + i < S ? t0 + i : 0;
        v0[i] = pb[(size_t)si * st + 2 + c0];
        v1[i] = pb[(size_t)si * st + 2 + c1];
      }
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        v0[i] = (t0 + i < S && lane < hd) ? v0[i] : 0.f;
        v1[i] = (t0 + i < S && lane + 64 < hd) ? v1[i] : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float w = __shfl(wt, (t0 + i) & 63, 64);
      o0 = fmaf(w, v0[i], o0);
      o1 = fmaf(w, v1[i], o1);
    }
  }
  const float inv = 1.0f / lsum;
  if (lane < hd) out[(size_t)h * hd + lane] = o0 * inv;
  if (lane + 64 < hd) out[(size_t)h * hd + 64 + lane] = o1 * inv;
}

// ---------------------------------------------------------------------------
// Embedding row of the current token (llama.js:216-225), dequantised exactly
// from the resident token_embd planes (gguf.js:239-314) or copied (F32).
// ---------------------------------------------------------------------------
struct EmbedArgs {
  const uint8_t *qs;
  const uint16_t *dsc;
  float *x;
  const int *state;  // state[1] = token
  int type;          // PBX_Q4 / PBX_Q8 / PBX_F32 / PBX_Q41 / PBX_F16 / PBX_Q6K
  int dim, vocab;
  const uint16_t *msc;  // Q4_1 minima
};

extern "C" __global__ void __launch_bounds__(256) pbx_embed(EmbedArgs a) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.dim) return;
  int tok = a.state[1];
  if (tok < 0 || tok >= a.vocab) tok = 0;  // never read outside the table
  a.x[i] = row_value(a.qs, a.dsc, a.msc, a.type, tok, i, a.dim);
}

// ---------------------------------------------------------------------------
// Final argmax over the LM head's per-tile partial keys; records the token,
// appends it to the history and advances the position, then writes the
// token's embedding row into x for the next step (the step's first op), so
// a step ends where the next one begins.
// ---------------------------------------------------------------------------
struct ArgmaxArgs {
  const uint64_t *partials;
  int *state;
  int *hist;
  int n_partials;
  int hist_cap;
  EmbedArgs emb;  // the embedding table and x
  // the joined FFN's pending attention updates, cleared for the next step
  // (clr_n 64-bit words; null: none)
  long long *clr;
  int clr_n;
};

extern "C" __global__ void __launch_bounds__(1024) pbx_argmax_final(ArgmaxArgs a) {
  __shared__ uint64_t red[16];
  __shared__ int tok_sh;
  if (a.clr)
    for (int i = threadIdx.x; 2 * i < a.clr_n; i += blockDim.x)
      reinterpret_cast<i64x2_t *>(a.clr)[i] = i64x2_t{0, 0};
  uint64_t best = 0;
  for (int i = threadIdx.x; i < a.n_partials; i += blockDim.x) {
    const uint64_t k = a.partials[i];
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) best = red[w] > best ? red[w] : best;
    best = red[0] > best ? red[0] : best;
    const int tok = best ? (int)(0xFFFFFFFFu - (unsigned)(best & 0xFFFFFFFFu)) : 0;
    a.state[1] = tok;
    const int step = a.state[2];
    if (a.hist && step >= 0 && step < a.hist_cap) a.hist[step] = tok;
    a.state[2] = step + 1;
    a.state[0] = a.state[0] + 1;
    tok_sh = tok < 0 || tok >= a.emb.vocab ? 0 : tok;
  }
  __syncthreads();
  const int tok = tok_sh;
  for (int i = threadIdx.x; i < a.emb.dim; i += blockDim.x)
    a.emb.x[i] = row_value(a.emb.qs, a.emb.dsc, a.emb.msc, a.emb.type, tok, i, a.emb.dim);
}

// Zero cache positions [from, max_seq) of every layer (resetCache /
// rollbackCache, llama-streaming.js:828-862).  A kernel rather than a
// memset so it can sit inside a captured graph.
extern "C" __global__ void __launch_bounds__(256)
pbx_kv_fill(float *kcache, float *vcache, int64_t layer_stride, int64_t from_off, int64_t count,
            int n_layers) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count * n_layers) return;
  const int64_t l = i / count, o = from_off + i % count;
  kcache[l * layer_stride + o] = 0.f;
  vcache[l * layer_stride + o] = 0.f;
}

// Writes the token and position of a host-driven step into the device state.
extern "C" __global__ void pbx_set_state(int *state, int pos, int token, int step) {
  if (threadIdx.x == 0) {
    if (pos >= 0) state[0] = pos;
    if (token >= 0) state[1] = token;
    if (step >= 0) state[2] = step;
  }
}
