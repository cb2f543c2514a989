// pbx_prefill.hip -- row-batched kernels of the multi-token forward (prefill
// and speculative verify): llama.js:204-371 with seqLen = M > 1.  The matrix
// products run on the MFMA GEMM (pbx_gemm.hip); these kernels do the rest,
// one row (token) per workgroup unless noted.

#include "pbx_gemv_impl.h"

using namespace pbx;

#define PBX_ATTN_MAX_SEQ 8192
#define PBX_ATTN_MAX_HD 256

namespace {

__device__ __forceinline__ float block_reduce256(float v, bool is_max, float *scratch) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = __shfl_xor(v, off, 64);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
  for (int w = 1; w < nw; ++w) r = is_max ? fmaxf(r, scratch[w]) : r + scratch[w];
  return r;
}

}  // namespace

// Embedding rows (llama.js:216-225): x[t] = dequantised row tokens[t].
extern "C" __global__ void __launch_bounds__(256)
pbx_embed_rows(const uint8_t *qs, const uint16_t *dsc, const uint16_t *msc, const int *tokens,
               float *x, int type, int dim, int vocab) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= dim) return;
  int tok = tokens[t];
  if (tok < 0 || tok >= vocab) tok = 0;
  x[(size_t)t * dim + i] = row_value(qs, dsc, msc, type, tok, i, dim);
}

// The same for at most 16 rows with the tokens passed by value (a short
// verify: no memory read before the embedding).
struct TokRows {
  int t[16];
};
extern "C" __global__ void __launch_bounds__(256)
pbx_embed_rows_arg(const uint8_t *qs, const uint16_t *dsc, const uint16_t *msc, TokRows toks,
                   float *x, int type, int dim, int vocab) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= dim || t >= 16) return;
  int tok = toks.t[t];
  if (tok < 0 || tok >= vocab) tok = 0;
  x[(size_t)t * dim + i] = row_value(qs, dsc, msc, type, tok, i, dim);
}

// RMSNorm of rows (engine.js:429-449): out[t] = x[t] * (1/rms) * w.
extern "C" __global__ void __launch_bounds__(256)
pbx_rmsnorm_rows(const float *x, const float *w, float *out, int dim, float eps) {
  __shared__ float red[4];
  const float *xr = x + (size_t)blockIdx.x * dim;
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += blockDim.x) ss = fmaf(xr[i], xr[i], ss);
  ss = block_reduce256(ss, false, red);
  const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
  float *o = out + (size_t)blockIdx.x * dim;
  for (int i = threadIdx.x; i < dim; i += blockDim.x) o[i] = xr[i] * inv * w[i];
}

// RoPE of q and k in place for each row t (position start + t) and append of
// k, v to the cache (llama.js:159-191, 243-255).  qkv rows: [dim | kv | kv].
// With part, the rows are first the sum of the KS split-K partials
// [KS][rows][dim + 2 kv] of the q|k|v GEMM (summed in split order).  One pass
// over float4 columns: a column holds the pairs (2p, 2p + 1) and (2p + 2,
// 2p + 3) of one head (head_dim is a multiple of 4), rotated as the decode
// GEMV's epilogue rotates them (the same fused multiply-adds), then stored to
// the row and, for k and v, to the cache.
extern "C" __global__ void __launch_bounds__(256)
pbx_rope_append_rows(float *qkv, float *kcache, float *vcache, const float *rope, int start,
                     int n_heads, int n_kv_heads, int head_dim, const float *part, int KS) {
  const int t = blockIdx.x, pos = start + t;
  const int dim = n_heads * head_dim, kvdim = n_kv_heads * head_dim;
  const int rl = dim + 2 * kvdim;
  float4 *row = reinterpret_cast<float4 *>(qkv + (size_t)t * rl);
  const float *rp = rope + (size_t)pos * head_dim;
  // all partial loads of a column are issued before the sum (KS <= 8)
  const size_t stride4 = (size_t)gridDim.x * rl / 4;
  const float4 *pr = part ? reinterpret_cast<const float4 *>(part + (size_t)t * rl) : nullptr;
  for (int i = threadIdx.x; i < rl / 4; i += blockDim.x) {
    float4 v;
    if (pr) {
      float4 p[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) p[k] = k < KS ? pr[k * stride4 + i] : make_float4(0.f, 0.f, 0.f, 0.f);
      v = p[0];
#pragma unroll
      for (int k = 1; k < 8; ++k)
        if (k < KS) {
          v.x += p[k].x; v.y += p[k].y; v.z += p[k].z; v.w += p[k].w;
        }
    } else {
      v = row[i];
    }
    const int e = 4 * i;
    if (e < dim + kvdim) {
      // (x0, x1) -> (x0 c - x1 s, x0 s + x1 c) for both pairs of the column
      const int j = (e < dim ? e : e - dim) % head_dim;
      const float4 cs = *reinterpret_cast<const float4 *>(rp + j);  // c, s of pair j / 2, then j / 2 + 1
      v = make_float4(fmaf(v.x, cs.x, -v.y * cs.y), fmaf(v.x, cs.y, v.y * cs.x),
                      fmaf(v.z, cs.z, -v.w * cs.w), fmaf(v.z, cs.w, v.w * cs.z));
    }
    row[i] = v;
    if (e >= dim + kvdim)
      *reinterpret_cast<float4 *>(vcache + (size_t)pos * kvdim + (e - dim - kvdim)) = v;
    else if (e >= dim)
      *reinterpret_cast<float4 *>(kcache + (size_t)pos * kvdim + (e - dim)) = v;
  }
}

// Causal attention for query row t (position start + t) and head h over cache
// positions 0..start+t (llama.js:258-301: positions after the query are
// masked), after pbx_rope_append_rows has written every row's k, v.
extern "C" __global__ void __launch_bounds__(256)
pbx_attention_rows(const float *qkv, const float *kcache, const float *vcache, float *out,
                   int start, int n_heads, int n_kv_heads, int head_dim, float scale) {
  __shared__ float qr[PBX_ATTN_MAX_HD];
  __shared__ float sc[PBX_ATTN_MAX_SEQ];
  __shared__ float4 part[256];
  __shared__ float red[8];
  const int h = blockIdx.x, t = blockIdx.y, hd = head_dim;
  const int group = n_heads / n_kv_heads, kvh = h / group;
  const int dim = n_heads * hd, kvdim = n_kv_heads * hd;
  const int L = start + t + 1;
  const float *q = qkv + (size_t)t * (dim + 2 * kvdim) + (size_t)h * hd;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) qr[d] = q[d];
  __syncthreads();
  const float *krow = kcache + (size_t)kvh * hd;
  const float *vrow = vcache + (size_t)kvh * hd;
  const int hd4 = hd / 4;
  for (int j = threadIdx.x; j < L; j += blockDim.x) {
    const float4 *kr = reinterpret_cast<const float4 *>(krow + (size_t)j * kvdim);
    float dot = 0.f;
    for (int d4 = 0; d4 < hd4; ++d4) {
      const float4 k4 = kr[d4];
      dot = fmaf(qr[4 * d4], k4.x, dot);
      dot = fmaf(qr[4 * d4 + 1], k4.y, dot);
      dot = fmaf(qr[4 * d4 + 2], k4.z, dot);
      dot = fmaf(qr[4 * d4 + 3], k4.w, dot);
    }
    sc[j] = dot * scale;
  }
  __syncthreads();
  float m = -INFINITY;
  for (int j = threadIdx.x; j < L; j += blockDim.x) m = fmaxf(m, sc[j]);
  m = block_reduce256(m, true, red);
  float sum = 0.f;
  for (int j = threadIdx.x; j < L; j += blockDim.x) {
    const float e = expf(sc[j] - m);
    sc[j] = e;
    sum += e;
  }
  sum = block_reduce256(sum, false, red);
  for (int j = threadIdx.x; j < L; j += blockDim.x) sc[j] = sc[j] / sum;
  __syncthreads();
  const int G = (int)blockDim.x / hd4;
  const int c = threadIdx.x % hd4, g = threadIdx.x / hd4;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (g < G) {
    const float4 *vb = reinterpret_cast<const float4 *>(vrow) + c;
    const size_t stride4 = (size_t)kvdim / 4;
    for (int j = g; j < L; j += G) {
      const float4 vv = vb[(size_t)j * stride4];
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
      const float4 v = part[gg * hd4 + threadIdx.x];
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    reinterpret_cast<float4 *>(out + (size_t)t * dim + (size_t)h * hd)[threadIdx.x] = s;
  }
}

// Tiled causal attention for head_dim <= 64 (llama.js:258-301 over a block
// of query rows): workgroup (head h, query tile of 64 rows).  K and V of 64
// positions at a time are staged in LDS and shared by the 64 rows; thread
// (qi, j) holds rows 4qi..4qi+3 and, for the scores, keys 4j..4j+3 of the
// tile, for the weighted V sum dims 4j..4j+3.  A running max, sum and
// accumulator per row (online softmax) carry across key tiles; the rows of a
// thread group are reduced with lane shuffles (the 16 threads of a row group
// are consecutive lanes).  Keys after a row's own position are masked.
#define PF_QT 64
#define PF_KT 64
#define PF_LD 68  // padded row stride (floats): 16-byte rows, distinct banks

extern "C" __global__ void __launch_bounds__(256)
pbx_attention_tiled(const float *qkv, const float *kcache, const float *vcache, float *out,
                    int start, int n_rows, int n_heads, int n_kv_heads, int head_dim,
                    float scale) {
  __shared__ __attribute__((aligned(16))) float Qs[PF_QT * PF_LD];
  __shared__ __attribute__((aligned(16))) float Ks[PF_KT * PF_LD];
  __shared__ __attribute__((aligned(16))) float Vs[PF_KT * PF_LD];
  __shared__ float Ps[PF_QT * (PF_KT + 1)];
  const int h = blockIdx.x, t0 = blockIdx.y * PF_QT, hd = head_dim, hd4 = hd / 4;
  const int group = n_heads / n_kv_heads, kvh = h / group;
  const int dim = n_heads * hd, kvdim = n_kv_heads * hd, rs = dim + 2 * kvdim;
  const int tid = threadIdx.x, qi = tid >> 4, j = tid & 15;
  const int nq = min(PF_QT, n_rows - t0);
  // queries of this tile (already rotated by pbx_rope_append_rows)
  for (int i = tid; i < PF_QT * hd4; i += 256) {
    const int r = i / hd4, c = 4 * (i % hd4);
    const float4 v = r < nq ? *reinterpret_cast<const float4 *>(qkv + (size_t)(t0 + r) * rs + (size_t)h * hd + c)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    *reinterpret_cast<float4 *>(&Qs[r * PF_LD + c]) = v;
  }
  float m[4], l[4], acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[r][e] = 0.f;
  }
  const int last_key = start + t0 + nq - 1;  // the tile's last row sees keys 0..last_key
  const float *kb = kcache + (size_t)kvh * hd, *vb = vcache + (size_t)kvh * hd;
  for (int k0 = 0; k0 <= last_key; k0 += PF_KT) {
    const int nk = min(PF_KT, last_key + 1 - k0);
    __syncthreads();  // previous tile's K/V/P reads are done
    for (int i = tid; i < PF_KT * hd4; i += 256) {
      const int r = i / hd4, c = 4 * (i % hd4);
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      if (r < nk) {
        kv = *reinterpret_cast<const float4 *>(kb + (size_t)(k0 + r) * kvdim + c);
        vv = *reinterpret_cast<const float4 *>(vb + (size_t)(k0 + r) * kvdim + c);
      }
      *reinterpret_cast<float4 *>(&Ks[r * PF_LD + c]) = kv;
      *reinterpret_cast<float4 *>(&Vs[r * PF_LD + c]) = vv;
    }
    __syncthreads();
    float sc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) sc[r][c] = 0.f;
    for (int d = 0; d < hd; d += 4) {
      float4 q[4], k[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) q[r] = *reinterpret_cast<const float4 *>(&Qs[(4 * qi + r) * PF_LD + d]);
#pragma unroll
      for (int c = 0; c < 4; ++c) k[c] = *reinterpret_cast<const float4 *>(&Ks[(4 * j + c) * PF_LD + d]);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          sc[r][c] = fmaf(q[r].x, k[c].x, sc[r][c]);
          sc[r][c] = fmaf(q[r].y, k[c].y, sc[r][c]);
          sc[r][c] = fmaf(q[r].z, k[c].z, sc[r][c]);
          sc[r][c] = fmaf(q[r].w, k[c].w, sc[r][c]);
        }
    }
    float f[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qpos = start + t0 + 4 * qi + r;
      float mt = -INFINITY;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int kpos = k0 + 4 * j + c;
        sc[r][c] = (4 * j + c < nk && kpos <= qpos) ? sc[r][c] * scale : -INFINITY;
        mt = fmaxf(mt, sc[r][c]);
      }
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
      const float mn = fmaxf(m[r], mt);
      // rows past the end of the tile or with no visible key yet keep -inf
      f[r] = mn == -INFINITY ? 1.f : expf(m[r] - mn);
      float ps = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float p = mn == -INFINITY ? 0.f : expf(sc[r][c] - mn);
        Ps[(4 * qi + r) * (PF_KT + 1) + 4 * j + c] = p;
        ps += p;
      }
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) ps += __shfl_xor(ps, off, 64);
      l[r] = fmaf(l[r], f[r], ps);
      m[r] = mn;
    }
    __syncthreads();
    if (4 * j < hd) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[r][e] *= f[r];
      for (int k = 0; k < nk; ++k) {
        const float4 v = *reinterpret_cast<const float4 *>(&Vs[k * PF_LD + 4 * j]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = Ps[(4 * qi + r) * (PF_KT + 1) + k];
          acc[r][0] = fmaf(p, v.x, acc[r][0]);
          acc[r][1] = fmaf(p, v.y, acc[r][1]);
          acc[r][2] = fmaf(p, v.z, acc[r][2]);
          acc[r][3] = fmaf(p, v.w, acc[r][3]);
        }
      }
    }
  }
  if (4 * j < hd) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * qi + r;
      if (row < nq) {
        const float inv = 1.0f / l[r];
        *reinterpret_cast<float4 *>(out + (size_t)(t0 + row) * dim + (size_t)h * hd + 4 * j) =
            make_float4(acc[r][0] * inv, acc[r][1] * inv, acc[r][2] * inv, acc[r][3] * inv);
      }
    }
  }
}

// Causal attention on 32x32x16 MFMAs for head_dim 16..64 (a multiple of 16),
// the computation of pbx_attention_tiled.  Operand layout of
// v_mfma_f32_32x32x16_f16: A: lane l holds A[l%32][8*(l/32) + e]; B: lane l
// holds B[8*(l/32) + e][l%32]; D: lane l, register r holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32].  fp32 values enter as fp16 pairs
// hi = fp16(x), lo = fp16(x - hi), and a product of two such values is taken
// as hi*hi + hi*lo + lo*hi (three MFMAs; ~22 significant bits, the lo*lo term
// is below fp32 rounding of the sum).
// Workgroup: 64 query rows of one head, four waves; wave (qg, kh) holds the
// 32 queries qg and, of every 64-key stage in LDS, the 32 keys kh.  Scores
// are computed transposed, S^T = K . Q^T (A = keys x dims from LDS, B = the
// wave's queries' dims, kept in registers), so each lane owns one query:
// the softmax max and sum run over the lane's 16 registers and one exchange
// with lane l ^ 32.  The lane's probabilities are then exactly the B operand
// of O^T = V^T . P^T for 16 keys when the keys of a 16-key chunk are taken
// in the order {0-3, 8-11} (h = 0) and {4-7, 12-15} (h = 1), which V^T
// (stored [dim][key] in LDS) follows.  The two key halves of a query group
// merge their running max, sum and output through LDS at the end.
#define FA_KT 64           // keys per LDS stage
#define FA_KP (64 + 8)     // halves per K row (dims)
// halves per V^T row (keys): the stage writes rows 4 apart from 16 threads,
// which a 72-half row puts on 4 bank groups and a 68-half row on 8 (still
// 8-byte aligned for the operand reads, which stay conflict-free)
#define FA_VP (64 + 4)

// hi = fp16(x), lo = fp16(x - hi), assigned to H and L (vector elements allowed)
#define SPLIT_F16(x, H, L)                       \
  do {                                           \
    const float x_ = (x);                        \
    const _Float16 h_ = (_Float16)x_;            \
    (H) = h_;                                    \
    (L) = (_Float16)(x_ - (float)h_);            \
  } while (0)

// KG > 1: KG groups of four waves share the workgroup's 64 queries and take
// the 64-key stages round robin (group g: stages g, g + KG, ...), each with
// its own LDS stage, so the longest tile (the last one: every key) runs in
// 1/KG of the stage steps; the 2 KG states per query (key halves x groups)
// merge through LDS at the end.  All groups run the same number of steps
// (a group past the last key only keeps the barriers).
template <int KG>
__device__ __forceinline__ void attention_mfma_body(const float *qkv, const float *kcache,
                                                    const float *vcache, float *out, int start,
                                                    int n_rows, int n_heads, int n_kv_heads,
                                                    int head_dim, float scale) {
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  typedef _Float16 half2t __attribute__((ext_vector_type(2)));
  typedef _Float16 half4t __attribute__((ext_vector_type(4)));
  typedef float floatx16 __attribute__((ext_vector_type(16)));
  // each group's stage: K hi, K lo ([key][dim]), V^T hi, V^T lo ([dim][key]);
  // one array, so the merge below may reuse all of it
  __shared__ __attribute__((aligned(16))) _Float16 KVsh[KG][4][FA_KT * FA_KP];
  static_assert(64 * FA_VP <= FA_KT * FA_KP, "the V^T stage fits a K stage's space");
  static_assert(2 * (2 * KG - 1) * 64 * 34 * 4 <= KG * 4 * FA_KT * FA_KP * 2, "merge fits the stages");
  const int h = blockIdx.x, t0 = blockIdx.y * 64, hd = head_dim, hd4 = hd / 4, nc = hd / 16;
  const int group = n_heads / n_kv_heads, kvh = h / group;
  const int dim = n_heads * hd, kvdim = n_kv_heads * hd, rs = dim + 2 * kvdim;
  const int tid = threadIdx.x & 255, lane = tid & 63, wave = tid >> 6;
  const int kg = KG > 1 ? (int)(threadIdx.x >> 8) : 0;  // the wave's key group
  _Float16 *Kh = KVsh[kg][0], *Kl = KVsh[kg][1], *Vh = KVsh[kg][2], *Vl = KVsh[kg][3];
  const int qg = wave & 1, kh = wave >> 1, lq = lane & 31, hh = lane >> 5;
  const int nq = min(64, n_rows - t0);
  const int qrow = 32 * qg + lq;  // this lane's query within the tile
  const int qpos = start + t0 + qrow;
  const floatx16 zero16 = {};

  // the lane's query dims 16c + 8hh .. +7 (scaled), as hi / lo B operands
  half8 Qh[4], Ql[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (c < nc) {
      float qv[8];
      if (qrow < nq) {
        const float *q = qkv + (size_t)(t0 + qrow) * rs + (size_t)h * hd + 16 * c + 8 * hh;
        const float4 a = *reinterpret_cast<const float4 *>(q);
        const float4 b = *reinterpret_cast<const float4 *>(q + 4);
        qv[0] = a.x; qv[1] = a.y; qv[2] = a.z; qv[3] = a.w;
        qv[4] = b.x; qv[5] = b.y; qv[6] = b.z; qv[7] = b.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) SPLIT_F16(qv[e] * scale, Qh[c][e], Ql[c][e]);
    }
  }

  float m_run = -INFINITY, l_run = 0.f;
  floatx16 acc[2] = {zero16, zero16};  // O^T, dims 32 dt + 8 (r/4) + 4 hh + r%4
  const int last_key = start + t0 + nq - 1;
  const float *kb = kcache + (size_t)kvh * hd, *vb = vcache + (size_t)kvh * hd;
  // the next stage's K and V rows are loaded into registers while the current
  // stage is multiplied: K item i (< 4) = key (tid + 256 i) / hd4, float4
  // column (tid + 256 i) % hd4; V item i = keys 2 p, 2 p + 1 of item
  // p = (tid + 256 i) / hd4 (< 32 key pairs), same column
  float4 kreg[4], vreg0[2], vreg1[2];
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  // Loads are unconditional from clamped addresses (key k0 is always in
  // the cache) and nothing reads the registers until the stage is stored
  // to LDS, where the keys past the stage's end become zeros: a condition
  // on the load (or a select right after it) makes the compiler wait for
  // the data at once, and the next stage's loads no longer overlap this
  // stage's arithmetic.
  auto kv_ok = [&](int k0, int i, int which) -> bool {  // which: 0 K, 1 V row kp, 2 V row kp + 1
    const int nk = min(FA_KT, last_key + 1 - k0);
    const int it = tid + 256 * i;
    if (which == 0) return it < FA_KT * hd4 && it / hd4 < nk;
    const int kp = 2 * (it / hd4) + (which - 1);
    return it < (FA_KT / 2) * hd4 && kp < nk;
  };
  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int it = tid + 256 * i, key = it / hd4, c4 = 4 * (it % hd4);
      const bool ok = kv_ok(k0, i, 0);
      kreg[i] =
          *reinterpret_cast<const float4 *>(kb + (size_t)(k0 + (ok ? key : 0)) * kvdim + (ok ? c4 : 0));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int it = tid + 256 * i, kp = 2 * (it / hd4), c4 = 4 * (it % hd4);
      const bool ok0 = kv_ok(k0, i, 1), ok1 = kv_ok(k0, i, 2);
      vreg0[i] =
          *reinterpret_cast<const float4 *>(vb + (size_t)(k0 + (ok0 ? kp : 0)) * kvdim + (ok0 ? c4 : 0));
      vreg1[i] =
          *reinterpret_cast<const float4 *>(vb + (size_t)(k0 + (ok1 ? kp + 1 : 0)) * kvdim + (ok1 ? c4 : 0));
    }
  };
  if (kg * FA_KT <= last_key) load_stage(kg * FA_KT);
  for (int step = 0; KG * FA_KT * step <= last_key; ++step) {
    const int k0 = (KG * step + kg) * FA_KT;  // this group's stage
    const bool live = k0 <= last_key;
    __syncthreads();  // the previous stage's reads are done
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int it = tid + 256 * i, key = it / hd4, c4 = 4 * (it % hd4);
      if (live && it < FA_KT * hd4) {
        const float4 v = kv_ok(k0, i, 0) ? kreg[i] : z4;
        half4t hv, lv;
        SPLIT_F16(v.x, hv[0], lv[0]);
        SPLIT_F16(v.y, hv[1], lv[1]);
        SPLIT_F16(v.z, hv[2], lv[2]);
        SPLIT_F16(v.w, hv[3], lv[3]);
        *reinterpret_cast<half4t *>(&Kh[key * FA_KP + c4]) = hv;
        *reinterpret_cast<half4t *>(&Kl[key * FA_KP + c4]) = lv;
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int it = tid + 256 * i, kp = 2 * (it / hd4), c4 = 4 * (it % hd4);
      if (live && it < (FA_KT / 2) * hd4) {
        const float4 v0 = kv_ok(k0, i, 1) ? vreg0[i] : z4, v1 = kv_ok(k0, i, 2) ? vreg1[i] : z4;
#define FA_PUTV(e, x0, x1)                                                  \
  do {                                                                      \
    half2t hv_, lv_;                                                        \
    SPLIT_F16(x0, hv_[0], lv_[0]);                                          \
    SPLIT_F16(x1, hv_[1], lv_[1]);                                          \
    *reinterpret_cast<half2t *>(&Vh[(c4 + (e)) * FA_VP + kp]) = hv_;        \
    *reinterpret_cast<half2t *>(&Vl[(c4 + (e)) * FA_VP + kp]) = lv_;        \
  } while (0)
        FA_PUTV(0, v0.x, v1.x);
        FA_PUTV(1, v0.y, v1.y);
        FA_PUTV(2, v0.z, v1.z);
        FA_PUTV(3, v0.w, v1.w);
#undef FA_PUTV
      }
    }
    __syncthreads();
    if (k0 + KG * FA_KT <= last_key) load_stage(k0 + KG * FA_KT);
    if (!live) continue;

    // S^T for this wave's 32 keys (rows) x 32 queries (columns)
    const int kr = 32 * kh + lq;  // A row: key kr of the stage
    floatx16 s = zero16;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c < nc) {
        const half8 ah = *reinterpret_cast<const half8 *>(&Kh[kr * FA_KP + 16 * c + 8 * hh]);
        const half8 al = *reinterpret_cast<const half8 *>(&Kl[kr * FA_KP + 16 * c + 8 * hh]);
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, Qh[c], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, Ql[c], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, Qh[c], s, 0, 0, 0);
      }
    }
    // mask, online softmax for the lane's query over its 16 keys and lane ^ 32's
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kpos = k0 + 32 * kh + 8 * (r >> 2) + 4 * hh + (r & 3);
      if (kpos > qpos || kpos > last_key) s[r] = -INFINITY;
      mt = fmaxf(mt, s[r]);
    }
    mt = pair_max<32>(mt);
    const float mn = fmaxf(m_run, mt);
    const float f = mn == -INFINITY ? 1.f : expf(m_run - mn);
    float ps = 0.f;
    half8 Ph[2], Pl[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = mn == -INFINITY ? 0.f : expf(s[r] - mn);
      ps += pr;
      SPLIT_F16(pr, Ph[r >> 3][r & 7], Pl[r >> 3][r & 7]);
    }
    ps = pair_sum<32>(ps);
    l_run = fmaf(l_run, f, ps);
    m_run = mn;
    // O^T += V^T . P^T over the 32 keys (two chunks of 16)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      if (32 * dt < hd) {
        acc[dt] *= f;
        const int vr = (32 * dt + lq) * FA_VP + 32 * kh + 4 * hh;  // V^T row (dim), key base
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          half8 ah, al;
          const half4t h0 = *reinterpret_cast<const half4t *>(&Vh[vr + 16 * cc]);
          const half4t h1 = *reinterpret_cast<const half4t *>(&Vh[vr + 16 * cc + 8]);
          const half4t l0 = *reinterpret_cast<const half4t *>(&Vl[vr + 16 * cc]);
          const half4t l1 = *reinterpret_cast<const half4t *>(&Vl[vr + 16 * cc + 8]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            ah[e] = h0[e]; ah[4 + e] = h1[e];
            al[e] = l0[e]; al[4 + e] = l1[e];
          }
          acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, Ph[cc], acc[dt], 0, 0, 0);
          acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, Pl[cc], acc[dt], 0, 0, 0);
          acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, Ph[cc], acc[dt], 0, 0, 0);
        }
      }
    }
  }

  // merge the 2 KG key slices of each query group (key halves x groups):
  // every slice but (kh 0, group 0) hands its state over through LDS
  __syncthreads();
  float *mg = reinterpret_cast<float *>(&KVsh[0][0][0]);  // [qg][slice - 1][lane][34]: acc, m, l
  const int slice = 2 * kg + kh;
  if (slice > 0) {
    float *mine = mg + ((qg * (2 * KG - 1) + slice - 1) * 64 + lane) * 34;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      mine[r] = acc[0][r];
      mine[16 + r] = acc[1][r];
    }
    mine[32] = m_run;
    mine[33] = l_run;
  }
  __syncthreads();
  if (slice == 0 && qrow < nq) {
    float M = m_run;
#pragma unroll
    for (int j = 1; j < 2 * KG; ++j)
      M = fmaxf(M, mg[((qg * (2 * KG - 1) + j - 1) * 64 + lane) * 34 + 32]);
    const float f0 = m_run == -INFINITY ? 0.f : expf(m_run - M);
    float den = l_run * f0;
    floatx16 o0 = acc[0] * f0, o1 = acc[1] * f0;
#pragma unroll
    for (int j = 1; j < 2 * KG; ++j) {
      const float *src = mg + ((qg * (2 * KG - 1) + j - 1) * 64 + lane) * 34;
      const float mj = src[32];
      const float fj = mj == -INFINITY ? 0.f : expf(mj - M);
      den = fmaf(src[33], fj, den);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        o0[r] = fmaf(src[r], fj, o0[r]);
        o1[r] = fmaf(src[16 + r], fj, o1[r]);
      }
    }
    const float inv = 1.0f / den;
    float *o = out + (size_t)(t0 + qrow) * dim + (size_t)h * hd;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = 8 * g4 + 4 * hh;
      if (d0 < hd)
        *reinterpret_cast<float4 *>(o + d0) = make_float4(
            o0[4 * g4] * inv, o0[4 * g4 + 1] * inv, o0[4 * g4 + 2] * inv, o0[4 * g4 + 3] * inv);
      if (32 + d0 < hd)
        *reinterpret_cast<float4 *>(o + 32 + d0) = make_float4(
            o1[4 * g4] * inv, o1[4 * g4 + 1] * inv, o1[4 * g4 + 2] * inv, o1[4 * g4 + 3] * inv);
    }
  }
}

extern "C" __global__ void __launch_bounds__(256)
pbx_attention_mfma(const float *qkv, const float *kcache, const float *vcache, float *out,
                   int start, int n_rows, int n_heads, int n_kv_heads, int head_dim,
                   float scale) {
  attention_mfma_body<1>(qkv, kcache, vcache, out, start, n_rows, n_heads, n_kv_heads, head_dim,
                         scale);
}
#define PBX_ATTN_MFMA_KG(KG)                                                                   \
  extern "C" __global__ void __launch_bounds__(256 * KG)                                       \
      pbx_attention_mfma_g##KG(const float *qkv, const float *kcache, const float *vcache,     \
                               float *out, int start, int n_rows, int n_heads, int n_kv_heads, \
                               int head_dim, float scale) {                                    \
    attention_mfma_body<KG>(qkv, kcache, vcache, out, start, n_rows, n_heads, n_kv_heads,      \
                            head_dim, scale);                                                  \
  }
PBX_ATTN_MFMA_KG(2)
#undef PBX_ATTN_MFMA_KG

// SwiGLU rows (llama.js:329-333): h[t][i] = silu(gate[t][i]) * up[t][i],
// gate and up side by side in gu[t] = [gate | up].
extern "C" __global__ void __launch_bounds__(256)
pbx_swiglu_rows(const float *gu, float *h, int hidden) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= hidden) return;
  const float *r = gu + (size_t)t * 2 * hidden;
  h[(size_t)t * hidden + i] = silu(r[i]) * r[hidden + i];
}

// y += x, elementwise (residual connection for paths without a fused epilogue).
extern "C" __global__ void __launch_bounds__(256)
pbx_add_inplace(float *y, const float *x, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] += x[i];
}

// Argmax of each row of logits [M][vocab] (first maximum wins,
// llama.js:432-442), each row scanned by P workgroups in one launch:
// workgroup (p, row) reduces columns [p*chunk, (p+1)*chunk) to one key and
// folds it into the row's cell cells[row * stride] by a device-scope atomic max, waits for that to
// return, and only then counts itself in at cells[row * stride + 1]; the
// workgroup that completes the count of P therefore reads the final
// maximum (one more atomic, at the same coherence point), writes the row's
// token and clears both cells for the next launch (zero before the first).
extern "C" __global__ void __launch_bounds__(256)
pbx_argmax_rows(const float *logits, int vocab, int chunk, unsigned long long *cells, int stride,
                int P, int *out) {
  __shared__ uint64_t red[4];
  const int row = blockIdx.y, p = blockIdx.x;
  const float *r = logits + (size_t)row * vocab;
  const int lo = p * chunk, hi = min(vocab, lo + chunk);
  uint64_t best = 0;
  for (int i = lo + threadIdx.x; i < hi; i += blockDim.x) {
    const uint64_t k = argmax_key(r[i], (unsigned)i);
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) best = red[w] > best ? red[w] : best;
    best = red[0] > best ? red[0] : best;
    unsigned long long *c = cells + (size_t)row * stride;
    const unsigned long long prev =
        __hip_atomic_fetch_max(c, (unsigned long long)best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::"v"(prev) : "memory");  // the max has been applied
    const unsigned long long n =
        __hip_atomic_fetch_add(c + 1, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n == (unsigned long long)(P - 1)) {
      const unsigned long long k =
          __hip_atomic_fetch_max(c, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      out[row] = k ? (int)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFu)) : 0;
      __hip_atomic_store(c, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(c + 1, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

