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
extern "C" __global__ void __launch_bounds__(256)
pbx_rope_append_rows(float *qkv, float *kcache, float *vcache, const float *rope, int start,
                     int n_heads, int n_kv_heads, int head_dim) {
  const int t = blockIdx.x, pos = start + t;
  const int dim = n_heads * head_dim, kvdim = n_kv_heads * head_dim;
  float *row = qkv + (size_t)t * (dim + 2 * kvdim);
  const float *rp = rope + (size_t)pos * head_dim;
  const int half = head_dim / 2;
  for (int p = threadIdx.x; p < (n_heads + n_kv_heads) * half; p += blockDim.x) {
    const int h = p / half, i = p % half;
    float *v = h < n_heads ? row + h * head_dim + 2 * i : row + dim + (h - n_heads) * head_dim + 2 * i;
    const float c = rp[2 * i], s = rp[2 * i + 1];
    const float a0 = v[0], a1 = v[1];
    v[0] = a0 * c - a1 * s;
    v[1] = a0 * s + a1 * c;
  }
  __syncthreads();
  for (int d = threadIdx.x; d < kvdim; d += blockDim.x) {
    kcache[(size_t)pos * kvdim + d] = row[dim + d];
    vcache[(size_t)pos * kvdim + d] = row[dim + kvdim + d];
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
// llama.js:432-442), in two passes so a row is scanned by many workgroups:
// workgroup (p, row) reduces columns [p*chunk, (p+1)*chunk) to one key,
// then one wave per row reduces the P keys.
extern "C" __global__ void __launch_bounds__(256)
pbx_argmax_rows_partial(const float *logits, int vocab, int chunk, uint64_t *keys, int P) {
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
    keys[(size_t)row * P + p] = best;
  }
}

extern "C" __global__ void __launch_bounds__(64)
pbx_argmax_rows_final(const uint64_t *keys, int P, int *out) {
  const uint64_t *k = keys + (size_t)blockIdx.x * P;
  uint64_t best = 0;
  for (int i = threadIdx.x; i < P; i += 64) best = k[i] > best ? k[i] : best;
  best = wave_max_u64(best);
  if (threadIdx.x == 0)
    out[blockIdx.x] = best ? (int)(0xFFFFFFFFu - (unsigned)(best & 0xFFFFFFFFu)) : 0;
}
