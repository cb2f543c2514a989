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
pbx_embed_rows(const uint8_t *qs, const uint16_t *dsc, const int *tokens, float *x, int type,
               int dim, int vocab) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= dim) return;
  int tok = tokens[t];
  if (tok < 0 || tok >= vocab) tok = 0;
  const int B = dim / 32, b = i / 32, j = i % 32;
  float v;
  if (type == PBX_F32) {
    v = reinterpret_cast<const float *>(qs)[(size_t)tok * dim + i];
  } else {
    const float d = f16_bits_to_f32(dsc[dsc_index(tok, b, B)]);
    if (type == PBX_Q4) {
      const unsigned byte = qs[((size_t)tok * B + b) * 16 + (j & 15)];
      v = (float)((int)(j < 16 ? (byte & 15u) : (byte >> 4)) - 8) * d;
    } else {
      v = (float)(int8_t)qs[((size_t)tok * B + b) * 32 + j] * d;
    }
  }
  x[(size_t)t * dim + i] = v;
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
