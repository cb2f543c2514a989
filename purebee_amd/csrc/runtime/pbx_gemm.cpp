// pbx_gemm.cpp -- launch path of the M >= 4 instruction: row scaling of the
// activations to fp16, the MFMA GEMM (pbx_gemm.hip) and, when the K blocks
// are split across workgroups, the reduction of the partial sums.  F32
// weights take the fp32 MFMA kernels, which read the activations as they are.

#include <algorithm>
#include <string>

#include "pbx_internal.h"

namespace {

struct GemmArgsHost {  // GemmArgs in pbx_gemm.hip
  const void *qs;
  const void *dsc;
  const void *X16;
  const void *X16lo;
  const float *inv;
  const float *bias;
  float *Y;
  int M, N, Npad, B, KS;
  int accumulate;
  const void *msc;
};

struct GemmF32ArgsHost {  // GemmF32Args in pbx_gemm.hip
  const void *W;
  const float *X;
  const float *bias;
  float *Y;
  int M, N, Npad, B, KS;
  int accumulate;
};

const char *gemm_tag(int type) {
  switch (type) {
    case PBX_TYPE_Q4_0: return "q4";
    case PBX_TYPE_Q8_0: return "q8";
    case PBX_TYPE_Q4_1: return "q41";
    case PBX_TYPE_F16: return "f16";
    case PBX_TYPE_F32: return "f32";
    default: return nullptr;
  }
}

// `need` bytes of workspace: from ws when the caller brings one (an error if
// it is too small), else the context's grow-only GEMM buffer.
int workspace(pbx_ctx *c, const pbx_workspace *ws, size_t need, char **out) {
  if (ws) {
    if (!ws->ptr)
      return pbx_fail(c, PBX_ENOTSUP, "pbx_linear: no device workspace available");
    if (need > ws->bytes)
      return pbx_fail(c, PBX_EINVAL,
                      "pbx_linear: this shape needs %zu bytes of workspace, above the %zu-byte "
                      "limit of the no-allocation entry point",
                      need, ws->bytes);
    *out = (char *)ws->ptr;
    return PBX_OK;
  }
  int rc = pbx_ensure_dev(c, &c->d_gemm, &c->d_gemm_cap, need);
  if (rc) return rc;
  *out = (char *)c->d_gemm;
  return PBX_OK;
}

// Sum of the split-K partials into dY (+ bias, or accumulated).
int launch_reduce(pbx_ctx *c, float *part, const float *dBias, float *dY, int M, int N, int KS,
                  int accumulate, hipStream_t stream) {
  hipFunction_t fred = pbx_kernel_by_name(c, "pbx_gemm_reduce");
  if (!fred) return pbx_fail(c, PBX_ELOAD, "pbx_gemm: kernel pbx_gemm_reduce missing");
  int m = M, n = N, ks = KS, acc = accumulate;
  void *args[] = {&part, (void *)&dBias, &dY, &m, &n, &ks, &acc};
  const int64_t MN = (int64_t)M * N;
  return pbx_launch_fn(c, fred, "pbx_gemm_reduce", dim3((unsigned)((MN + 255) / 256)), dim3(256),
                       args, stream);
}

// F32 weights: fp32 MFMA.  M > 32: the LDS-DMA 128 x 128 kernel; otherwise
// wave tile 16*MT x 16*NT (MT 1 / 2 for M <= 16 / <= 32), K split for about
// eight waves per CU.
int launch_f32(pbx_ctx *c, const pbx_weight *w, const float *dX, int M, const float *dBias,
               float *dY, int accumulate, hipStream_t stream, const pbx_workspace *ws) {
  const int N = (int)w->N, B = (int)w->B;
  if (M > 32) {
    // 128 x 128 tiles on the LDS-DMA kernel, K split (16-k steps) for about
    // one workgroup per CU
    const int nwg = (N + 127) / 128, mtiles = (M + 127) / 128, wgs = nwg * mtiles;
    int KS = 1;
    if (wgs < c->cu_count) KS = std::min({2 * B, 8, (c->cu_count + wgs - 1) / wgs});
    float *part = nullptr;
    if (KS > 1) {
      char *p = nullptr;
      int rc = workspace(c, ws, (size_t)KS * M * N * 4, &p);
      if (rc) return rc;
      part = (float *)p;
    }
    hipFunction_t fg = pbx_kernel_by_name(c, "pbx_gemm_f32_big");
    if (!fg) return pbx_fail(c, PBX_ELOAD, "pbx_gemm: kernel pbx_gemm_f32_big missing");
    GemmF32ArgsHost g{w->qs, dX, KS == 1 ? dBias : nullptr, KS == 1 ? dY : part,
                      M, N, (int)w->Npad, B, KS, KS == 1 ? accumulate : 0};
    void *args[] = {&g};
    int rc = pbx_launch_fn(c, fg, "pbx_gemm_f32_big", dim3(nwg, mtiles, KS), dim3(256), args, stream);
    if (rc || KS == 1) return rc;
    return launch_reduce(c, part, dBias, dY, M, N, KS, accumulate, stream);
  }
  const int MT = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  const int mtiles = (M + 16 * MT - 1) / (16 * MT);
  int NT;
  if (MT == 1)
    NT = ((N + 255) / 256) * mtiles >= 2 * c->cu_count ? 4
         : ((N + 127) / 128) * mtiles >= 2 * c->cu_count ? 2 : 1;
  else
    NT = MT == 2 ? 2 : 4;
  const int nwg = (N + 64 * NT - 1) / (64 * NT);
  int KS = 1;
  const int waves = nwg * mtiles * 4;
  if (waves < 8 * c->cu_count) KS = std::min({B, 8, (8 * c->cu_count + waves - 1) / waves});
  float *part = nullptr;
  if (KS > 1) {
    char *p = nullptr;
    int rc = workspace(c, ws, (size_t)KS * M * N * 4, &p);
    if (rc) return rc;
    part = (float *)p;
  }
  const std::string name = "pbx_gemm_f32_m" + std::to_string(MT) + "_n" + std::to_string(NT);
  hipFunction_t fg = pbx_kernel_by_name(c, name);
  if (!fg) return pbx_fail(c, PBX_ELOAD, "pbx_gemm: kernel %s missing", name.c_str());
  GemmF32ArgsHost g{w->qs, dX, KS == 1 ? dBias : nullptr, KS == 1 ? dY : part,
                    M, N, (int)w->Npad, B, KS, KS == 1 ? accumulate : 0};
  void *args[] = {&g};
  int rc = pbx_launch_fn(c, fg, name.c_str(), dim3(nwg, mtiles, KS), dim3(256), args, stream);
  if (rc || KS == 1) return rc;
  return launch_reduce(c, part, dBias, dY, M, N, KS, accumulate, stream);
}

}  // namespace

int pbx_gemm_make_plan(pbx_ctx *c, const pbx_weight *w, int M, pbx_gemm_plan *p, bool swiglu) {
  if (!gemm_tag(w->type) || w->type == PBX_TYPE_F32)
    return pbx_fail(c, PBX_ENOTSUP, "pbx_gemm: weight type %d has no fp16 MFMA path", w->type);
  if (M <= 0 || M > 65535) return pbx_fail(c, PBX_ENOTSUP, "pbx_gemm: M=%d out of range", M);
  const int N = (int)w->N, B = (int)w->B;
  // M > 32: the LDS-tiled 128 x 128 kernel; otherwise one wave per 16*MT
  // rows x 16*NT weight rows.
  const bool big = M > 32;
  const int MT = big ? 8 : M <= 16 ? 1 : 2;
  const int Mpad = (M + 16 * MT - 1) / (16 * MT) * (16 * MT);
  const int mtiles = Mpad / (16 * MT);
  const int want_wg = 2 * c->cu_count;
  int NT, nwg;
  if (big) {
    NT = 8;
    nwg = (N + 127) / 128;
  } else {
    // Largest n tile that still gives two workgroups per CU.
    if (MT == 1)
      NT = ((N + 255) / 256) * mtiles >= want_wg ? 4 : ((N + 127) / 128) * mtiles >= want_wg ? 2 : 1;
    else
      NT = 2;
    nwg = (N + 64 * NT - 1) / (64 * NT);
  }
  // Split K so the grid has about one workgroup (big) or eight waves
  // (small) per CU.
  int KS = 1;
  int mt_rows = 128;
  int mtl = mtiles;
  if (big) {
    // 128 x 128 tiles where they give two workgroups a CU (the prefill's
    // gate|up); otherwise 64-row M tiles (pbx_gemm_<type>_b64) with the K
    // split to two workgroups a CU (PBX_GEMM_M64 = workgroups a CU, 0: the
    // 128-row tiles at about one a CU).  512-token prefill: 4.34 against
    // 4.48 ms (q|k|v 37.3 -> 32.2 us, o 25 -> 22.5 us; down unchanged);
    // three or four a CU: 4.48 and 4.67 ms.  With 128-row tiles a deeper
    // split costs more in partial traffic and per-workgroup start-up than
    // the extra occupancy returns (measured against 0.5, 0.75, 1.5, 2 and 3
    // per CU).
    const int wgs = nwg * mtiles;
    const char *e = getenv("PBX_GEMM_M64");
    const int per_cu = e ? atoi(e) : 2;
    if (per_cu > 0 && wgs < per_cu * c->cu_count) {
      mt_rows = 64;
      mtl = Mpad / 64;
      const int w64 = nwg * mtl;
      if (w64 < per_cu * c->cu_count)
        KS = std::min({B, 8, (per_cu * c->cu_count + w64 - 1) / w64});
    } else if (wgs < c->cu_count) {
      KS = std::min({B, 8, (c->cu_count + wgs - 1) / wgs});
    }
  } else {
    const int waves = nwg * mtiles * 4;
    if (waves < 8 * c->cu_count) KS = std::min({B, 8, (8 * c->cu_count + waves - 1) / waves});
  }
  p->M = M;
  p->Mpad = Mpad;
  p->mtiles = mtl;
  p->nwg = nwg;
  p->KS = KS;
  // gate|up with silu(gate) * up in the epilogue (M > 32 kernels, no K
  // split, 64 hidden columns a workgroup, 32-bit weight offsets);
  // PBX_GEMM_SWIGLU=0 keeps gate and up side by side
  const char *sw_env = getenv("PBX_GEMM_SWIGLU");
  p->swiglu = swiglu && big && KS == 1 && N % 128 == 0 &&
              (double)N * pbx_type_row_bytes(w->type, w->K) < 4294967296.0 &&
              !(sw_env && sw_env[0] == '0');
  p->name = std::string("pbx_gemm_") + gemm_tag(w->type) +
            (big ? std::string(mt_rows == 64 ? "_b64" : "_big")
                 : "_m" + std::to_string(MT) + "_n" + std::to_string(NT)) +
            (p->swiglu ? "_sw" : "");
  return PBX_OK;
}

int pbx_gemm_run(pbx_ctx *c, const pbx_weight *w, const pbx_gemm_plan &p, const void *x16,
                 const void *x16lo, const float *inv, const float *dBias, float *out,
                 int accumulate, hipStream_t stream) {
  hipFunction_t fg = pbx_kernel_by_name(c, p.name);
  if (!fg) return pbx_fail(c, PBX_ELOAD, "pbx_gemm: kernel %s missing", p.name.c_str());
  GemmArgsHost g{w->qs, w->d, x16, x16lo, inv, p.KS == 1 ? dBias : nullptr, out,
                 p.M, (int)w->N, (int)w->Npad, (int)w->B, p.KS, p.KS == 1 ? accumulate : 0, w->m};
  void *args[] = {&g};
  return pbx_launch_fn(c, fg, p.name.c_str(), dim3(p.nwg, p.mtiles, p.KS), dim3(256), args, stream);
}

int pbx_gemm_launch(pbx_ctx *c, const pbx_weight *w, const float *dX, int64_t M64,
                    const float *dBias, float *dY, int accumulate, hipStream_t stream,
                    const pbx_workspace *wsp) {
  if (!gemm_tag(w->type))
    return pbx_fail(c, PBX_ENOTSUP, "pbx_gemm: weight type %d has no MFMA path", w->type);
  if (M64 > 65535) return pbx_fail(c, PBX_ENOTSUP, "pbx_gemm: M=%lld too large", (long long)M64);
  if (w->type == PBX_TYPE_F32)
    return launch_f32(c, w, dX, (int)M64, dBias, dY, accumulate, stream, wsp);
  const int M = (int)M64, N = (int)w->N, K = (int)w->B * 32;
  pbx_gemm_plan p;
  int rc = pbx_gemm_make_plan(c, w, M, &p);
  if (rc) return rc;
  // fp16 activations and their fp16 rounding residuals
  const size_t x16_bytes = ((size_t)p.Mpad * K * 2 + 255) / 256 * 256;
  const size_t lo_bytes = x16_bytes;
  const size_t inv_bytes = ((size_t)p.Mpad * 4 + 255) / 256 * 256;
  const size_t part_bytes = p.KS > 1 ? (size_t)p.KS * M * N * 4 : 0;
  char *ws = nullptr;
  if ((rc = workspace(c, wsp, x16_bytes + lo_bytes + inv_bytes + part_bytes, &ws))) return rc;
  void *x16 = ws;
  void *x16lo = ws + x16_bytes;
  float *inv = (float *)(ws + x16_bytes + lo_bytes);
  float *part = (float *)(ws + x16_bytes + lo_bytes + inv_bytes);
  hipFunction_t fprep = pbx_kernel_by_name(c, "pbx_gemm_prep_x");
  if (!fprep) return pbx_fail(c, PBX_ELOAD, "pbx_gemm: kernel pbx_gemm_prep_x missing");
  {
    int m = M, k = K;
    void *args[] = {(void *)&dX, &x16, &x16lo, &inv, &m, &k};
    if ((rc = pbx_launch_fn(c, fprep, "pbx_gemm_prep_x", dim3(p.Mpad), dim3(256), args, stream)))
      return rc;
  }
  if ((rc = pbx_gemm_run(c, w, p, x16, x16lo, inv, dBias, p.KS == 1 ? dY : part, accumulate,
                         stream)))
    return rc;
  if (p.KS > 1) return launch_reduce(c, part, dBias, dY, M, N, p.KS, accumulate, stream);
  return PBX_OK;
}

int pbx_gemm_enqueue(pbx_ctx *c, const pbx_weight *w, const float *dX, int64_t M,
                     const float *dBias, float *dY, hipStream_t stream, const pbx_workspace *ws) {
  return pbx_gemm_launch(c, w, dX, M, dBias, dY, 0, stream, ws);
}
