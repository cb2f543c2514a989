// pbx_gemm.cpp -- launch path of the M >= 4 instruction: row scaling of the
// activations to fp16, the MFMA GEMM (pbx_gemm.hip) and, when the K blocks
// are split across workgroups, the reduction of the partial sums.

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
};

}  // namespace

int pbx_gemm_launch(pbx_ctx *c, const pbx_weight *w, const float *dX, int64_t M64,
                    const float *dBias, float *dY, int accumulate, hipStream_t stream) {
  if (w->type != PBX_TYPE_Q4_0 && w->type != PBX_TYPE_Q8_0)
    return pbx_fail(c, PBX_ENOTSUP, "pbx_gemm: weight type %d has no MFMA path", w->type);
  if (M64 > 65535) return pbx_fail(c, PBX_ENOTSUP, "pbx_gemm: M=%lld too large", (long long)M64);
  const int M = (int)M64, N = (int)w->N, B = (int)w->B, K = B * 32;
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
  // Split K so the grid has about two workgroups (big) or eight waves
  // (small) per CU.
  int KS = 1;
  if (big) {
    const int wgs = nwg * mtiles;
    if (wgs < want_wg) KS = std::min({B, 8, (want_wg + wgs - 1) / wgs});
  } else {
    const int waves = nwg * mtiles * 4;
    if (waves < 8 * c->cu_count) KS = std::min({B, 8, (8 * c->cu_count + waves - 1) / waves});
  }
  // fp16 activations and their fp16 rounding residuals
  const size_t x16_bytes = ((size_t)Mpad * K * 2 + 255) / 256 * 256;
  const size_t lo_bytes = x16_bytes;
  const size_t inv_bytes = ((size_t)Mpad * 4 + 255) / 256 * 256;
  const size_t part_bytes = KS > 1 ? (size_t)KS * M * N * 4 : 0;
  int rc = pbx_ensure_dev(c, &c->d_gemm, &c->d_gemm_cap,
                          x16_bytes + lo_bytes + inv_bytes + part_bytes);
  if (rc) return rc;
  char *ws = (char *)c->d_gemm;
  void *x16 = ws;
  void *x16lo = ws + x16_bytes;
  float *inv = (float *)(ws + x16_bytes + lo_bytes);
  float *part = (float *)(ws + x16_bytes + lo_bytes + inv_bytes);

  hipFunction_t fprep = pbx_kernel_by_name(c, "pbx_gemm_prep_x");
  const std::string name = std::string("pbx_gemm_") + (w->type == PBX_TYPE_Q4_0 ? "q4" : "q8") +
                           (big ? std::string("_big")
                                : "_m" + std::to_string(MT) + "_n" + std::to_string(NT));
  hipFunction_t fg = pbx_kernel_by_name(c, name);
  hipFunction_t fred = pbx_kernel_by_name(c, "pbx_gemm_reduce");
  if (!fprep || !fg || !fred) return pbx_fail(c, PBX_ELOAD, "pbx_gemm: kernel %s missing", name.c_str());
  {
    int m = M, k = K;
    void *args[] = {(void *)&dX, &x16, &x16lo, &inv, &m, &k};
    if ((rc = pbx_launch_fn(c, fprep, "pbx_gemm_prep_x", dim3(Mpad), dim3(256), args, stream)))
      return rc;
  }
  GemmArgsHost g{w->qs, w->d, x16, x16lo, inv, KS == 1 ? dBias : nullptr, KS == 1 ? dY : part,
                 M, N, (int)w->Npad, B, KS, KS == 1 ? accumulate : 0};
  {
    void *args[] = {&g};
    if ((rc = pbx_launch_fn(c, fg, name.c_str(), dim3(nwg, mtiles, KS), dim3(256), args, stream)))
      return rc;
  }
  if (KS > 1) {
    int m = M, n = N, ks = KS, acc = accumulate;
    void *args[] = {&part, (void *)&dBias, &dY, &m, &n, &ks, &acc};
    const int64_t MN = (int64_t)M * N;
    if ((rc = pbx_launch_fn(c, fred, "pbx_gemm_reduce", dim3((unsigned)((MN + 255) / 256)),
                            dim3(256), args, stream)))
      return rc;
  }
  return PBX_OK;
}

int pbx_gemm_enqueue(pbx_ctx *c, const pbx_weight *w, const float *dX, int64_t M,
                     const float *dBias, float *dY, hipStream_t stream) {
  return pbx_gemm_launch(c, w, dX, M, dBias, dY, 0, stream);
}
