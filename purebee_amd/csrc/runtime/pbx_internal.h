// pbx_internal.h -- shared definitions of the runtime's translation units.
#ifndef PBX_INTERNAL_H
#define PBX_INTERNAL_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <string>
#include <unordered_map>

#include "pbx.h"

// Kernels of pbx_kernels.hsaco, looked up by name at pbx_init.
#define PBX_KERNEL_LIST(X)                                   \
  X(PBX_K_REPACK_Q4_0, "pbx_repack_q4_0")                    \
  X(PBX_K_REPACK_Q8_0, "pbx_repack_q8_0")                    \
  X(PBX_K_REPACK_Q4_1, "pbx_repack_q4_1")                    \
  X(PBX_K_DEQUANT_Q4_1, "pbx_dequant_q4_1")                  \
  X(PBX_K_GEMV_Q4_1_WIDE_R4, "pbx_gemv_q4_1_wide_r4")        \
  X(PBX_K_GEMV_Q4_1_WIDE_R8, "pbx_gemv_q4_1_wide_r8")        \
  X(PBX_K_GEMV_Q4_1_WIDE_R16, "pbx_gemv_q4_1_wide_r16")      \
  X(PBX_K_GEMV_Q4_1_SMALL, "pbx_gemv_q4_1_small")            \
  X(PBX_K_REPACK_Q6_K, "pbx_repack_q6_k")                    \
  X(PBX_K_DEQUANT_F16, "pbx_dequant_f16")                    \
  X(PBX_K_DEQUANT_Q6_K, "pbx_dequant_q6_k")                  \
  X(PBX_K_GEMV_F16_WIDE_R4, "pbx_gemv_f16_wide_r4")          \
  X(PBX_K_GEMV_F16_WIDE_R8, "pbx_gemv_f16_wide_r8")          \
  X(PBX_K_GEMV_F16_SMALL, "pbx_gemv_f16_small")              \
  X(PBX_K_GEMV_Q6_K_WIDE_R4, "pbx_gemv_q6_k_wide_r4")        \
  X(PBX_K_GEMV_Q6_K_WIDE_R8, "pbx_gemv_q6_k_wide_r8")        \
  X(PBX_K_GEMV_Q6_K_SMALL, "pbx_gemv_q6_k_small")            \
  X(PBX_K_DEQUANT_Q4_0, "pbx_dequant_q4_0")                  \
  X(PBX_K_DEQUANT_Q8_0, "pbx_dequant_q8_0")                  \
  X(PBX_K_DEQUANT_Q8REF, "pbx_dequant_q8ref")                \
  X(PBX_K_GEMV_Q4_0_WIDE_R4, "pbx_gemv_q4_0_wide_r4")        \
  X(PBX_K_GEMV_Q4_0_WIDE_R8, "pbx_gemv_q4_0_wide_r8")        \
  X(PBX_K_GEMV_Q4_0_WIDE_R16, "pbx_gemv_q4_0_wide_r16")      \
  X(PBX_K_GEMV_Q8_0_WIDE_R4, "pbx_gemv_q8_0_wide_r4")        \
  X(PBX_K_GEMV_Q8_0_WIDE_R8, "pbx_gemv_q8_0_wide_r8")        \
  X(PBX_K_GEMV_F32_WIDE_R2, "pbx_gemv_f32_wide_r2")          \
  X(PBX_K_GEMV_F32_WIDE_R4, "pbx_gemv_f32_wide_r4")          \
  X(PBX_K_GEMV_Q4_0_SMALL, "pbx_gemv_q4_0_small")            \
  X(PBX_K_GEMV_Q8_0_SMALL, "pbx_gemv_q8_0_small")            \
  X(PBX_K_GEMV_F32_SMALL, "pbx_gemv_f32_small")              \
  X(PBX_K_GEMV_Q8REF, "pbx_gemv_q8ref")                      \
  X(PBX_K_COPY16, "pbx_copy16")

enum {
#define X(id, name) id,
  PBX_KERNEL_LIST(X)
#undef X
  PBX_K_COUNT
};

// Row count from which quantized linears take the MFMA GEMM path.
#define PBX_GEMM_MIN_M 4

#define PBX_MAX_MODULES 8

#define PBX_WEIGHT_MAGIC 0x50425857u  // "PBXW"

// Host-side layout of GemvArgs (pbx_gemv_impl.h), passed by value to the
// GEMV kernels that take the argument block.
struct pbx_gemv_args {
  const void *qs;
  const void *dsc;
  const float *X;
  const float *X2;
  const float *normw;
  const float *bias;
  float *Y;
  uint64_t *partials;
  int N, B;
  float eps;
  const void *msc;
  int rows;
  // the q|k|v rows of a decode step or a batch (RoPE + cache append
  // epilogue; a batch's row m sits at position pos0 + m)
  const int *state = nullptr;
  const float *rope = nullptr;
  float *kcache = nullptr, *vcache = nullptr;
  int qdim = 0, kvdim = 0, head_dim = 0;
  int pos0 = 0;
  // the residual's pending update (2^-32 units) that the gate|up GEMV adds
  // to its input and the down GEMV folds into the residual
  long long *acc = nullptr;
  // rows GEMV with the K blocks split over workgroups: one 64-bit cell per
  // output element (zero between launches)
  unsigned long long *xcell = nullptr;
  // builder waves: clr_n 64-bit words of clr zeroed by the launch; adv: an
  // epoch advanced once by the launch
  long long *clr = nullptr;
  int clr_n = 0;
  unsigned long long *adv = nullptr;
};

struct pbx_ctx {
  int device = 0;
  int cu_count = 256;
  bool gemv_int = true;  // integer-limb GEMVs for the instruction (PBX_GEMV_INT=0: off)
  char name[256] = {0};
  std::string code_object;
  std::string err;
  hipModule_t modules[PBX_MAX_MODULES] = {};
  hipFunction_t fn[PBX_K_COUNT] = {};
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  hipEvent_t ev_stage[2] = {nullptr, nullptr};
  // grow-only scratch
  void *d_x = nullptr, *d_y = nullptr, *d_b = nullptr;
  size_t d_x_cap = 0, d_y_cap = 0, d_b_cap = 0;
  void *d_gemm = nullptr;  // GEMM workspace: fp16 activations, row scales, split-K partials
  size_t d_gemm_cap = 0;
  void *d_stage[2] = {nullptr, nullptr};
  size_t d_stage_cap[2] = {0, 0};
  void *h_io = nullptr;
  size_t h_io_cap = 0;
  // pbx_linear with M < 4: x is read from coherent pinned memory by a copy
  // kernel (h_x, device address d_hx) and the GEMV stores y straight into
  // h_y (device address d_hy): no copy operation
  void *h_x = nullptr, *d_hx = nullptr, *h_y = nullptr, *d_hy = nullptr;
  size_t h_x_cap = 0, h_y_cap = 0;
  void *h_stage[2] = {nullptr, nullptr};
  size_t h_stage_cap[2] = {0, 0};
  void *models = nullptr;  // decode-step models owned by this context
  // this device's copy of the library's static device array (pbx_scratch.hip),
  // the workspace of pbx_linear_dev_noalloc; null when the lookup failed
  void *scratch = nullptr;
  size_t scratch_bytes = 0;
  std::string scratch_err;
  std::unordered_map<std::string, hipFunction_t> named;  // kernels looked up by name
};

struct pbx_weight {
  uint32_t magic = 0;
  int type = 0;
  int64_t N = 0, K = 0, B = 0, Npad = 0;
  int64_t n_scales = 0;
  void *qs = nullptr;  // nibble / int8 / f32 plane (Q8_REF: flat int8 [K,N])
  void *d = nullptr;   // fp16 scale plane (Q8_REF: f32 scales)
  void *m = nullptr;   // Q4_1: fp16 min plane (inside the d allocation)
  size_t bytes = 0;
};

int pbx_fail(pbx_ctx *c, int code, const char *fmt, ...)
    __attribute__((format(printf, 3, 4)));
int pbx_launch(pbx_ctx *c, int kernel, dim3 grid, dim3 block, void **args,
               hipStream_t stream = nullptr);
hipFunction_t pbx_kernel_by_name(pbx_ctx *c, const std::string &name);
int pbx_launch_fn(pbx_ctx *c, hipFunction_t f, const char *name, dim3 grid, dim3 block,
                  void **args, hipStream_t stream);
int pbx_launch_fn_timed(pbx_ctx *c, hipFunction_t f, const char *name, dim3 grid, dim3 block,
                        void **args, hipStream_t stream, hipEvent_t start, hipEvent_t stop);
int pbx_weight_alloc(pbx_ctx *c, int type, int64_t N, int64_t K, pbx_weight **out);
int pbx_weight_write_rows(pbx_ctx *c, pbx_weight *w, int64_t row0, int64_t rows,
                          const void *host);
void pbx_weight_release(pbx_weight *w);
int pbx_ensure_dev(pbx_ctx *c, void **p, size_t *cap, size_t need);
int pbx_ensure_pinned(pbx_ctx *c, void **p, size_t *cap, size_t need);
// Device memory a launch path may use instead of growing the context's own
// buffers (pbx_linear_dev_noalloc); a path that would need more fails.
struct pbx_workspace {
  void *ptr;
  size_t bytes;
};
int pbx_linear_enqueue(pbx_ctx *c, const pbx_weight *w, const float *dX, int64_t M,
                       const float *dBias, float *dY, hipStream_t stream,
                       const pbx_workspace *ws = nullptr);
// Bytes of the static device workspace (pbx_scratch.hip) and the lookup of
// its address on the context's device (call with that device current).
#define PBX_SCRATCH_BYTES ((size_t)PBX_NOALLOC_WORKSPACE_BYTES)
int pbx_scratch_lookup(pbx_ctx *c);
// The fp16 MFMA GEMM in two parts, for callers that prepare the fp16
// activation pair (X16, X16lo, inv: [Mpad][K]) themselves: the kernel, grid
// and K split for M rows of weight w, and the launch, which writes Y (KS == 1,
// += if accumulate) or the KS partials [KS][M][N].
struct pbx_gemm_plan {
  int M = 0, Mpad = 0, mtiles = 0, nwg = 0, KS = 1;
  std::string name;
  bool swiglu = false;  // the kernel stores silu(gate) * up: Y is [M][N / 2]
};
// swiglu: w is a gate|up weight (N / 2 gate rows, then the up rows) and the
// caller takes silu(gate) * up where the shape allows it (p->swiglu says
// whether it does; otherwise Y holds gate and up side by side)
int pbx_gemm_make_plan(pbx_ctx *c, const pbx_weight *w, int M, pbx_gemm_plan *p,
                       bool swiglu = false);
int pbx_gemm_run(pbx_ctx *c, const pbx_weight *w, const pbx_gemm_plan &p, const void *x16,
                 const void *x16lo, const float *inv, const float *dBias, float *out,
                 int accumulate, hipStream_t stream);
int pbx_gemm_enqueue(pbx_ctx *c, const pbx_weight *w, const float *dX, int64_t M,
                     const float *dBias, float *dY, hipStream_t stream,
                     const pbx_workspace *ws = nullptr);
int pbx_gemm_launch(pbx_ctx *c, const pbx_weight *w, const float *dX, int64_t M,
                    const float *dBias, float *dY, int accumulate, hipStream_t stream,
                    const pbx_workspace *ws = nullptr);
// Bytes of one GGUF row of K elements (0 for an unknown type).
size_t pbx_type_row_bytes(int type, int64_t K);
void pbx_model_release_all(pbx_ctx *c);
int pbx_model_clear_range(pbx_model *m, int from, int to);
// pbx_model_generate with every step stopping after the first max_layers
// layers (0: all); the self-speculative draft.
int pbx_model_generate_layers(pbx_model *m, int32_t token, int start_pos, int n_steps,
                              int max_layers, int32_t *out_tokens);
const pbx_model_config *pbx_model_cfg(const pbx_model *m);
pbx_ctx *pbx_model_ctx(const pbx_model *m);

#endif
