// pbx_runtime.cpp -- host side of the C ABI declared in include/pbx.h.
//
// Owns the HIP device context, the context's stream, the gfx950 code object
// (loaded with hipModuleLoad, kernels launched with hipModuleLaunchKernel),
// resident weights and the launch heuristics.  No torch, no CUDA shims: the
// only dependency is the HIP runtime.

#include "pbx_internal.h"

#include <dlfcn.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>

static thread_local std::string g_err;  // failures before a context exists

int pbx_fail(pbx_ctx *c, int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (c) c->err = buf;
  g_err = buf;
  return code;
}

#define HIPCHK(ctx, call)                                                        \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess)                                                        \
      return pbx_fail((ctx), PBX_EHIP, "%s failed: %s", #call, hipGetErrorString(e_)); \
  } while (0)

extern "C" const char *pbx_last_error(const pbx_ctx *ctx) {
  return ctx ? ctx->err.c_str() : g_err.c_str();
}

// ---------------------------------------------------------------------------
// Kernel table.
// ---------------------------------------------------------------------------
static const char *const kKernelNames[PBX_K_COUNT] = {
#define X(id, name) name,
    PBX_KERNEL_LIST(X)
#undef X
};

// Code objects built from purebee_amd/csrc/kernels/*.hip, found next to this
// library (or in the directory named by PBX_KERNEL_DIR).
static const char *const kModuleFiles[] = {"pbx_gemv.hsaco", "pbx_decode.hsaco", "pbx_gemm.hsaco",
                                          "pbx_prefill.hsaco"};
static const int kModuleCount = (int)(sizeof kModuleFiles / sizeof kModuleFiles[0]);

static std::string code_object_dir() {
  const char *env = getenv("PBX_KERNEL_DIR");
  if (env && *env) return env;
  Dl_info info;
  if (dladdr((void *)&pbx_init, &info) && info.dli_fname) {
    std::string p = info.dli_fname;
    size_t slash = p.rfind('/');
    return slash == std::string::npos ? "." : p.substr(0, slash);
  }
  return ".";
}

static void unload_modules(pbx_ctx *c) {
  for (int i = 0; i < PBX_MAX_MODULES; ++i)
    if (c->modules[i]) {
      hipModuleUnload(c->modules[i]);
      c->modules[i] = nullptr;
    }
}

extern "C" int pbx_init(int device, pbx_ctx **out) {
  if (!out) return pbx_fail(nullptr, PBX_EINVAL, "pbx_init: out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return pbx_fail(nullptr, PBX_ENODEV, "pbx_init: no HIP device (%s)",
                    e == hipSuccess ? "device count is 0" : hipGetErrorString(e));
  if (device < 0 || device >= n)
    return pbx_fail(nullptr, PBX_ENODEV, "pbx_init: device %d out of range [0, %d)", device, n);
  const std::string dir = code_object_dir();
  for (int m = 0; m < kModuleCount; ++m) {
    std::string path = dir + "/" + kModuleFiles[m];
    FILE *f = fopen(path.c_str(), "rb");
    if (!f)
      return pbx_fail(nullptr, PBX_ELOAD, "pbx_init: code object '%s' not found (build it first)",
                      path.c_str());
    fclose(f);
  }

  pbx_ctx *c = new pbx_ctx();
  c->device = device;
  c->code_object = dir;
  if (hipSetDevice(device) != hipSuccess) {
    delete c;
    return pbx_fail(nullptr, PBX_EHIP, "pbx_init: hipSetDevice(%d) failed", device);
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
    snprintf(c->name, sizeof c->name, "%s (%s)", prop.name, prop.gcnArchName);
    c->cu_count = prop.multiProcessorCount;
  }
  {
    const char *gi = getenv("PBX_GEMV_INT");
    c->gemv_int = !(gi && gi[0] == '0');
  }
  // the no-allocation entry point's workspace on this device (a failed
  // lookup only disables that entry point)
  (void)pbx_scratch_lookup(c);
  for (int m = 0; m < kModuleCount; ++m) {
    std::string path = dir + "/" + kModuleFiles[m];
    e = hipModuleLoad(&c->modules[m], path.c_str());
    if (e != hipSuccess) {
      c->modules[m] = nullptr;
      unload_modules(c);
      delete c;
      return pbx_fail(nullptr, PBX_ELOAD, "pbx_init: hipModuleLoad('%s') failed: %s "
                      "(the code objects are built for gfx950)", path.c_str(), hipGetErrorString(e));
    }
  }
  for (int i = 0; i < PBX_K_COUNT; ++i) {
    c->fn[i] = nullptr;
    for (int m = 0; m < kModuleCount && !c->fn[i]; ++m) {
      hipFunction_t f = nullptr;
      if (hipModuleGetFunction(&f, c->modules[m], kKernelNames[i]) == hipSuccess) c->fn[i] = f;
    }
    if (!c->fn[i]) {
      unload_modules(c);
      delete c;
      return pbx_fail(nullptr, PBX_ELOAD, "pbx_init: kernel '%s' missing from the code objects in '%s'",
                      kKernelNames[i], dir.c_str());
    }
  }
  (void)hipGetLastError();  // lookups that missed in earlier modules are not errors
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreate(&c->ev0) != hipSuccess || hipEventCreate(&c->ev1) != hipSuccess ||
      hipEventCreate(&c->ev_stage[0]) != hipSuccess ||
      hipEventCreate(&c->ev_stage[1]) != hipSuccess) {
    unload_modules(c);
    delete c;
    return pbx_fail(nullptr, PBX_EHIP, "pbx_init: stream/event creation failed");
  }
  *out = c;
  return PBX_OK;
}

extern "C" void pbx_shutdown(pbx_ctx *c) {
  if (!c) return;
  hipSetDevice(c->device);
  hipStreamSynchronize(c->stream);
  pbx_model_release_all(c);
  for (void *p : {c->d_x, c->d_y, c->d_b, c->d_gemm, c->d_stage[0], c->d_stage[1]})
    if (p) hipFree(p);
  for (void *p : {c->h_io, c->h_x, c->h_y, c->h_stage[0], c->h_stage[1]})
    if (p) hipHostFree(p);
  hipEventDestroy(c->ev0);
  hipEventDestroy(c->ev1);
  hipEventDestroy(c->ev_stage[0]);
  hipEventDestroy(c->ev_stage[1]);
  hipStreamDestroy(c->stream);
  unload_modules(c);
  delete c;
}

extern "C" int pbx_device_info(pbx_ctx *c, char *name, size_t cap, int *cu_count) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_device_info: ctx is NULL");
  if (name && cap) {
    strncpy(name, c->name, cap - 1);
    name[cap - 1] = 0;
  }
  if (cu_count) *cu_count = c->cu_count;
  return PBX_OK;
}

hipFunction_t pbx_kernel_by_name(pbx_ctx *c, const std::string &name) {
  auto it = c->named.find(name);
  if (it != c->named.end()) return it->second;
  hipFunction_t f = nullptr;
  for (int m = 0; m < PBX_MAX_MODULES && !f; ++m) {
    hipFunction_t g = nullptr;
    if (c->modules[m] && hipModuleGetFunction(&g, c->modules[m], name.c_str()) == hipSuccess) f = g;
  }
  (void)hipGetLastError();
  if (f) c->named[name] = f;
  return f;
}

int pbx_launch_fn(pbx_ctx *c, hipFunction_t f, const char *name, dim3 grid, dim3 block,
                  void **args, hipStream_t stream) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return PBX_OK;
  hipError_t e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, 0,
                                       stream ? stream : c->stream, args, nullptr);
  if (e != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "launch of %s failed: %s", name, hipGetErrorString(e));
  return PBX_OK;
}

// hip/hip_ext.h (its templates need the device-side headers a host-only
// build does not include)
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX,
                                               uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
                                               uint32_t localWorkSizeX, uint32_t localWorkSizeY,
                                               uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void **kernelParams,
                                               void **extra, hipEvent_t startEvent,
                                               hipEvent_t stopEvent, uint32_t flags);

// As pbx_launch_fn, with `start` / `stop` stamped by the kernel's own
// dispatch (hipExtModuleLaunchKernel): their elapsed time is the kernel's
// execution, without the queue's gaps before or after it.
int pbx_launch_fn_timed(pbx_ctx *c, hipFunction_t f, const char *name, dim3 grid, dim3 block,
                        void **args, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return PBX_OK;
  hipError_t e = hipExtModuleLaunchKernel(f, grid.x * block.x, grid.y * block.y, grid.z * block.z,
                                          block.x, block.y, block.z, 0,
                                          stream ? stream : c->stream, args, nullptr, start, stop,
                                          0);
  if (e != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "launch of %s failed: %s", name, hipGetErrorString(e));
  return PBX_OK;
}

int pbx_launch(pbx_ctx *c, int kernel, dim3 grid, dim3 block, void **args,
               hipStream_t stream) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return PBX_OK;
  hipError_t e = hipModuleLaunchKernel(c->fn[kernel], grid.x, grid.y, grid.z, block.x,
                                       block.y, block.z, 0, stream ? stream : c->stream,
                                       args, nullptr);
  if (e != hipSuccess)
    return pbx_fail(c, PBX_EHIP, "launch of %s failed: %s", kKernelNames[kernel],
                    hipGetErrorString(e));
  return PBX_OK;
}

// Grow-only scratch buffers owned by the context.
int pbx_ensure_dev(pbx_ctx *c, void **p, size_t *cap, size_t need) {
  if (*cap >= need) return PBX_OK;
  if (*p) {
    HIPCHK(c, hipStreamSynchronize(c->stream));
    hipFree(*p);
    *p = nullptr;
    *cap = 0;
  }
  size_t sz = std::max<size_t>(need, 1 << 16);
  if (hipMalloc(p, sz) != hipSuccess) {
    *p = nullptr;
    return pbx_fail(c, PBX_ENOMEM, "hipMalloc(%zu) failed", sz);
  }
  *cap = sz;
  return PBX_OK;
}

int pbx_ensure_pinned(pbx_ctx *c, void **p, size_t *cap, size_t need) {
  if (*cap >= need) return PBX_OK;
  if (*p) {
    HIPCHK(c, hipStreamSynchronize(c->stream));
    hipHostFree(*p);
    *p = nullptr;
    *cap = 0;
  }
  size_t sz = std::max<size_t>(need, 1 << 16);
  if (hipHostMalloc(p, sz, hipHostMallocDefault) != hipSuccess) {
    *p = nullptr;
    return pbx_fail(c, PBX_ENOMEM, "hipHostMalloc(%zu) failed", sz);
  }
  *cap = sz;
  return PBX_OK;
}

// ---------------------------------------------------------------------------
// Upload: host bytes -> pinned staging (2 x 32 MiB, double buffered) ->
// hipMemcpyAsync -> device staging -> optional repack kernel.
// ---------------------------------------------------------------------------
static const size_t kStageBytes = 32u << 20;

// Copies `bytes` from host to device memory dst through the pinned ring.
static int stage_copy(pbx_ctx *c, void *dst, const void *src, size_t bytes) {
  for (int i = 0; i < 2; ++i) {
    int rc = pbx_ensure_pinned(c, &c->h_stage[i], &c->h_stage_cap[i], kStageBytes);
    if (rc) return rc;
  }
  size_t off = 0;
  int slot = 0;
  while (off < bytes) {
    size_t n = std::min(kStageBytes, bytes - off);
    HIPCHK(c, hipEventSynchronize(c->ev_stage[slot]));
    memcpy(c->h_stage[slot], (const char *)src + off, n);
    HIPCHK(c, hipMemcpyAsync((char *)dst + off, c->h_stage[slot], n, hipMemcpyHostToDevice,
                             c->stream));
    HIPCHK(c, hipEventRecord(c->ev_stage[slot], c->stream));
    off += n;
    slot ^= 1;
  }
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return PBX_OK;
}

// Raw GGUF rows -> planes, chunk by chunk through device staging.
static int stage_repack(pbx_ctx *c, pbx_weight *w, int64_t first_row, int64_t n_rows,
                        const uint8_t *src, int kernel, size_t row_bytes) {
  for (int i = 0; i < 2; ++i) {
    int rc = pbx_ensure_pinned(c, &c->h_stage[i], &c->h_stage_cap[i], kStageBytes);
    if (rc) return rc;
    rc = pbx_ensure_dev(c, &c->d_stage[i], &c->d_stage_cap[i], kStageBytes);
    if (rc) return rc;
  }
  const int64_t rows_per_chunk = std::max<int64_t>(1, (int64_t)(kStageBytes / row_bytes));
  if ((size_t)rows_per_chunk * row_bytes > kStageBytes)
    return pbx_fail(c, PBX_ENOTSUP, "row of %zu bytes exceeds the staging buffer", row_bytes);
  int slot = 0;
  for (int64_t r0 = 0; r0 < n_rows; r0 += rows_per_chunk) {
    const int64_t rows = std::min(rows_per_chunk, n_rows - r0);
    const size_t n = (size_t)rows * row_bytes;
    HIPCHK(c, hipEventSynchronize(c->ev_stage[slot]));
    memcpy(c->h_stage[slot], src + (size_t)r0 * row_bytes, n);
    HIPCHK(c, hipMemcpyAsync(c->d_stage[slot], c->h_stage[slot], n, hipMemcpyHostToDevice,
                             c->stream));
    int B = (int)(kernel == PBX_K_REPACK_Q6_K ? w->K / 256 : w->B);  // blocks per row
    int64_t row0 = first_row + r0, nrows = rows;
    void *raw = c->d_stage[slot];
    void *args[] = {&raw, &w->qs, &w->d, &row0, &nrows, &B};
    void *args_q41[] = {&raw, &w->qs, &w->d, &w->m, &row0, &nrows, &B};
    const int64_t blocks = rows * w->B;
    int rc = pbx_launch(c, kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256),
                        kernel == PBX_K_REPACK_Q4_1 ? args_q41 : args);
    if (rc) return rc;
    HIPCHK(c, hipEventRecord(c->ev_stage[slot], c->stream));
    slot ^= 1;
  }
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return PBX_OK;
}

size_t pbx_type_row_bytes(int type, int64_t K) {
  switch (type) {
    case PBX_TYPE_Q4_0: return (size_t)(K / 32) * 18;
    case PBX_TYPE_Q4_1: return (size_t)(K / 32) * 20;
    case PBX_TYPE_Q8_0: return (size_t)(K / 32) * 34;
    case PBX_TYPE_Q6_K: return (size_t)(K / 256) * 210;
    case PBX_TYPE_F16: return (size_t)K * 2;
    case PBX_TYPE_F32: return (size_t)K * 4;
    default: return 0;
  }
}

static bool weight_ok(const pbx_weight *w) { return w && w->magic == PBX_WEIGHT_MAGIC; }

static bool upload_type(int type) {
  return type == PBX_TYPE_Q4_0 || type == PBX_TYPE_Q4_1 || type == PBX_TYPE_Q8_0 ||
         type == PBX_TYPE_Q6_K || type == PBX_TYPE_F16 || type == PBX_TYPE_F32;
}

static int64_t k_multiple(int type) { return type == PBX_TYPE_Q6_K ? 256 : 32; }

int pbx_weight_alloc(pbx_ctx *c, int type, int64_t N, int64_t K, pbx_weight **out) {
  *out = nullptr;
  if (!upload_type(type))
    return pbx_fail(c, PBX_EINVAL, "unsupported weight type %d", type);
  if (N <= 0 || K <= 0 || K % k_multiple(type) != 0)
    return pbx_fail(c, PBX_EINVAL, "bad shape N=%lld K=%lld (need N>0, K>0, K%%%lld==0)",
                    (long long)N, (long long)K, (long long)k_multiple(type));
  if (N > INT32_MAX || K / 32 > (1 << 20))
    return pbx_fail(c, PBX_ENOTSUP, "shape N=%lld K=%lld too large", (long long)N, (long long)K);
  HIPCHK(c, hipSetDevice(c->device));
  pbx_weight *w = new pbx_weight();
  w->magic = PBX_WEIGHT_MAGIC;
  w->type = type;
  w->N = N;
  w->K = K;
  w->B = K / 32;
  w->Npad = (N + 63) / 64 * 64;
  size_t qs_bytes, d_bytes = 0;
  if (type == PBX_TYPE_F32 || type == PBX_TYPE_F16) {
    qs_bytes = (size_t)w->Npad * K * (type == PBX_TYPE_F32 ? 4 : 2);
  } else if (type == PBX_TYPE_Q6_K) {
    qs_bytes = (size_t)w->Npad * (K / 256) * 208;
    d_bytes = (size_t)w->Npad * (K / 256) * 2;
  } else {
    qs_bytes = (size_t)w->Npad * w->B * (type == PBX_TYPE_Q8_0 ? 32 : 16);
    d_bytes = (size_t)w->Npad * w->B * 2;
    if (type == PBX_TYPE_Q4_1) d_bytes *= 2;  // d plane, then the m plane
  }
  if (hipMalloc(&w->qs, qs_bytes) != hipSuccess) {
    delete w;
    return pbx_fail(c, PBX_ENOMEM, "hipMalloc(%zu) failed", qs_bytes);
  }
  if (d_bytes && hipMalloc(&w->d, d_bytes) != hipSuccess) {
    hipFree(w->qs);
    delete w;
    return pbx_fail(c, PBX_ENOMEM, "hipMalloc(%zu) failed", d_bytes);
  }
  if (type == PBX_TYPE_Q4_1) w->m = (char *)w->d + d_bytes / 2;
  w->bytes = qs_bytes + d_bytes;
  // Pad rows read as zero weights with zero scales.
  if (hipMemsetAsync(w->qs, 0, qs_bytes, c->stream) != hipSuccess ||
      (d_bytes && hipMemsetAsync(w->d, 0, d_bytes, c->stream) != hipSuccess)) {
    hipFree(w->qs);
    if (w->d) hipFree(w->d);
    delete w;
    return pbx_fail(c, PBX_EHIP, "hipMemsetAsync failed");
  }
  *out = w;
  return PBX_OK;
}

void pbx_weight_release(pbx_weight *w) {
  if (!w) return;
  w->magic = 0;
  if (w->qs) hipFree(w->qs);
  if (w->d) hipFree(w->d);
  delete w;
}

int pbx_weight_write_rows(pbx_ctx *c, pbx_weight *w, int64_t row0, int64_t rows,
                          const void *host) {
  if (row0 < 0 || rows <= 0 || row0 + rows > w->N)
    return pbx_fail(c, PBX_EINVAL, "rows [%lld, %lld) outside a weight of %lld rows",
                    (long long)row0, (long long)(row0 + rows), (long long)w->N);
  const size_t row_bytes = pbx_type_row_bytes(w->type, w->K);
  if (w->type == PBX_TYPE_F32 || w->type == PBX_TYPE_F16)
    return stage_copy(c, (char *)w->qs + (size_t)row0 * row_bytes, host, (size_t)rows * row_bytes);
  const int k = w->type == PBX_TYPE_Q4_0   ? PBX_K_REPACK_Q4_0
                : w->type == PBX_TYPE_Q4_1 ? PBX_K_REPACK_Q4_1
                : w->type == PBX_TYPE_Q6_K ? PBX_K_REPACK_Q6_K
                                           : PBX_K_REPACK_Q8_0;
  return stage_repack(c, w, row0, rows, (const uint8_t *)host, k, row_bytes);
}

extern "C" int pbx_weight_upload(pbx_ctx *c, int type, int64_t N, int64_t K,
                                 const void *host, size_t nbytes, pbx_weight **out) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_weight_upload: ctx is NULL");
  if (!out) return pbx_fail(c, PBX_EINVAL, "pbx_weight_upload: out is NULL");
  *out = nullptr;
  if (!upload_type(type))
    return pbx_fail(c, PBX_EINVAL, "pbx_weight_upload: unsupported weight type %d", type);
  if (N <= 0 || K <= 0 || K % k_multiple(type) != 0)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_weight_upload: bad shape N=%lld K=%lld (need N>0, K>0, K%%%lld==0)",
                    (long long)N, (long long)K, (long long)k_multiple(type));
  if (!host) return pbx_fail(c, PBX_EINVAL, "pbx_weight_upload: host buffer is NULL");
  const size_t need = (size_t)N * pbx_type_row_bytes(type, K);
  if (nbytes < need)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_weight_upload: buffer holds %zu bytes, N=%lld x K=%lld needs %zu",
                    nbytes, (long long)N, (long long)K, need);
  pbx_weight *w = nullptr;
  int rc = pbx_weight_alloc(c, type, N, K, &w);
  if (rc) return rc;
  rc = pbx_weight_write_rows(c, w, 0, N, host);
  if (rc) {
    hipStreamSynchronize(c->stream);
    pbx_weight_release(w);
    return rc;
  }
  *out = w;
  return PBX_OK;
}

extern "C" int pbx_weight_upload_q8ref(pbx_ctx *c, int64_t K, int64_t N, const int8_t *q,
                                       const float *scales, int64_t n_scales,
                                       pbx_weight **out) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_weight_upload_q8ref: ctx is NULL");
  if (!out) return pbx_fail(c, PBX_EINVAL, "pbx_weight_upload_q8ref: out is NULL");
  *out = nullptr;
  if (K <= 0 || N <= 0 || !q || !scales)
    return pbx_fail(c, PBX_EINVAL, "pbx_weight_upload_q8ref: bad arguments K=%lld N=%lld",
                    (long long)K, (long long)N);
  if (N > INT32_MAX || K > INT32_MAX)
    return pbx_fail(c, PBX_ENOTSUP, "pbx_weight_upload_q8ref: shape too large");
  const int64_t need_scales = (K * N + 31) / 32;
  if (n_scales < need_scales)
    return pbx_fail(c, PBX_EINVAL,
                    "pbx_weight_upload_q8ref: %lld scales given, [%lld,%lld] needs %lld",
                    (long long)n_scales, (long long)K, (long long)N, (long long)need_scales);
  HIPCHK(c, hipSetDevice(c->device));
  pbx_weight *w = new pbx_weight();
  w->magic = PBX_WEIGHT_MAGIC;
  w->type = PBX_TYPE_Q8_REF;
  w->N = N;
  w->K = K;
  w->B = 0;
  w->Npad = N;
  w->n_scales = need_scales;
  const size_t qb = (size_t)K * N, sb = (size_t)need_scales * 4;
  if (hipMalloc(&w->qs, qb) != hipSuccess || hipMalloc(&w->d, sb) != hipSuccess) {
    if (w->qs) hipFree(w->qs);
    delete w;
    return pbx_fail(c, PBX_ENOMEM, "pbx_weight_upload_q8ref: hipMalloc failed");
  }
  w->bytes = qb + sb;
  int rc = stage_copy(c, w->qs, q, qb);
  if (!rc) rc = stage_copy(c, w->d, scales, sb);
  if (rc) {
    hipFree(w->qs);
    hipFree(w->d);
    delete w;
    return rc;
  }
  *out = w;
  return PBX_OK;
}

extern "C" int pbx_weight_free(pbx_ctx *c, pbx_weight *w) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_weight_free: ctx is NULL");
  if (!w) return PBX_OK;
  if (!weight_ok(w)) return pbx_fail(c, PBX_EINVAL, "pbx_weight_free: not a live weight handle");
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  pbx_weight_release(w);
  return PBX_OK;
}

extern "C" int pbx_weight_info(const pbx_weight *w, int *type, int64_t *N, int64_t *K,
                               size_t *device_bytes) {
  if (!weight_ok(w)) return pbx_fail(nullptr, PBX_EINVAL, "pbx_weight_info: not a live weight handle");
  if (type) *type = w->type;
  if (N) *N = w->N;
  if (K) *K = w->K;
  if (device_bytes) *device_bytes = w->bytes;
  return PBX_OK;
}

// ---------------------------------------------------------------------------
// The instruction.
// ---------------------------------------------------------------------------
int pbx_linear_enqueue(pbx_ctx *c, const pbx_weight *w, const float *dX, int64_t M,
                       const float *dBias, float *dY, hipStream_t stream,
                       const pbx_workspace *ws) {
  if (M > 65535) return pbx_fail(c, PBX_ENOTSUP, "pbx_linear: M=%lld > 65535", (long long)M);
  int N = (int)w->N;
  const unsigned gy = (unsigned)M;
  if (w->type == PBX_TYPE_Q8_REF) {
    int K = (int)w->K;
    void *args[] = {(void *)&w->qs, (void *)&w->d, &dX, &dBias, &dY, &N, &K};
    return pbx_launch(c, PBX_K_GEMV_Q8REF, dim3((unsigned)((N + 63) / 64), gy), dim3(512),
                      args, stream);
  }
  // Q6_K rows stay on the GEMV kernels for every M (one grid row per
  // activation row); the MFMA GEMM covers the other types.
  if (M >= PBX_GEMM_MIN_M && w->type != PBX_TYPE_Q6_K)
    return pbx_gemm_enqueue(c, w, dX, M, dBias, dY, stream, ws);
  int B = (int)w->B;
  // Integer-limb kernels (gemv_int) for Q4_0 / Q8_0 with K = 2048..8192 (not
  // 4097..6144): rows per workgroup by N so the grid keeps >= 256 workgroups
  // where it can, and the tile loop (two workgroups a CU) for tall matrices
  // without a bias.
  if (c->gemv_int && (w->type == PBX_TYPE_Q4_0 || w->type == PBX_TYPE_Q8_0) && B >= 64 &&
      B <= 256 && (B + 63) / 64 != 3) {
    const bool is_q4 = w->type == PBX_TYPE_Q4_0;
    const int ib = (B + 63) / 64;
    int wv = 4, rt = 1, bw = 0, pre = 0;
    bool loop = false;
    if (ib == 1 && N >= 65536 && !dBias) {
      rt = 8;
      loop = true;
    } else if (ib <= 2 && N >= 8192) {
      wv = ib == 1 && is_q4 ? 16 : 8;
      rt = 4;
      if (wv == 16) pre = 2;  // two rows requested before the limb barrier
    } else if (N >= 2048) {
      rt = 2;
      if (ib == 4 && is_q4) bw = 8;  // K = 8192: 8 builder waves
    }
    const std::string name = std::string("pbx_gemv_") + (is_q4 ? "q4_0" : "q8_0") + "_i" +
                             std::to_string(wv) + "x" + std::to_string(rt) + "b" +
                             std::to_string(ib) + (bw ? "w" + std::to_string(bw) : "") +
                             (pre ? "p" + std::to_string(pre) : "") + (loop ? "l" : "");
    hipFunction_t f = pbx_kernel_by_name(c, name);
    if (!f) return pbx_fail(c, PBX_ELOAD, "pbx_linear: kernel %s missing", name.c_str());
    const int tiles = (N + wv * rt - 1) / (wv * rt);
    pbx_gemv_args g{w->qs, w->d, dX, nullptr, nullptr, dBias, dY, nullptr, N, B, 0.f, w->m};
    void *gargs[] = {&g};
    return pbx_launch_fn(c, f, name.c_str(),
                         dim3((unsigned)(loop ? std::min(tiles, 2 * c->cu_count) : tiles), gy),
                         dim3(64 * (wv + bw)), gargs, stream);
  }
  void *args[] = {(void *)&w->qs, (void *)&w->d, (void *)&w->m, &dX, &dBias, &dY, &N, &B};
  const bool q4 = w->type == PBX_TYPE_Q4_0 || w->type == PBX_TYPE_Q4_1;
  if (B <= 32) {
    // Small-K path: 4 waves per workgroup, each wave a tile of P*(64/B) rows.
    const int P = q4 ? 8 : w->type == PBX_TYPE_F32 ? 2 : 4;
    const int T = P * (64 / B);
    const int k = w->type == PBX_TYPE_Q4_0   ? PBX_K_GEMV_Q4_0_SMALL
                  : w->type == PBX_TYPE_Q4_1 ? PBX_K_GEMV_Q4_1_SMALL
                  : w->type == PBX_TYPE_Q8_0 ? PBX_K_GEMV_Q8_0_SMALL
                  : w->type == PBX_TYPE_F16  ? PBX_K_GEMV_F16_SMALL
                  : w->type == PBX_TYPE_Q6_K ? PBX_K_GEMV_Q6_K_SMALL
                                             : PBX_K_GEMV_F32_SMALL;
    return pbx_launch(c, k, dim3((unsigned)((N + 4 * T - 1) / (4 * T)), gy), dim3(256), args,
                      stream);
  }
  const int W = (B + 63) / 64;
  if (W > 8)
    return pbx_fail(c, PBX_ENOTSUP, "pbx_linear: K=%lld exceeds the GEMV limit of 16384",
                    (long long)w->K);
  // Rows per tile: the largest tile that still gives >= 4 workgroups per CU.
  const int target = std::max(4 * c->cu_count, 256);
  int R, k;
  if (q4) {
    const bool q41 = w->type == PBX_TYPE_Q4_1;
    if (N / 16 >= target) { R = 16; k = q41 ? PBX_K_GEMV_Q4_1_WIDE_R16 : PBX_K_GEMV_Q4_0_WIDE_R16; }
    else if (N / 8 >= target) { R = 8; k = q41 ? PBX_K_GEMV_Q4_1_WIDE_R8 : PBX_K_GEMV_Q4_0_WIDE_R8; }
    else { R = 4; k = q41 ? PBX_K_GEMV_Q4_1_WIDE_R4 : PBX_K_GEMV_Q4_0_WIDE_R4; }
  } else if (w->type == PBX_TYPE_Q8_0) {
    if (N / 8 >= target) { R = 8; k = PBX_K_GEMV_Q8_0_WIDE_R8; }
    else { R = 4; k = PBX_K_GEMV_Q8_0_WIDE_R4; }
  } else if (w->type == PBX_TYPE_F16) {
    if (N / 8 >= target) { R = 8; k = PBX_K_GEMV_F16_WIDE_R8; }
    else { R = 4; k = PBX_K_GEMV_F16_WIDE_R4; }
  } else if (w->type == PBX_TYPE_Q6_K) {
    if (N / 8 >= target) { R = 8; k = PBX_K_GEMV_Q6_K_WIDE_R8; }
    else { R = 4; k = PBX_K_GEMV_Q6_K_WIDE_R4; }
  } else {
    if (N / 4 >= target) { R = 4; k = PBX_K_GEMV_F32_WIDE_R4; }
    else { R = 2; k = PBX_K_GEMV_F32_WIDE_R2; }
  }
  return pbx_launch(c, k, dim3((unsigned)((N + R - 1) / R), gy), dim3(64 * W), args, stream);
}

static int check_linear_args(pbx_ctx *c, const pbx_weight *w, const void *X, int64_t M,
                             const void *Y, const char *who) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "%s: ctx is NULL", who);
  if (!weight_ok(w)) return pbx_fail(c, PBX_EINVAL, "%s: not a live weight handle", who);
  if (!X || !Y) return pbx_fail(c, PBX_EINVAL, "%s: X or Y is NULL", who);
  if (M <= 0) return pbx_fail(c, PBX_EINVAL, "%s: M=%lld must be positive", who, (long long)M);
  return PBX_OK;
}

extern "C" int pbx_linear_dev(pbx_ctx *c, const pbx_weight *w, const float *dX, int64_t M,
                              const float *dBias, float *dY) {
  int rc = check_linear_args(c, w, dX, M, dY, "pbx_linear_dev");
  if (rc) return rc;
  HIPCHK(c, hipSetDevice(c->device));
  return pbx_linear_enqueue(c, w, dX, M, dBias, dY, c->stream);
}

extern "C" int pbx_linear_dev_noalloc(pbx_ctx *c, const pbx_weight *w, const float *dX,
                                      int64_t M, const float *dBias, float *dY) {
  int rc = check_linear_args(c, w, dX, M, dY, "pbx_linear_dev_noalloc");
  if (rc) return rc;
  if (!c->scratch)
    return pbx_fail(c, PBX_ENOTSUP, "pbx_linear_dev_noalloc: no device workspace (%s)",
                    c->scratch_err.c_str());
  HIPCHK(c, hipSetDevice(c->device));
  const pbx_workspace ws{c->scratch, c->scratch_bytes};
  return pbx_linear_enqueue(c, w, dX, M, dBias, dY, c->stream, &ws);
}

extern "C" int pbx_workspace_info(const pbx_ctx *c, size_t *grown_bytes, size_t *static_bytes) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_workspace_info: ctx is NULL");
  if (grown_bytes) *grown_bytes = c->d_gemm_cap;
  if (static_bytes) *static_bytes = c->scratch ? c->scratch_bytes : 0;
  return PBX_OK;
}

extern "C" void *pbx_ctx_stream(const pbx_ctx *c) { return c ? (void *)c->stream : nullptr; }

// Coherent pinned memory of at least `need` bytes with a device address.
static int ensure_mapped(pbx_ctx *c, void **h, void **d, size_t *cap, size_t need) {
  if (*cap >= need) return PBX_OK;
  if (*h) {
    HIPCHK(c, hipStreamSynchronize(c->stream));
    hipHostFree(*h);
    *h = *d = nullptr;
    *cap = 0;
  }
  const size_t sz = std::max<size_t>(need, 1 << 16);
  if (hipHostMalloc(h, sz, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
      hipHostGetDevicePointer(d, *h, 0) != hipSuccess) {
    if (*h) hipHostFree(*h);
    *h = *d = nullptr;
    return pbx_fail(c, PBX_ENOMEM, "hipHostMalloc(%zu, mapped) failed", sz);
  }
  *cap = sz;
  return PBX_OK;
}

extern "C" int pbx_linear(pbx_ctx *c, const pbx_weight *w, const float *X, int64_t M,
                          const float *bias, float *Y) {
  int rc = check_linear_args(c, w, X, M, Y, "pbx_linear");
  if (rc) return rc;
  HIPCHK(c, hipSetDevice(c->device));
  const size_t xb = (size_t)M * w->K * 4, yb = (size_t)M * w->N * 4;
  const size_t bb = bias ? (size_t)w->N * 4 : 0;
  // M < 4 (the GEMVs): x and the bias are read from coherent pinned memory
  // by a copy kernel and y goes straight into coherent pinned memory, so a
  // call is two launches and a synchronisation, no copy operation (the
  // synchronous per-matmul seam of llama-streaming.js pays each operation's
  // latency on every call: 24.3 us a call with the three copies)
  const bool direct = M < PBX_GEMM_MIN_M && w->type != PBX_TYPE_Q8_REF;
  // the bias follows x (whole 128-byte blocks) in 16-byte units
  const size_t bpad = (bb + 15) / 16 * 16;
  if ((rc = pbx_ensure_dev(c, &c->d_x, &c->d_x_cap, xb + bpad))) return rc;
  if (bias && (rc = pbx_ensure_dev(c, &c->d_b, &c->d_b_cap, bb))) return rc;
  if (direct) {
    if ((rc = ensure_mapped(c, &c->h_x, &c->d_hx, &c->h_x_cap, xb + bpad)) ||
        (rc = ensure_mapped(c, &c->h_y, &c->d_hy, &c->h_y_cap, yb)))
      return rc;
    memcpy(c->h_x, X, xb);
    if (bias) memcpy((char *)c->h_x + xb, bias, bb);
    const void *src = c->d_hx;
    void *dst = c->d_x;
    const int64_t n16 = (int64_t)(xb + bpad) / 16;
    void *args[] = {(void *)&src, &dst, (void *)&n16};
    if ((rc = pbx_launch(c, PBX_K_COPY16, dim3((unsigned)((n16 + 255) / 256)), dim3(256), args)))
      return rc;
    if ((rc = pbx_linear_enqueue(c, w, (const float *)c->d_x, M,
                                 bias ? (const float *)((char *)c->d_x + xb) : nullptr,
                                 (float *)c->d_hy, c->stream)))
      return rc;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    memcpy(Y, c->h_y, yb);
    return PBX_OK;
  }
  if ((rc = pbx_ensure_dev(c, &c->d_y, &c->d_y_cap, yb))) return rc;
  if ((rc = pbx_ensure_pinned(c, &c->h_io, &c->h_io_cap, std::max(xb + bb, yb)))) return rc;
  memcpy(c->h_io, X, xb);
  if (bias) memcpy((char *)c->h_io + xb, bias, bb);
  HIPCHK(c, hipMemcpyAsync(c->d_x, c->h_io, xb, hipMemcpyHostToDevice, c->stream));
  if (bias)
    HIPCHK(c, hipMemcpyAsync(c->d_b, (char *)c->h_io + xb, bb, hipMemcpyHostToDevice, c->stream));
  if ((rc = pbx_linear_enqueue(c, w, (const float *)c->d_x, M,
                               bias ? (const float *)c->d_b : nullptr, (float *)c->d_y,
                               c->stream)))
    return rc;
  HIPCHK(c, hipMemcpyAsync(c->h_io, c->d_y, yb, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  memcpy(Y, c->h_io, yb);
  return PBX_OK;
}

extern "C" int pbx_dequant_dev(pbx_ctx *c, const pbx_weight *w, float *dY) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_dequant_dev: ctx is NULL");
  if (!weight_ok(w)) return pbx_fail(c, PBX_EINVAL, "pbx_dequant_dev: not a live weight handle");
  if (!dY) return pbx_fail(c, PBX_EINVAL, "pbx_dequant_dev: output is NULL");
  HIPCHK(c, hipSetDevice(c->device));
  if (w->type == PBX_TYPE_F32) {
    HIPCHK(c, hipMemcpyAsync(dY, w->qs, (size_t)w->N * w->K * 4, hipMemcpyDeviceToDevice,
                             c->stream));
    return PBX_OK;
  }
  if (w->type == PBX_TYPE_Q8_REF) {
    int64_t n = w->N * w->K;
    void *args[] = {(void *)&w->qs, (void *)&w->d, &dY, &n};
    return pbx_launch(c, PBX_K_DEQUANT_Q8REF, dim3((unsigned)((n + 255) / 256)), dim3(256), args);
  }
  int N = (int)w->N, B = (int)w->B;
  const int64_t blocks = (int64_t)N * B;
  if (w->type == PBX_TYPE_Q4_1) {
    void *args[] = {(void *)&w->qs, (void *)&w->d, (void *)&w->m, &dY, &N, &B};
    return pbx_launch(c, PBX_K_DEQUANT_Q4_1, dim3((unsigned)((blocks + 255) / 256)), dim3(256),
                      args);
  }
  if (w->type == PBX_TYPE_F16) {
    int64_t n = w->N * w->K;
    void *args[] = {(void *)&w->qs, &dY, &n};
    return pbx_launch(c, PBX_K_DEQUANT_F16, dim3((unsigned)((n + 255) / 256)), dim3(256), args);
  }
  if (w->type == PBX_TYPE_Q6_K) {
    int SB = (int)(w->K / 256);
    void *args[] = {(void *)&w->qs, (void *)&w->d, &dY, &N, &SB};
    return pbx_launch(c, PBX_K_DEQUANT_Q6_K, dim3((unsigned)((blocks + 255) / 256)), dim3(256),
                      args);
  }
  void *args[] = {(void *)&w->qs, (void *)&w->d, &dY, &N, &B};
  return pbx_launch(c, w->type == PBX_TYPE_Q4_0 ? PBX_K_DEQUANT_Q4_0 : PBX_K_DEQUANT_Q8_0,
                    dim3((unsigned)((blocks + 255) / 256)), dim3(256), args);
}

extern "C" int pbx_dequant(pbx_ctx *c, const pbx_weight *w, float *Y) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_dequant: ctx is NULL");
  if (!weight_ok(w)) return pbx_fail(c, PBX_EINVAL, "pbx_dequant: not a live weight handle");
  if (!Y) return pbx_fail(c, PBX_EINVAL, "pbx_dequant: output is NULL");
  HIPCHK(c, hipSetDevice(c->device));
  const size_t bytes = (size_t)w->N * w->K * 4;
  void *d = nullptr;
  if (hipMalloc(&d, bytes) != hipSuccess)
    return pbx_fail(c, PBX_ENOMEM, "pbx_dequant: hipMalloc(%zu) failed", bytes);
  int rc = pbx_dequant_dev(c, w, (float *)d);
  if (!rc && hipMemcpyAsync(Y, d, bytes, hipMemcpyDeviceToHost, c->stream) != hipSuccess)
    rc = pbx_fail(c, PBX_EHIP, "pbx_dequant: copy back failed");
  if (!rc && hipStreamSynchronize(c->stream) != hipSuccess)
    rc = pbx_fail(c, PBX_EHIP, "pbx_dequant: synchronize failed");
  hipFree(d);
  return rc;
}

// ---------------------------------------------------------------------------
// Device memory, timing.
// ---------------------------------------------------------------------------
extern "C" int pbx_dev_alloc(pbx_ctx *c, size_t bytes, void **out) {
  if (!c || !out) return pbx_fail(c, PBX_EINVAL, "pbx_dev_alloc: NULL argument");
  *out = nullptr;
  HIPCHK(c, hipSetDevice(c->device));
  if (hipMalloc(out, bytes ? bytes : 1) != hipSuccess) {
    *out = nullptr;
    return pbx_fail(c, PBX_ENOMEM, "pbx_dev_alloc: hipMalloc(%zu) failed", bytes);
  }
  return PBX_OK;
}

extern "C" int pbx_dev_free(pbx_ctx *c, void *p) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_dev_free: ctx is NULL");
  if (!p) return PBX_OK;
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipFree(p));
  return PBX_OK;
}

extern "C" int pbx_memcpy_h2d(pbx_ctx *c, void *dst, const void *src, size_t bytes) {
  if (!c || !dst || !src) return pbx_fail(c, PBX_EINVAL, "pbx_memcpy_h2d: NULL argument");
  HIPCHK(c, hipSetDevice(c->device));
  return stage_copy(c, dst, src, bytes);
}

extern "C" int pbx_memcpy_d2h(pbx_ctx *c, void *dst, const void *src, size_t bytes) {
  if (!c || !dst || !src) return pbx_fail(c, PBX_EINVAL, "pbx_memcpy_d2h: NULL argument");
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return PBX_OK;
}

extern "C" int pbx_memset_dev(pbx_ctx *c, void *dst, int value, size_t bytes) {
  if (!c || !dst) return pbx_fail(c, PBX_EINVAL, "pbx_memset_dev: NULL argument");
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipMemsetAsync(dst, value, bytes, c->stream));
  return PBX_OK;
}

extern "C" int pbx_dev_copy(pbx_ctx *c, void *dst, const void *src, size_t bytes) {
  if (!c || !dst || !src) return pbx_fail(c, PBX_EINVAL, "pbx_dev_copy: NULL argument");
  if (bytes % 16 || ((uintptr_t)dst | (uintptr_t)src) % 16)
    return pbx_fail(c, PBX_EINVAL, "pbx_dev_copy: size and addresses must be 16-byte aligned");
  HIPCHK(c, hipSetDevice(c->device));
  int64_t n16 = (int64_t)(bytes / 16);
  const unsigned grid = (unsigned)std::min<int64_t>((n16 + 255) / 256, 4 * 1024);
  void *args[] = {(void *)&src, &dst, &n16};
  return pbx_launch(c, PBX_K_COPY16, dim3(grid ? grid : 1), dim3(256), args);
}

extern "C" int pbx_sync(pbx_ctx *c) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_sync: ctx is NULL");
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return PBX_OK;
}

extern "C" int pbx_timer_start(pbx_ctx *c) {
  if (!c) return pbx_fail(nullptr, PBX_EINVAL, "pbx_timer_start: ctx is NULL");
  HIPCHK(c, hipEventRecord(c->ev0, c->stream));
  return PBX_OK;
}

extern "C" int pbx_timer_stop(pbx_ctx *c, double *ms) {
  if (!c || !ms) return pbx_fail(c, PBX_EINVAL, "pbx_timer_stop: NULL argument");
  HIPCHK(c, hipEventRecord(c->ev1, c->stream));
  HIPCHK(c, hipEventSynchronize(c->ev1));
  float f = 0.f;
  HIPCHK(c, hipEventElapsedTime(&f, c->ev0, c->ev1));
  *ms = f;
  return PBX_OK;
}

extern "C" int pbx_bench_linear(pbx_ctx *c, int n_ops, const pbx_weight *const *W,
                                const float *const *dX, float *const *dY, int64_t M, int reps,
                                double *ms) {
  if (!c || !W || !dX || !dY || !ms || n_ops <= 0 || reps <= 0 || M <= 0)
    return pbx_fail(c, PBX_EINVAL, "pbx_bench_linear: bad arguments");
  for (int i = 0; i < n_ops; ++i)
    if (!weight_ok(W[i]) || !dX[i] || !dY[i])
      return pbx_fail(c, PBX_EINVAL, "pbx_bench_linear: bad operand %d", i);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipEventRecord(c->ev0, c->stream));
  for (int r = 0; r < reps; ++r)
    for (int i = 0; i < n_ops; ++i) {
      int rc = pbx_linear_enqueue(c, W[i], dX[i], M, nullptr, dY[i], c->stream);
      if (rc) return rc;
    }
  return pbx_timer_stop(c, ms);
}

extern "C" int pbx_bench_linear_graph(pbx_ctx *c, int n_ops, const pbx_weight *const *W,
                                      const float *const *dX, float *const *dY, int64_t M,
                                      int reps, double *ms) {
  if (!c || !W || !dX || !dY || !ms || n_ops <= 0 || reps <= 0 || M <= 0 || M >= PBX_GEMM_MIN_M)
    return pbx_fail(c, PBX_EINVAL, "pbx_bench_linear_graph: bad arguments (M < %d)",
                    PBX_GEMM_MIN_M);
  for (int i = 0; i < n_ops; ++i)
    if (!weight_ok(W[i]) || !dX[i] || !dY[i])
      return pbx_fail(c, PBX_EINVAL, "pbx_bench_linear_graph: bad operand %d", i);
  HIPCHK(c, hipSetDevice(c->device));
  hipStream_t s = c->stream;
  HIPCHK(c, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  int rc = PBX_OK;
  for (int i = 0; i < n_ops && !rc; ++i) rc = pbx_linear_enqueue(c, W[i], dX[i], M, nullptr, dY[i], s);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(s, &g);
  if (rc || e != hipSuccess || !g) {
    if (g) hipGraphDestroy(g);
    return rc ? rc : pbx_fail(c, PBX_EHIP, "pbx_bench_linear_graph: capture failed");
  }
  hipGraphExec_t x = nullptr;
  if (hipGraphInstantiate(&x, g, nullptr, nullptr, 0) != hipSuccess) {
    hipGraphDestroy(g);
    return pbx_fail(c, PBX_EHIP, "pbx_bench_linear_graph: instantiate failed");
  }
  if (hipGraphLaunch(x, s) != hipSuccess) rc = pbx_fail(c, PBX_EHIP, "graph launch failed");
  if (!rc && hipEventRecord(c->ev0, s) != hipSuccess) rc = pbx_fail(c, PBX_EHIP, "event failed");
  for (int r = 0; r < reps && !rc; ++r)
    if (hipGraphLaunch(x, s) != hipSuccess) rc = pbx_fail(c, PBX_EHIP, "graph launch failed");
  if (!rc) rc = pbx_timer_stop(c, ms);
  hipStreamSynchronize(s);
  hipGraphExecDestroy(x);
  hipGraphDestroy(g);
  return rc;
}
