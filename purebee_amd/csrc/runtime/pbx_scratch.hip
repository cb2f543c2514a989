// pbx_scratch.hip -- the device workspace of pbx_linear_dev_noalloc.
//
// A file-scope device array, one copy per GPU: the HIP runtime places it when
// this library's code object is loaded on a device and keeps it until the
// process ends, so the no-allocation entry point never calls hipMalloc.  The
// array's name is only a host-side stand-in: pbx_scratch_lookup asks the
// runtime for each device's own address, and every launch path passes that
// address to its kernels.  Calls that use it on one GPU share its contents
// (each call rewrites what it reads before reading it), so calls that overlap
// on one GPU race.

#include <hip/hip_runtime.h>

#include "pbx_internal.h"

static __device__ __align__(256) unsigned char scratch[PBX_SCRATCH_BYTES];

// Called once per context with its device current (pbx_init).
int pbx_scratch_lookup(pbx_ctx *c) {
  void *ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr) {
    (void)hipGetLastError();
    c->scratch = nullptr;
    c->scratch_bytes = 0;
    c->scratch_err = std::string("hipGetSymbolAddress failed: ") + hipGetErrorString(e);
    return PBX_EHIP;
  }
  c->scratch = ptr;
  c->scratch_bytes = PBX_SCRATCH_BYTES;
  return PBX_OK;
}
