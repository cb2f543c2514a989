"""Build recipe for the native parts of purebee_amd.

* ``csrc/kernels/*.hip``  -> ``lib/<name>.hsaco``  (hipcc --genco, gfx950 only)
* ``csrc/runtime/*.cpp``  -> ``lib/libpbhip.so``   (the C ABI of include/pbx.h)
* ``napi/pbx_napi.cc``    -> ``lib/pbx_napi.node`` (N-API addon for Node.js)

Everything is built in-tree so the built files travel with the source tree.
Run ``python -m purebee_amd.build`` or call :func:`build`.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# Packed-FP32 VALU forms are kept out of every code object.
HIP_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Per-file additions: the GEMM keeps MFMA accumulators in VGPRs, so the
# per-block scale FMAs read them without v_accvgpr moves.
KERNEL_FLAGS = {"pbx_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
HOST_FLAGS = ["-O2", "-g", "-fPIC", "-std=c++17", "-Wall", "-Wextra", "-Wno-unused-parameter",
              "-D__HIP_PLATFORM_AMD__"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}")
    return r.stdout


def kernel_sources():
    kdir = os.path.join(PKG, "csrc", "kernels")
    return sorted(os.path.join(kdir, f) for f in os.listdir(kdir) if f.endswith(".hip"))


def build_kernels(verbose=False):
    os.makedirs(LIB, exist_ok=True)

    def one(src):
        out = os.path.join(LIB, os.path.basename(src)[:-4] + ".hsaco")
        tmp = out + ".tmp"
        extra = KERNEL_FLAGS.get(os.path.basename(src), [])
        _run([HIPCC, "--genco", *HIP_FLAGS, *extra, src, "-o", tmp], verbose)
        os.replace(tmp, out)
        return out

    with ThreadPoolExecutor(max_workers=4) as ex:
        return list(ex.map(one, kernel_sources()))


def build_runtime(verbose=False):
    os.makedirs(LIB, exist_ok=True)
    rdir = os.path.join(PKG, "csrc", "runtime")
    srcs = sorted(os.path.join(rdir, f) for f in os.listdir(rdir) if f.endswith(".cpp"))
    incs = ["-I", os.path.join(ROOT, "include"), "-I", rdir]
    # runtime files with device code (the static workspace array): compiled by
    # hipcc for gfx950 into objects linked into the library
    objs = []
    for f in sorted(os.listdir(rdir)):
        if f.endswith(".hip"):
            obj = os.path.join(LIB, f[:-4] + ".o")
            _run([HIPCC, "-c", "-fPIC", *HIP_FLAGS, *incs, os.path.join(rdir, f), "-o", obj],
                 verbose)
            objs.append(obj)
    out = os.path.join(LIB, "libpbhip.so")
    tmp = out + ".tmp"
    _run(["g++", *HOST_FLAGS, "-shared", "-fopenmp",
          *incs, "-I", os.path.join(ROCM, "include"),
          *srcs, *objs, "-o", tmp,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib",
          "-Wl,--no-undefined"], verbose)
    os.replace(tmp, out)
    return out


def node_include_dir():
    for d in ("/usr/include/node", "/usr/local/include/node"):
        if os.path.exists(os.path.join(d, "node_api.h")):
            return d
    return None


def build_napi(verbose=False):
    inc = node_include_dir()
    if inc is None:
        if verbose:
            print("node_api.h not found: N-API addon skipped", flush=True)
        return None
    src = os.path.join(PKG, "napi", "pbx_napi.cc")
    out = os.path.join(LIB, "pbx_napi.node")
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-fPIC", "-std=c++17", "-Wall", "-shared", "-DNAPI_VERSION=3",
          "-I", inc, "-I", os.path.join(ROOT, "include"), src, "-o", tmp,
          "-L", LIB, "-lpbhip", "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, out)
    return out


def build(verbose=False):
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    outs = build_kernels(verbose)
    outs.append(build_runtime(verbose))
    napi = build_napi(verbose)
    if napi:
        outs.append(napi)
    return outs


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print(p)
