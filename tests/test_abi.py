"""The C ABI library loads and exports what include/pbx.h declares; its
host-side argument checks and quantisers work without a GPU."""
import ctypes
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import purebee_amd as pb
from purebee_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_entry_points():
    names = set()
    for f in os.listdir(os.path.join(ROOT, "include")):
        if f.endswith(".h"):
            src = open(os.path.join(ROOT, "include", f)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names |= set(re.findall(r"\b(pbx_[a-z0-9_]+)\s*\(", src))
    return names


def test_library_exports_every_declared_symbol():
    L = native.load_library()
    declared = declared_entry_points()
    assert "pbx_linear" in declared and "pbx_weight_upload" in declared
    missing = [n for n in sorted(declared) if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding covers the same set
    assert declared == set(native.EXPORTS), declared ^ set(native.EXPORTS)


def test_code_objects_are_gfx950():
    lib = os.path.join(ROOT, "purebee_amd", "lib")
    cos = [f for f in os.listdir(lib) if f.endswith(".hsaco")]
    assert cos
    for f in cos:
        blob = open(os.path.join(lib, f), "rb").read()
        # hipcc --genco writes a clang offload bundle around the gfx950 ELF
        assert blob[:4] == b"\x7fELF" or blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
        assert b"amdgcn-amd-amdhsa--gfx950" in blob


def test_null_context_errors_are_reported():
    L = native.load_library()
    w = ctypes.c_void_p()
    rc = L.pbx_weight_upload(None, 2, 32, 32, None, 0, ctypes.byref(w))
    assert rc == -1
    assert b"ctx is NULL" in L.pbx_last_error(None)
    assert L.pbx_linear(None, None, None, 1, None, None) == -1
    assert L.pbx_init(0, None) == -1


def test_init_without_device_fails_cleanly():
    # In a container without a GPU pbx_init must fail with a status, not crash.
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK):
        pytest.skip("a GPU is present")
    with pytest.raises(pb.PbxError) as ei:
        pb.Context(0)
    assert ei.value.code in (-2, -4, -6)


def test_quantiser_argument_validation():
    L = native.load_library()
    w = np.zeros((2, 33), np.float32)
    out = np.zeros(10, np.uint8)
    assert L.pbx_quantize_q4_0(w, 2, 33, out) == -1   # K % 32 != 0
    assert b"K=33" in L.pbx_last_error(None)
    with pytest.raises(pb.PbxError):
        pb.quantize_q8_0(np.zeros((2, 40), np.float32))


@pytest.mark.skipif(shutil.which("node") is None, reason="node not installed")
def test_napi_addon_loads_and_exports():
    addon = os.path.join(ROOT, "purebee_amd", "lib", "pbx_napi.node")
    assert os.path.exists(addon), "N-API addon not built"
    js = (f"const a = require({addon!r});"
          "console.log(JSON.stringify(Object.keys(a).sort()));")
    r = subprocess.run(["node", "-e", js], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    keys = set(__import__("json").loads(r.stdout))
    for k in ("init", "upload", "linear", "dequant", "free", "deviceInfo", "modelCreate",
              "modelSetTensor", "modelForward", "modelForwardBatch", "modelGenerate",
              "modelRollback", "modelReset", "modelFree", "speculative", "modelLoadGGUF"):
        assert k in keys, keys


@pytest.mark.skipif(shutil.which("node") is None, reason="node not installed")
def test_js_module_reports_missing_gpu_as_error():
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK):
        pytest.skip("a GPU is present")
    mod = os.path.join(ROOT, "purebee_amd", "js", "hip-q4.js")
    js = (f"const q = require({mod!r});"
          "const ok = q.init(); console.log(JSON.stringify({ok, supported: q.supported}));"
          "try { q.q4_0_matvec(new Float32Array(32), new Uint8Array(18), 1, 32); console.log('nothrow'); }"
          "catch (e) { console.log('threw:' + e.message); }")
    r = subprocess.run(["node", "-e", js], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.strip().splitlines()
    assert '"ok":false' in lines[-2]
    assert lines[-1].startswith("threw:")
