"""The GGUF reader (purebee_amd/csrc/runtime/pbx_gguf.cpp) under host
AddressSanitizer + UBSan: thousands of truncated and corrupted files must be
rejected or parsed without a single out-of-bounds access, overflow or leak
of control.  CPU only: the reader is host code."""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

from tests import gguf_writer as gw
from tests.test_gguf import ALL_VALUES, small_tensors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def build_driver(out):
    cmd = ["g++", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROOT, "purebee_amd", "csrc", "runtime"), "-I", "/opt/rocm/include",
           os.path.join(ROOT, "purebee_amd", "csrc", "runtime", "pbx_gguf.cpp"),
           os.path.join(ROOT, "tests", "gguf_fuzz_main.cpp"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]


def corpus(tmp, seed=0):
    rng = np.random.default_rng(seed)
    cfg = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2)
    kv = gw.llama_kv(cfg, n_tokens=20) + list(ALL_VALUES)
    blob, _ = gw.build(kv, small_tensors())
    files = []

    def add(data):
        p = os.path.join(tmp, f"f{len(files)}.gguf")
        with open(p, "wb") as f:
            f.write(bytes(data))
        files.append(p)

    add(blob)
    for cut in range(0, len(blob), max(1, len(blob) // 400)):
        add(blob[:cut])
    # random byte flips
    for _ in range(600):
        b = bytearray(blob)
        for _ in range(int(rng.integers(1, 8))):
            b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
        add(b)
    # every 8-byte field of the header region set to extreme values
    head_end = min(len(blob), 1200)
    for off in range(8, head_end - 8, 4):
        for v in (0xFFFFFFFFFFFFFFFF, 0x7FFFFFFFFFFFFFFF, 1 << 40, 0):
            b = bytearray(blob)
            b[off:off + 8] = struct.pack("<Q", v)
            add(b)
    return files


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_reader_under_asan(tmp_path):
    exe = str(tmp_path / "fuzz")
    build_driver(exe)
    files = corpus(str(tmp_path))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    # in chunks, to stay under the argument-length limit
    opened = 0
    for i in range(0, len(files), 500):
        r = subprocess.run([exe] + files[i:i + 500], capture_output=True, text=True, env=env,
                           timeout=300)
        assert r.returncode == 0, (r.stdout[-500:], r.stderr[-4000:])
        assert "Sanitizer" not in r.stderr, r.stderr[-4000:]
        opened += int(r.stdout.split("opened ")[1].split()[0])
    assert opened >= 1   # the intact file (and harmless flips) parse
