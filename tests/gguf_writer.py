"""A small GGUF v2/v3 writer for test fixtures.

Written from the file format as the reference reads it (gguf.js:76-194,
streaming-loader.js:35-87): little-endian; header (magic "GGUF", u32
version, u64 tensor count, u64 kv count); kv pairs (string key, u32 value
type, value); tensor infos (string name, u32 n_dims, u64 dims, u32 ggml
type, u64 offset into the data section); the data section at the end of the
tensor table rounded up to general.alignment (default 32), each tensor's
data at an offset that is a multiple of the alignment.  Strings are u64
length + UTF-8 bytes; arrays are u32 element type + u64 count + elements.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def encode_value(vtype, value):
    if vtype == STR:
        return _str(value)
    if vtype == ARR:
        etype, items = value
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(encode_value(etype, v) for v in items)
    return struct.pack(_FMT[vtype], value)


def build(kv, tensors, version=3, alignment=32, header_version=None):
    """kv: [(key, vtype, value)]; tensors: [(name, dims, ggml_type, bytes)].
    Returns the file bytes and each tensor's absolute data offset."""
    head = struct.pack("<4sIQQ", b"GGUF", header_version or version, len(tensors), len(kv))
    for key, vtype, value in kv:
        head += _str(key) + struct.pack("<I", vtype) + encode_value(vtype, value)
    rel, off = [], 0
    for _, _, _, data in tensors:
        rel.append(off)
        off += np.asarray(data).nbytes
        off = (off + alignment - 1) // alignment * alignment
    for (name, dims, ttype, _), r in zip(tensors, rel):
        head += _str(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ttype, r)
    start = (len(head) + alignment - 1) // alignment * alignment
    blob = bytearray(head) + bytes(start - len(head))
    for (_, _, _, data), r in zip(tensors, rel):
        blob += bytes(start + r - len(blob))
        blob += bytes(np.ascontiguousarray(data).view(np.uint8).ravel())
    return bytes(blob), [start + r for r in rel]


def write(path, kv, tensors, **kw):
    blob, offsets = build(kv, tensors, **kw)
    with open(path, "wb") as f:
        f.write(blob)
    return offsets


def llama_kv(cfg, n_tokens=None, arch="llama", extra=()):
    """Metadata of a Llama-family model as llama.cpp writes it."""
    p = arch + "."
    kv = [("general.architecture", STR, arch), ("general.name", STR, "synthetic"),
          (p + "embedding_length", U32, cfg["dim"]), (p + "feed_forward_length", U32, cfg["hidden_dim"]),
          (p + "block_count", U32, cfg["n_layers"]), (p + "attention.head_count", U32, cfg["n_heads"]),
          (p + "attention.head_count_kv", U32, cfg["n_kv_heads"]),
          (p + "context_length", U32, cfg.get("context_length", 2048)),
          (p + "attention.layer_norm_rms_epsilon", F32, cfg.get("rms_eps", 1e-5)),
          (p + "rope.freq_base", F32, cfg.get("rope_theta", 10000.0))]
    if n_tokens:
        kv.append(("tokenizer.ggml.model", STR, "gpt2"))
        kv.append(("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(n_tokens)])))
    return kv + list(extra)
