"""Seeded synthetic Llama-family models: the random-init workloads.

Every weight matrix is drawn from N(0, 0.02) with its own seed
(base + tensor index), quantised with the host quantisers of the C ABI
(pbx_quantize_q4_0 / pbx_quantize_q4_1 / pbx_quantize_q8_0) into GGUF blocks; norm weights are
1.0 (f32, as GGUF stores them).  Shapes follow the GGUF tensors the reference
loads (gguf.js:378-410): matrices are [out_features, in_features].
"""
import numpy as np

from . import native
from .native import (Model, TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q6_K, TYPE_Q8_0,
                     T_TOKEN_EMBD, T_OUTPUT,
                     T_OUTPUT_NORM, T_ATTN_NORM, T_FFN_NORM, T_ATTN_Q, T_ATTN_K, T_ATTN_V,
                     T_ATTN_OUTPUT, T_FFN_GATE, T_FFN_UP, T_FFN_DOWN)

# The three model shapes of the workloads.
CONFIGS = {
    # stories15M (llama2.c): MHA, f32 embedding/LM head, Q8_0 layer matrices
    "stories15m": dict(dim=288, hidden_dim=768, n_layers=6, n_heads=6, n_kv_heads=6,
                       vocab_size=32000, max_seq=256, weight_type=TYPE_Q8_0,
                       embed_type=TYPE_F32, rope_theta=10000.0),
    # SmolLM2-135M: GQA 9/3, tied Q8_0 embedding
    "smollm2_135m": dict(dim=576, hidden_dim=1536, n_layers=30, n_heads=9, n_kv_heads=3,
                         vocab_size=49152, max_seq=512, weight_type=TYPE_Q8_0,
                         embed_type=TYPE_Q8_0, rope_theta=10000.0),
    # Llama-3.2-1B: GQA 32/8, head_dim 64, tied Q4_0 embedding, theta 5e5
    "llama32_1b": dict(dim=2048, hidden_dim=8192, n_layers=16, n_heads=32, n_kv_heads=8,
                       vocab_size=128256, max_seq=1024, weight_type=TYPE_Q4_0,
                       embed_type=TYPE_Q4_0, rope_theta=500000.0),
}

WEIGHT_STD = 0.02


def tensor_specs(cfg):
    """(tensor id, layer, N, K, type) of every tensor, in upload order."""
    d, h = cfg["dim"], cfg["hidden_dim"]
    hd = cfg.get("head_dim") or d // cfg["n_heads"]
    kv = cfg["n_kv_heads"] * hd
    wt = cfg["weight_type"]
    specs = [(T_TOKEN_EMBD, -1, cfg["vocab_size"], d, cfg["embed_type"]),
             (T_OUTPUT_NORM, -1, 1, d, TYPE_F32)]
    if cfg.get("output_type", -1) >= 0:
        specs.append((T_OUTPUT, -1, cfg["vocab_size"], d, cfg["output_type"]))
    for l in range(cfg["n_layers"]):
        specs += [(T_ATTN_NORM, l, 1, d, TYPE_F32), (T_FFN_NORM, l, 1, d, TYPE_F32),
                  (T_ATTN_Q, l, d, d, wt), (T_ATTN_K, l, kv, d, wt), (T_ATTN_V, l, kv, d, wt),
                  (T_ATTN_OUTPUT, l, d, d, wt), (T_FFN_GATE, l, h, d, wt),
                  (T_FFN_UP, l, h, d, wt), (T_FFN_DOWN, l, d, h, wt)]
    return specs


def make_tensor(spec, base_seed, index, std=WEIGHT_STD):
    """Bytes of one tensor as the loaders hand them over (GGUF blocks or f32);
    matrices are drawn from N(0, std)."""
    tid, layer, N, K, t = spec
    if tid in (T_OUTPUT_NORM, T_ATTN_NORM, T_FFN_NORM):
        return np.ones(K, np.float32)
    w = native.synth_normal(base_seed + index, N * K, 0.0, std).reshape(N, K)
    if t == TYPE_F32:
        return w
    return {TYPE_Q4_0: native.quantize_q4_0, TYPE_Q4_1: native.quantize_q4_1,
            TYPE_Q8_0: native.quantize_q8_0, TYPE_Q6_K: native.quantize_q6_k,
            TYPE_F16: native.to_f16_bytes}[t](w)


def build(ctx, cfg, seed=1000, keep=None):
    """Create a Model of config `cfg` (a CONFIGS key or a dict; "weight_std"
    overrides the 0.02 of the matrices) and load seeded weights;
    keep(spec, data) sees every tensor (for oracles / CPU baselines)."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    m = Model(ctx, cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["n_heads"],
              cfg["n_kv_heads"], cfg["vocab_size"], cfg["max_seq"], cfg["weight_type"],
              cfg["embed_type"], cfg.get("output_type", -1), cfg.get("head_dim"),
              cfg.get("rms_eps", 1e-5), cfg.get("rope_theta", 10000.0))
    std = cfg.get("weight_std", WEIGHT_STD)
    for i, spec in enumerate(tensor_specs(cfg)):
        data = make_tensor(spec, seed, i, std)
        m.set_tensor(spec[0], spec[1], data)
        if keep is not None:
            keep(spec, data)
    return m


def random_tokens(seed, n, vocab):
    """Uniform token ids in [0, vocab) from the seeded stream."""
    u = native.synth_normal(seed, n)
    # map the normal draws through their CDF-free rank: a fixed hash of the bits
    bits = u.view(np.uint32).astype(np.uint64)
    return ((bits * np.uint64(2654435761)) % np.uint64(vocab)).astype(np.int32)


# GGUF tensor names of the tensor ids (gguf.js:378-410).
GGUF_NAMES = {T_TOKEN_EMBD: "token_embd.weight", T_OUTPUT: "output.weight",
              T_OUTPUT_NORM: "output_norm.weight", T_ATTN_NORM: "attn_norm.weight",
              T_FFN_NORM: "ffn_norm.weight", T_ATTN_Q: "attn_q.weight",
              T_ATTN_K: "attn_k.weight", T_ATTN_V: "attn_v.weight",
              T_ATTN_OUTPUT: "attn_output.weight", T_FFN_GATE: "ffn_gate.weight",
              T_FFN_UP: "ffn_up.weight", T_FFN_DOWN: "ffn_down.weight"}


def write_gguf(path, cfg, seed=1000, alignment=32):
    """Write the seeded model of `cfg` as a GGUF v3 file (llama metadata,
    the tensors of tensor_specs in their types) for the file -> device
    path; returns the file size.  Tensor data is streamed, one tensor in
    memory at a time."""
    import struct
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    specs = tensor_specs(cfg)

    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    kv = [("general.architecture", 8, s("llama")),
          ("llama.embedding_length", 4, struct.pack("<I", cfg["dim"])),
          ("llama.feed_forward_length", 4, struct.pack("<I", cfg["hidden_dim"])),
          ("llama.block_count", 4, struct.pack("<I", cfg["n_layers"])),
          ("llama.attention.head_count", 4, struct.pack("<I", cfg["n_heads"])),
          ("llama.attention.head_count_kv", 4, struct.pack("<I", cfg["n_kv_heads"])),
          ("llama.context_length", 4, struct.pack("<I", cfg["max_seq"])),
          ("llama.attention.layer_norm_rms_epsilon", 6, struct.pack("<f", cfg.get("rms_eps", 1e-5))),
          ("llama.rope.freq_base", 6, struct.pack("<f", cfg.get("rope_theta", 10000.0))),
          ("general.alignment", 4, struct.pack("<I", alignment))]
    head = struct.pack("<4sIQQ", b"GGUF", 3, len(specs), len(kv))
    for key, vt, val in kv:
        head += s(key) + struct.pack("<I", vt) + val
    sizes = [native.row_bytes(t, K) * N if t != TYPE_F32 else 4 * N * K
             for (_, _, N, K, t) in specs]
    rel, off = [], 0
    for n in sizes:
        rel.append(off)
        off = (off + n + alignment - 1) // alignment * alignment
    for (tid, layer, N, K, t), r in zip(specs, rel):
        name = GGUF_NAMES[tid] if layer < 0 else f"blk.{layer}.{GGUF_NAMES[tid]}"
        dims = [K] if tid in (T_OUTPUT_NORM, T_ATTN_NORM, T_FFN_NORM) else [K, N]
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, r)
    start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head + bytes(start - len(head)))
        for i, (spec, r) in enumerate(zip(specs, rel)):
            f.write(bytes(start + r - f.tell()))
            f.write(np.ascontiguousarray(make_tensor(spec, seed, i)).view(np.uint8).tobytes())
        return f.tell()
