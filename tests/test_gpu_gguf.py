"""GGUF file -> resident model (pbx_model_load_gguf) on the GPU.

Synthetic Llama models are written as GGUF files (tests/gguf_writer.py)
with the tensor types real files carry (Q4_0 / Q4_1 / Q8_0 / F16 layer
matrices; Q6_K, F16, Q4_0 or F32 token embeddings; F32 norms), loaded with
the build's reader and compared with the oracle's llama.js forward on the
same bytes dequantised (gguf.js:219-367).  Bar: logits within 2e-3 max-abs,
greedy tokens equal to the oracle's argmax (ties below the bar allowed), and
bit-identical logits to the same model assembled tensor by tensor.
"""
import numpy as np
import pytest

import oracle
from purebee_amd import PbxError, synth
from purebee_amd.native import (Model, TYPE_F16, TYPE_F32, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q6_K,
                                TYPE_Q8_0, T_TOKEN_EMBD, T_OUTPUT, T_OUTPUT_NORM, T_ATTN_NORM,
                                T_FFN_NORM, T_ATTN_Q, T_ATTN_K, T_ATTN_V, T_ATTN_OUTPUT,
                                T_FFN_GATE, T_FFN_UP, T_FFN_DOWN)
from tests import gguf_writer as gw
from tests.e2e_util import LOGIT_TOL, check_greedy

pytestmark = pytest.mark.gpu

NAMES = {T_TOKEN_EMBD: "token_embd.weight", T_OUTPUT: "output.weight",
         T_OUTPUT_NORM: "output_norm.weight", T_ATTN_NORM: "attn_norm.weight",
         T_FFN_NORM: "ffn_norm.weight", T_ATTN_Q: "attn_q.weight", T_ATTN_K: "attn_k.weight",
         T_ATTN_V: "attn_v.weight", T_ATTN_OUTPUT: "attn_output.weight",
         T_FFN_GATE: "ffn_gate.weight", T_FFN_UP: "ffn_up.weight", T_FFN_DOWN: "ffn_down.weight"}
NORMS = (T_OUTPUT_NORM, T_ATTN_NORM, T_FFN_NORM)


def gguf_name(tid, layer):
    return NAMES[tid] if layer < 0 else f"blk.{layer}.{NAMES[tid]}"


def tensor_bytes(spec, seed, index):
    tid, layer, N, K, t = spec
    if tid in NORMS:  # non-trivial norms, so a swapped mapping shows
        return (1.0 + 0.1 * synth.native.synth_normal(seed + 500 + index, K)).astype(np.float32)
    return synth.make_tensor(spec, seed, index)


def write_model(path, cfg, seed, vocab_rows=None, n_tokens=None, order=None):
    """A GGUF file of cfg's tensors (token_embd with vocab_rows rows);
    returns [(spec, bytes)] in file order."""
    specs = synth.tensor_specs(cfg)
    if vocab_rows:
        specs = [(s[0], s[1], vocab_rows, s[3], s[4]) if s[0] in (T_TOKEN_EMBD, T_OUTPUT) else s
                 for s in specs]
    items = [(s, tensor_bytes(s, seed, i)) for i, s in enumerate(specs)]
    if order is not None:
        items = [items[i] for i in order(len(items))]
    tensors = [(gguf_name(s[0], s[1]), [s[3]] if s[0] in NORMS else [s[3], s[2]], s[4], b)
               for s, b in items]
    gw.write(path, gw.llama_kv(cfg, n_tokens=n_tokens), tensors)
    return items


def oracle_for(cfg, items, vocab):
    hd = cfg["dim"] // cfg["n_heads"]
    ref = oracle.LlamaRef(cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["n_heads"],
                          cfg["n_kv_heads"], hd, vocab, cfg["max_seq"], cfg["rope_theta"], 1e-5)
    for (tid, layer, N, K, t), b in items:
        if tid in (T_TOKEN_EMBD, T_OUTPUT):
            N = vocab  # the rows the model keeps
            b = np.asarray(b).view(np.uint8).ravel()[:vocab * oracle.row_bytes(t, K)]
        f = np.asarray(b, np.float32) if tid in NORMS else oracle.dequant(t, b, N * K)
        ref.set(tid, layer, f)
    return ref


def tiny(wt, et, ot=-1):
    return dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=1000,
                max_seq=64, weight_type=wt, embed_type=et, output_type=ot, rope_theta=10000.0)


@pytest.mark.parametrize("wt,et,ot", [(TYPE_Q4_0, TYPE_Q6_K, -1), (TYPE_Q8_0, TYPE_F16, TYPE_Q6_K),
                                      (TYPE_Q4_1, TYPE_Q4_0, -1), (TYPE_F16, TYPE_F32, TYPE_F16)])
def test_gguf_model_matches_oracle(ctx, tmp_path, wt, et, ot):
    print(f"[case] gguf model weights={wt} embed={et} output={ot}", flush=True)
    cfg = tiny(wt, et, ot)
    path = tmp_path / "m.gguf"
    # the tokenizer lists fewer tokens than token_embd has rows: the model
    # keeps the tokenizer's vocabulary (streaming-loader.js:57)
    items = write_model(path, cfg, seed=70 + wt + et, n_tokens=990,
                        order=lambda n: list(reversed(range(n))))
    model = Model.from_gguf(ctx, path, max_seq=64)
    assert model.vocab == 990
    ref = oracle_for(cfg, items, 990)
    prompt = synth.random_tokens(5, 7, 990)
    logits, nxt = model.forward(prompt, 0)
    rl = ref.forward(prompt, 0)
    err = float(np.abs(logits - rl).max())
    assert err <= LOGIT_TOL, err
    toks = model.generate(nxt, len(prompt), 12)
    exact, ties = check_greedy(ref, toks, nxt, len(prompt))
    assert exact >= 11
    model.free()
    ref.close()


def test_gguf_model_equals_tensor_by_tensor_model(ctx, tmp_path):
    """The loader only routes bytes: the GGUF-loaded model and the one built
    with pbx_model_set_tensor from the same bytes give identical logits."""
    print("[case] gguf vs set_tensor", flush=True)
    cfg = tiny(TYPE_Q4_0, TYPE_Q6_K)
    path = tmp_path / "m.gguf"
    items = write_model(path, cfg, seed=11)
    a = Model.from_gguf(ctx, path, max_seq=64)
    b = Model(ctx, 256, 512, 2, 4, 2, 1000, 64, TYPE_Q4_0, TYPE_Q6_K)
    for (tid, layer, N, K, t), data in items:
        b.set_tensor(tid, layer, data)
    prompt = synth.random_tokens(9, 5, 1000)
    la, _ = a.forward(prompt, 0)
    lb, _ = b.forward(prompt, 0)
    assert np.array_equal(la, lb)
    a.free(), b.free()


def test_gguf_loader_errors(ctx, tmp_path):
    print("[case] gguf loader errors", flush=True)
    cfg = tiny(TYPE_Q4_0, TYPE_Q4_0)
    specs = synth.tensor_specs(cfg)
    base = [(gguf_name(s[0], s[1]), [s[3]] if s[0] in NORMS else [s[3], s[2]], s[4],
             tensor_bytes(s, 3, i)) for i, s in enumerate(specs)]
    kv = gw.llama_kv(cfg)
    cases = {
        # an attention bias (Qwen-style) is not part of the Llama model
        "bias": (base + [("blk.0.attn_q.bias", [256], 0, np.zeros(256, np.float32))],
                 "not part of a Llama model"),
        # one layer matrix in another type
        "mixed": ([t if t[0] != "blk.1.ffn_up.weight" else
                   (t[0], t[1], TYPE_Q8_0, np.zeros(512 * 8 * 34, np.uint8)) for t in base],
                  "one type"),
        # a matrix whose shape disagrees with the metadata
        "shape": ([t if t[0] != "blk.0.attn_k.weight" else
                   (t[0], [256, 256], t[2], np.zeros(256 * 8 * 18, np.uint8)) for t in base],
                  "expected"),
    }
    for what, (tensors, msg) in cases.items():
        p = tmp_path / f"{what}.gguf"
        gw.write(p, kv, tensors)
        with pytest.raises(PbxError, match=msg):
            Model.from_gguf(ctx, p, max_seq=64)
    # a missing tensor loads but cannot run
    p = tmp_path / "missing.gguf"
    gw.write(p, kv, [t for t in base if t[0] != "blk.1.ffn_down.weight"])
    m = Model.from_gguf(ctx, p, max_seq=64)
    with pytest.raises(PbxError):
        m.forward([1, 2, 3], 0)
    m.free()
