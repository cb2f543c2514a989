"""Shared helpers for end-to-end decode parity: the GPU model and the oracle's
llama.js restatement built from the same seeded tensors."""
import numpy as np

import oracle
from purebee_amd import synth
from purebee_amd.native import TYPE_F32

LOGIT_TOL = 2e-3  # max-abs on logits


def make_pair(ctx, cfg, seed=1000):
    if isinstance(cfg, str):
        cfg = synth.CONFIGS[cfg]
    hd = cfg.get("head_dim") or cfg["dim"] // cfg["n_heads"]
    ref = oracle.LlamaRef(cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["n_heads"],
                          cfg["n_kv_heads"], hd, cfg["vocab_size"], cfg["max_seq"],
                          cfg.get("rope_theta", 10000.0), cfg.get("rms_eps", 1e-5))

    def keep(spec, data):
        tid, layer, N, K, t = spec
        if t == TYPE_F32:
            f = np.asarray(data, np.float32)
        else:
            f = oracle.dequant(t, data, N * K)
        ref.set(tid, layer, f)

    model = synth.build(ctx, cfg, seed, keep)
    return model, ref, cfg


def check_greedy(ref, tokens_gpu, first_token, start_pos, tol=LOGIT_TOL):
    """Walk the GPU's greedy choices through the oracle (teacher forcing on the
    GPU's own tokens).  Every choice must be the oracle's argmax, or within
    `tol` of the oracle's maximum (a tie below the logit tolerance).
    Returns (exact matches, near-ties)."""
    exact, ties = 0, 0
    tok, pos = first_token, start_pos
    for i, g in enumerate(tokens_gpu):
        L = ref.forward([tok], pos)
        best = oracle.argmax(L)
        if int(g) == best:
            exact += 1
        else:
            gap = float(L[best] - L[int(g)])
            assert gap < tol, f"step {i}: GPU chose {g}, oracle argmax {best}, gap {gap:.3e}"
            ties += 1
        tok, pos = int(g), pos + 1
    return exact, ties
