"""Reader for tests/golden/llama_tiny.json (written by make_llama_fixture.js
from the reference's LlamaRuntime): regenerates the fixture's f32 weights
with the same 32-bit LCG, in GGUF orientation [N,K]."""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# tensor ids as PBX_T_* / the oracle
T_EMBD, T_OUTPUT_NORM, T_ATTN_NORM, T_FFN_NORM = 0, 2, 3, 4
T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN = 5, 6, 7, 8, 9, 10, 11


def load():
    with open(os.path.join(HERE, "llama_tiny.json")) as f:
        return json.load(f)


def _draw(seed, n, scale, offset=0.0):
    out = np.empty(n, np.float64)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = ((s >> 8) / 16777216.0 - 0.5) * scale + offset
    return out.astype(np.float32)


def weights(fx):
    """[(tensor id, layer, array)] in the generator's draw order."""
    c = fx["config"]
    dim, hid, nl = c["dim"], c["hiddenDim"], c["nLayers"]
    hd = dim // c["nHeads"]
    kv = c["nKvHeads"] * hd
    s = fx["seed"]
    out = [(T_EMBD, -1, _draw(s, c["vocabSize"] * dim, 1.0).reshape(c["vocabSize"], dim))]
    out.append((T_OUTPUT_NORM, -1, _draw(s + 1, dim, 0.4, 1.0)))
    s += 2
    for l in range(nl):
        out.append((T_ATTN_NORM, l, _draw(s, dim, 0.4, 1.0)))
        out.append((T_FFN_NORM, l, _draw(s + 1, dim, 0.4, 1.0)))
        s += 2
        for tid, N, K in ((T_Q, dim, dim), (T_K, kv, dim), (T_V, kv, dim), (T_O, dim, dim),
                          (T_GATE, hid, dim), (T_UP, hid, dim), (T_DOWN, dim, hid)):
            out.append((tid, l, _draw(s, N * K, 0.4).reshape(N, K)))
            s += 1
    return out
