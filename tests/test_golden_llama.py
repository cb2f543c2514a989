"""Pins the oracle's Llama forward (oracle/llama_ref.c) against the
reference's own LlamaRuntime outputs (tests/golden/llama_tiny.json, written
by tests/golden/make_llama_fixture.js from llama.js), plus the invariants the
reference's two forward modes imply."""
import numpy as np
import pytest

import oracle
from tests.golden import llama_fixture as lf


@pytest.fixture(scope="module")
def fixture():
    return lf.load()


def oracle_model(fx):
    c = fx["config"]
    ref = oracle.LlamaRef(c["dim"], c["hiddenDim"], c["nLayers"], c["nHeads"], c["nKvHeads"],
                          c["dim"] // c["nHeads"], c["vocabSize"], c["seqLen"], c["ropeTheta"])
    for tid, layer, w in lf.weights(fx):
        ref.set(tid, layer, w)
    return ref


def test_oracle_matches_reference_llama_js(fixture):
    ref = oracle_model(fixture)
    for st in fixture["steps"]:
        got = ref.forward(st["tokens"], st["pos"])
        want = np.asarray(st["logits"], np.float32)
        # the reference accumulates LINEAR in f32 (engine.js:222-240), the
        # oracle in double: they agree far inside the 2e-3 logit bar
        assert np.abs(got - want).max() < 1e-4, (st["pos"], np.abs(got - want).max())
        assert oracle.argmax(got) == st["argmax"]
    ref.close()


def test_prefill_equals_sequential_decode(fixture):
    """llama.js forward over a prompt at once (causal mask) and token by token
    must agree: the reference's prefill and decode modes."""
    a = oracle_model(fixture)
    b = oracle_model(fixture)
    prompt = fixture["steps"][0]["tokens"]
    la = a.forward(prompt, 0)
    for p, t in enumerate(prompt):
        lb = b.forward([t], p)
    assert np.abs(la - lb).max() < 1e-5
    a.close()
    b.close()


def test_position_zero_attention_is_v(fixture):
    """With one cached position, softmax over a single score is 1 and the
    attention output equals V: zeroing wq and wk changes nothing at pos 0."""
    c = fixture["config"]
    base = oracle_model(fixture)
    alt = oracle_model(fixture)
    for tid, layer, w in lf.weights(fixture):
        if tid in (lf.T_Q, lf.T_K):
            alt.set(tid, layer, np.zeros_like(w))
    tok = [7]
    assert np.array_equal(base.forward(tok, 0), alt.forward(tok, 0))
    # ... but not at pos 1, where the scores matter
    assert not np.array_equal(base.forward([8], 1), alt.forward([8], 1))
    base.close()
    alt.close()


def test_max_layers_equals_truncated_model(fixture):
    """StreamingLlamaRuntime.forward(tokens, pos, {maxLayers: L})
    (llama-streaming.js:745, 764-792) runs the first L layers, then the final
    norm and head: bit for bit the forward of a model holding only those L
    layers, including over several calls that read the cache those layers
    wrote.  maxLayers 0 (or >= nLayers) is the full forward."""
    c = dict(fixture["config"])
    full = oracle_model(fixture)
    L = c["nLayers"] - 1
    trunc = oracle.LlamaRef(c["dim"], c["hiddenDim"], L, c["nHeads"], c["nKvHeads"],
                            c["dim"] // c["nHeads"], c["vocabSize"], c["seqLen"], c["ropeTheta"])
    for tid, layer, w in lf.weights(fixture):
        if layer < L:
            trunc.set(tid, layer, w)
    prompt = fixture["steps"][0]["tokens"]
    assert np.array_equal(full.forward(prompt, 0, max_layers=L), trunc.forward(prompt, 0))
    n = len(prompt)
    for p, t in enumerate([3, 9, 27]):
        assert np.array_equal(full.forward([t], n + p, max_layers=L), trunc.forward([t], n + p))
    ref = oracle_model(fixture)
    full.rollback(0)
    a = full.forward(prompt, 0, max_layers=0)
    full.rollback(0)
    b = full.forward(prompt, 0, max_layers=c["nLayers"] + 3)
    assert np.array_equal(a, ref.forward(prompt, 0)) and np.array_equal(a, b)
    # the truncated forward differs from the full one (the last layer matters)
    ref.rollback(0)
    assert not np.array_equal(ref.forward(prompt, 0, max_layers=L), a)
    full.close()
    trunc.close()
    ref.close()
