"""The Llama-3.2-1B-shaped Q4_0 workloads at their full length against the
oracle (llama.js:204-371, 452-505): a 128-token prompt and 256 greedy decode
steps (KV cache to 384 positions), and the 5-row speculative verify at the
full vocabulary (speculative.js:129-185).  One oracle model serves both
tests (loading it takes most of their time)."""
import numpy as np
import pytest

import oracle
from purebee_amd import synth
from tests.e2e_util import LOGIT_TOL, make_pair

pytestmark = pytest.mark.gpu

N_PROMPT, N_GEN, CHUNK = 128, 256, 8


@pytest.fixture(scope="module")
def llama_pair(ctx):
    model, ref, cfg = make_pair(ctx, "llama32_1b", 3300)
    yield model, ref, cfg
    model.free()
    ref.close()


def top_gap(logits, a, b):
    return float(logits[a] - logits[b])


@pytest.mark.timeout(600)
def test_llama1b_prompt128_greedy256(llama_pair):
    """The decode workload: 128-token prompt through the batched prefill, then
    256 greedy steps replayed from the captured multi-step graphs.  The GPU's
    tokens are fed again one decode step at a time from position 128 (each
    step must choose the token generate chose); the oracle takes the same
    tokens teacher-forced, one at a time for the first 64 steps and in
    forwards of 8 after that, and every step it yields logits for (all of
    the first 64, then every 8th up to KV 384) is compared at the logit
    tolerance, with the GPU's choice there its argmax or a near-tie."""
    model, ref, cfg = llama_pair
    print(f"[case] llama32_1b {N_PROMPT}-token prompt + {N_GEN} greedy, oracle every step "
          f"to 64 then every {CHUNK}th", flush=True)
    model.reset_cache()
    prompt = synth.random_tokens(3301, N_PROMPT, cfg["vocab_size"])
    ref_logits = ref.forward(prompt, 0)
    logits, nxt = model.forward(prompt, 0)
    worst = float(np.abs(logits - ref_logits).max())
    assert worst <= LOGIT_TOL, f"prefill logits max-abs {worst:.2e}"
    first = oracle.argmax(ref_logits)
    assert nxt == first or top_gap(ref_logits, first, nxt) < LOGIT_TOL
    toks = model.generate(nxt, N_PROMPT, N_GEN)
    model.rollback(N_PROMPT)
    feed = [nxt] + [int(t) for t in toks[:-1]]
    gpu = []
    for i, tok in enumerate(feed):
        g, gnext = model.forward([tok], N_PROMPT + i)
        assert gnext == int(toks[i]), f"step {i}: replay chose {gnext}, generate chose {toks[i]}"
        gpu.append(g)
    checked, exact, ties = 0, 0, 0
    i = 0
    while i < N_GEN:
        n = 1 if i < 64 else CHUNK
        r = ref.forward(feed[i:i + n], N_PROMPT + i)
        k = i + n - 1  # the step whose logits the oracle returned
        err = float(np.abs(gpu[k] - r).max())
        worst = max(worst, err)
        assert err <= LOGIT_TOL, f"step {k} (KV {N_PROMPT + k + 1}): logits max-abs {err:.2e}"
        best = oracle.argmax(r)
        if int(toks[k]) == best:
            exact += 1
        else:
            gap = top_gap(r, best, int(toks[k]))
            assert gap < LOGIT_TOL, f"step {k}: GPU {toks[k]} vs oracle {best}, gap {gap:.3e}"
            ties += 1
        checked += 1
        i += n
    print(f"  {checked} steps checked, exact={exact} ties={ties}, worst logits max-abs={worst:.1e}")
    assert checked == 64 + (N_GEN - 64) // CHUNK
    assert exact >= checked - 2


@pytest.mark.timeout(600)
def test_llama1b_verify5_vs_oracle(llama_pair):
    """The M>1 config's verify: one forward of 5 rows (next token + 4 drafts)
    after a 128-token prompt, at vocabulary 128256, against the oracle's
    forward of the same tokens one position at a time (the reference's
    verify loop, speculative.js:131-137): every row's logits at the logit
    tolerance and every row's argmax the oracle's (or a near-tie)."""
    model, ref, cfg = llama_pair
    print("[case] llama32_1b 5-row verify at vocab 128256 vs oracle", flush=True)
    vocab = cfg["vocab_size"]
    model.reset_cache()
    prompt = synth.random_tokens(3001, N_PROMPT, vocab)
    model.forward(prompt, 0, want_logits=False)
    ref.forward(prompt, 0)
    worst = 0.0
    for rep in range(2):
        start = N_PROMPT + 5 * rep
        rows = [int(t) for t in synth.random_tokens(3002 + rep, 5, vocab)]
        lb, nb = model.forward_batch(rows, start)
        for t, tok in enumerate(rows):
            r = ref.forward([tok], start + t)
            err = float(np.abs(lb[t] - r).max())
            worst = max(worst, err)
            assert err <= LOGIT_TOL, f"verify {rep} row {t}: max-abs {err:.2e}"
            best = oracle.argmax(r)
            assert nb[t] == best or top_gap(r, best, nb[t]) < LOGIT_TOL
    print(f"  worst max-abs {worst:.2e}")
