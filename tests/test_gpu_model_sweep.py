"""Seeded random model shapes through the on-GPU forward and decode step against the oracle's
llama.js restatement (llama.js:204-371, llama-streaming.js:505-606): head_dim 32..256, MHA and
GQA, 1-3 layers, every layer and embedding type, tied and untied heads, prompts of 1-20 tokens.
The decode step picks its kernels by shape and type (integer-limb or float GEMVs, the joined
q|k|v + attention launch, the one-launch small-model step, the attention variants), so this
walks that selection away from the three workload models.  Same bars as the fixed-shape
tests: logits within 2e-3 max-abs of the oracle after the prompt and after the greedy steps,
and every greedy token the oracle's argmax (or within that tolerance of it)."""
import numpy as np
import pytest

from purebee_amd import synth
from purebee_amd.native import TYPE_F16, TYPE_F32, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q6_K, TYPE_Q8_0
from tests.e2e_util import LOGIT_TOL, make_pair
from tests.test_gpu_decode import run_prompt_then_greedy

pytestmark = pytest.mark.gpu

WEIGHTS = [TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_1, TYPE_Q4_0, TYPE_Q8_0, TYPE_F16]
EMBEDS = [TYPE_Q4_0, TYPE_Q8_0, TYPE_F32, TYPE_F16, TYPE_Q4_1]
HEAD_DIMS = [32, 40, 48, 64, 64, 80, 96, 128, 256]


def draw(case):
    rng = np.random.default_rng(72000 + case)
    while True:
        hd = int(rng.choice(HEAD_DIMS))
        n_heads = int(rng.integers(1, 13))
        dim = hd * n_heads
        if dim % 32 == 0 and dim <= 1024:
            break
    kv_choices = [k for k in range(1, n_heads + 1) if n_heads % k == 0]
    n_kv = int(rng.choice(kv_choices))
    hidden = 32 * int(rng.integers(max(1, dim // 32), 3 * dim // 32 + 1))
    wt = WEIGHTS[case % len(WEIGHTS)]
    et = EMBEDS[case % len(EMBEDS)]
    n_prompt = int(rng.integers(1, 21))
    n_gen = int(rng.integers(4, 17))
    cfg = dict(dim=dim, hidden_dim=hidden, n_layers=int(rng.integers(1, 4)), n_heads=n_heads,
               n_kv_heads=n_kv, vocab_size=int(rng.integers(64, 3000)),
               max_seq=n_prompt + n_gen + 8, weight_type=wt, embed_type=et,
               rope_theta=float(rng.choice([10000.0, 500000.0])))
    if rng.random() < 0.3:
        cfg["output_type"] = int(rng.choice([TYPE_Q4_0, TYPE_Q8_0, TYPE_F32]))
    if dim % 256 == 0 and rng.random() < 0.3:
        cfg["output_type"] = TYPE_Q6_K  # the GGUF files' head type (K a multiple of 256)
    return cfg, n_prompt, n_gen


@pytest.mark.parametrize("case", range(30))
def test_random_model_prefill_and_greedy(ctx, case):
    cfg, n_prompt, n_gen = draw(case)
    print(f"[case] model sweep {case}: {cfg} prompt {n_prompt} steps {n_gen}", flush=True)
    exact, ties, e1, e2 = run_prompt_then_greedy(ctx, cfg, n_prompt, n_gen, seed=3000 + case)
    print(f"  exact={exact} ties={ties} prefill_err={e1:.1e} final_err={e2:.1e}", flush=True)
    assert exact + ties == n_gen
    assert exact >= n_gen - 2


@pytest.mark.parametrize("case", range(16))
def test_random_model_batched_rows(ctx, case):
    """The batched forward of 2-8 rows after a prompt (the speculative verify's
    forward_batch: rows at positions P .. P + n - 1 attending to the cache and to
    each other) against the oracle consuming the same tokens one at a time
    (speculative.js:129-185 runs the target over the draft the same way)."""
    cfg, n_prompt, n_gen = draw(100 + case)
    rng = np.random.default_rng(5000 + case)
    n = int(rng.integers(2, 9))
    cfg["max_seq"] = n_prompt + n + 8
    print(f"[case] batched rows {case}: {cfg} prompt {n_prompt} rows {n}", flush=True)
    model, ref, cfg = make_pair(ctx, cfg, 4000 + case)
    prompt = synth.random_tokens(4100 + case, n_prompt, cfg["vocab_size"])
    ref.forward(prompt, 0)
    model.forward(prompt, 0, want_logits=False)
    rows = synth.random_tokens(4200 + case, n, cfg["vocab_size"])
    logits, nxt = model.forward_batch(rows, n_prompt)
    worst = 0.0
    for i in range(n):
        ref_l = ref.forward([int(rows[i])], n_prompt + i)
        worst = max(worst, float(np.abs(logits[i] - ref_l).max()))
        assert int(nxt[i]) == int(np.argmax(logits[i]))
    print(f"  rows={n} worst logit max-abs {worst:.2e}", flush=True)
    assert worst <= LOGIT_TOL
    model.free()
    ref.close()
