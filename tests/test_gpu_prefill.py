"""The M > 1 path: batched prefill and speculative verify through the MFMA
GEMM (llama.js:204-371 with seqLen > 1; speculative.js:58-204).

Bars:
* batched prefill logits within 2e-3 max-abs of the oracle's forward;
* every row of a batched forward within 2e-3 of the same position's
  single-token (decode-step) forward, with the same argmax unless the two
  top logits are closer than that tolerance;
* speculative decoding emits exactly the target's greedy tokens, and the
  batched verify (one forward of drafts + 1 rows) takes exactly the accept /
  reject decisions of the reference's one-forward-per-draft verify.
"""
import numpy as np
import pytest

import oracle
from purebee_amd import PbxError, synth
from purebee_amd.native import (TYPE_F16, TYPE_F32, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q8_0,
                                self_speculative_generate, speculative_generate)
from tests.e2e_util import LOGIT_TOL, make_pair

pytestmark = pytest.mark.gpu


def tiny(weight_type, embed_type, **kw):
    cfg = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=1000,
               max_seq=128, weight_type=weight_type, embed_type=embed_type, rope_theta=10000.0)
    cfg.update(kw)
    return cfg


def top_gap(logits, a, b):
    return abs(float(logits[a]) - float(logits[b]))


@pytest.mark.parametrize("wt,et", [(TYPE_Q4_0, TYPE_Q4_0), (TYPE_Q8_0, TYPE_Q8_0),
                                   (TYPE_Q8_0, TYPE_F32), (TYPE_F32, TYPE_F32)])
def test_batched_rows_match_oracle_positions(ctx, wt, et):
    """forward_batch row t == the oracle's logits at position start + t."""
    print(f"[case] forward_batch rows vs oracle weights={wt} embed={et}", flush=True)
    model, ref, cfg = make_pair(ctx, tiny(wt, et), 300 + wt)
    prompt = [int(t) for t in synth.random_tokens(301, 6, cfg["vocab_size"])]
    model.forward(prompt, 0)
    ref.forward(prompt, 0)
    rows = [int(t) for t in synth.random_tokens(302, 9, cfg["vocab_size"])]
    logits, nxt = model.forward_batch(rows, len(prompt))
    worst = 0.0
    for t, tok in enumerate(rows):
        r = ref.forward([tok], len(prompt) + t)
        worst = max(worst, float(np.abs(logits[t] - r).max()))
        assert nxt[t] == int(np.argmax(logits[t]))
        best = oracle.argmax(r)
        if nxt[t] != best:
            assert top_gap(r, best, nxt[t]) < LOGIT_TOL
    print(f"  worst max-abs {worst:.2e}")
    assert worst <= LOGIT_TOL
    model.free()
    ref.close()


@pytest.mark.parametrize("n", [4, 5, 31, 64])
def test_batched_prefill_vs_oracle(ctx, n):
    print(f"[case] batched prefill n={n}", flush=True)
    model, ref, cfg = make_pair(ctx, tiny(TYPE_Q4_0, TYPE_Q4_0, n_layers=3), 310 + n)
    prompt = [int(t) for t in synth.random_tokens(311, n, cfg["vocab_size"])]
    g, nxt = model.forward(prompt, 0)
    r = ref.forward(prompt, 0)
    err = float(np.abs(g - r).max())
    print(f"  max-abs {err:.2e}")
    assert err <= LOGIT_TOL
    assert nxt == int(np.argmax(g))
    # the state left by the batched prefill continues like a decode: the
    # next greedy step sees all n cached positions
    toks = model.generate(nxt, n, 3)
    r2 = ref.forward([nxt], n)
    best = oracle.argmax(r2)
    assert toks[0] == best or top_gap(r2, best, toks[0]) < LOGIT_TOL
    model.free()
    ref.close()


@pytest.mark.parametrize("n_heads,n_kv", [(4, 2), (8, 2), (4, 4)])
def test_batched_chunks_every_row_vs_oracle(ctx, n_heads, n_kv):
    """A 50-token batched prefill, then a 30-token batch at position 50
    (forward_batch keeps every row's logits): the batched attention with a
    non-zero start, keys over two 64-key stages and a partial query tile, for
    head_dim 64 (4 heads) and 32 (8 heads), GQA and MHA; every row against the
    oracle at its position."""
    print(f"[case] batched chunks 50 + 30, heads {n_heads}/{n_kv}", flush=True)
    model, ref, cfg = make_pair(ctx, tiny(TYPE_Q4_0, TYPE_Q4_0, n_heads=n_heads, n_kv_heads=n_kv),
                                330 + n_heads + n_kv)
    first = [int(t) for t in synth.random_tokens(331, 50, cfg["vocab_size"])]
    model.forward(first, 0)
    ref.forward(first, 0)
    rows = [int(t) for t in synth.random_tokens(332, 30, cfg["vocab_size"])]
    logits, _ = model.forward_batch(rows, 50)
    worst = 0.0
    for t, tok in enumerate(rows):
        r = ref.forward([tok], 50 + t)
        worst = max(worst, float(np.abs(logits[t] - r).max()))
    print(f"  worst max-abs {worst:.2e}")
    assert worst <= LOGIT_TOL
    model.free()
    ref.close()


@pytest.mark.parametrize("start,n", [(0, 200), (37, 130), (0, 16)])
def test_prefill_attention_key_groups(ctx, monkeypatch, start, n):
    """The prefill attention with each workgroup's 64-key stages split over
    two groups of four waves (pbx_attention_mfma_g2, the default) against
    the one-group form (PBX_PREFILL_ATTN_GROUPS=1) on every row of a batched
    forward, ragged last tiles and a non-zero start included (tiles whose
    last stage falls to one group only), and against the oracle."""
    print(f"[case] prefill attention key groups, start {start}, {n} rows", flush=True)
    cfg = tiny(TYPE_Q8_0, TYPE_Q8_0, dim=512, hidden_dim=1024, n_heads=8, n_kv_heads=2,
               max_seq=256)
    model, ref, cfg = make_pair(ctx, cfg, 340 + start)
    toks = [int(t) for t in synth.random_tokens(341 + start, start + n, cfg["vocab_size"])]
    if start:
        model.forward(toks[:start], 0, want_logits=False)
    two, _ = model.forward_batch(toks[start:], start)
    monkeypatch.setenv("PBX_PREFILL_ATTN_GROUPS", "1")
    one, _ = model.forward_batch(toks[start:], start)
    monkeypatch.delenv("PBX_PREFILL_ATTN_GROUPS")
    r = ref.forward(toks, 0)
    d = float(np.abs(two - one).max())
    err = float(np.abs(two[-1] - r).max())
    print(f"  two groups vs one max-abs {d:.2e}, last row vs oracle {err:.2e}")
    assert d <= 1e-4
    assert err <= LOGIT_TOL
    model.free()
    ref.close()


def test_prefill_gqa_untied_head(ctx):
    print("[case] batched prefill, GQA 6/2, untied Q8_0 head, head_dim 48", flush=True)
    cfg = tiny(TYPE_Q8_0, TYPE_F32, dim=288, hidden_dim=768, n_heads=6, n_kv_heads=2,
               output_type=TYPE_Q8_0)
    model, ref, cfg = make_pair(ctx, cfg, 320)
    prompt = [int(t) for t in synth.random_tokens(321, 17, cfg["vocab_size"])]
    g, _ = model.forward(prompt, 0)
    r = ref.forward(prompt, 0)
    assert float(np.abs(g - r).max()) <= LOGIT_TOL
    # continue with a second batched chunk at a non-zero start position
    more = [int(t) for t in synth.random_tokens(322, 8, cfg["vocab_size"])]
    g2, _ = model.forward(more, 17)
    r2 = ref.forward(more, 17)
    assert float(np.abs(g2 - r2).max()) <= LOGIT_TOL
    model.free()
    ref.close()


def _sequential_logits(model, tokens, start):
    out = []
    for i, t in enumerate(tokens):
        lg, _ = model.forward([int(t)], start + i)
        out.append(lg)
    return np.stack(out)


def test_llama1b_verify_rows_equal_sequential(ctx):
    """Verify invariant of the M>1 config: one M=5 forward == 5 single-token
    forwards (the reference's verify loop, speculative.js:131-137), on the
    Llama-3.2-1B-shaped Q4_0 model after a 128-token prompt."""
    print("[case] llama32_1b M=5 verify vs sequential", flush=True)
    model = synth.build(ctx, "llama32_1b", 3000)
    vocab = synth.CONFIGS["llama32_1b"]["vocab_size"]
    prompt = [int(t) for t in synth.random_tokens(3001, 128, vocab)]
    rows = [int(t) for t in synth.random_tokens(3002, 5, vocab)]
    worst, flips = 0.0, 0
    for rep in range(3):
        model.reset_cache()
        model.forward(prompt, 0)
        start = 128 + 5 * rep
        if rep:
            model.forward(synth.random_tokens(3003 + rep, 5 * rep, vocab), 128)
        lb, nb = model.forward_batch(rows, start)
        ls = _sequential_logits(model, rows, start)
        worst = max(worst, float(np.abs(lb - ls).max()))
        for t in range(5):
            s = int(np.argmax(ls[t]))
            if nb[t] != s:
                flips += 1
                assert top_gap(ls[t], s, nb[t]) < LOGIT_TOL
    print(f"  worst max-abs {worst:.2e} argmax near-tie flips {flips}")
    assert worst <= LOGIT_TOL
    model.free()


def test_row_batched_kernels_vs_oracle(ctx):
    """The up-to-8-row verify kernels run for Q4_0 models with dim <= 2048,
    6144 < hidden <= 8192 and a Q4_0 head: for 1..5 rows the int8-MFMA rows
    kernels (q|k|v with RoPE and the cache append, o, gate|up + SwiGLU, down
    split over K slices, the LM head) and the batched-row attention; for 6..8
    rows the integer-limb rows GEMVs and the skinny MFMA kernels.  A
    one-layer model of that shape with a small vocabulary, after a 40-token
    prompt: forward_batch of n = 1, 5 and 8 rows, every row's logits against
    the oracle's forward at the same position (llama.js:204-371,
    teacher-forced on the same tokens)."""
    print("[case] 1-layer dim 2048 / hidden 8192 Q4_0 rows kernels vs oracle", flush=True)
    cfg = dict(dim=2048, hidden_dim=8192, n_layers=1, n_heads=32, n_kv_heads=8, vocab_size=4096,
               max_seq=128, weight_type=TYPE_Q4_0, embed_type=TYPE_Q4_0, rope_theta=500000.0)
    model, ref, cfg = make_pair(ctx, cfg, 3400)
    prompt = [int(t) for t in synth.random_tokens(3401, 40, cfg["vocab_size"])]
    model.forward(prompt, 0)
    ref.forward(prompt, 0)
    worst = 0.0
    for n in (1, 5, 8):
        rows = [int(t) for t in synth.random_tokens(3402 + n, n, cfg["vocab_size"])]
        model.rollback(40)
        ref.rollback(40)
        logits, nxt = model.forward_batch(rows, 40)
        for t, tok in enumerate(rows):
            r = ref.forward([tok], 40 + t)
            err = float(np.abs(logits[t] - r).max())
            worst = max(worst, err)
            assert err <= LOGIT_TOL, f"n={n} row {t}: max-abs {err:.2e}"
            best = oracle.argmax(r)
            assert nxt[t] == best or top_gap(r, best, nxt[t]) < LOGIT_TOL
    print(f"  worst max-abs {worst:.2e}")
    model.free()
    ref.close()


@pytest.mark.parametrize("n", [1, 3, 6, 8])
def test_llama1b_row_batched_gemvs(ctx, monkeypatch, n):
    """Up to 8 rows through the row-batched integer-limb GEMVs (one pass over
    the weights for all rows; 6..8 rows split 5 + rest for down) against the
    same rows through the MFMA GEMM path (PBX_GEMV_INT=0) and against n
    single-token forwards."""
    print(f"[case] llama32_1b row-batched GEMVs, {n} rows", flush=True)
    model = synth.build(ctx, "llama32_1b", 3300)
    monkeypatch.setenv("PBX_GEMV_INT", "0")
    ref = synth.build(ctx, "llama32_1b", 3300)
    monkeypatch.delenv("PBX_GEMV_INT")
    vocab = synth.CONFIGS["llama32_1b"]["vocab_size"]
    prompt = [int(t) for t in synth.random_tokens(3301, 40, vocab)]
    rows = [int(t) for t in synth.random_tokens(3302, n, vocab)]
    model.forward(prompt, 0)
    ref.forward(prompt, 0)
    lb, nb = model.forward_batch(rows, 40)
    lr, _ = ref.forward_batch(rows, 40)
    ls = _sequential_logits(model, rows, 40)
    e_gemm = float(np.abs(lb - lr).max())
    e_seq = float(np.abs(lb - ls).max())
    print(f"  vs GEMM path {e_gemm:.2e}, vs sequential {e_seq:.2e}")
    assert e_gemm <= LOGIT_TOL and e_seq <= LOGIT_TOL
    for t in range(n):
        s = int(np.argmax(ls[t]))
        assert nb[t] == s or top_gap(ls[t], s, nb[t]) < LOGIT_TOL
    model.free()
    ref.free()


def test_llama1b_prefill_512_equals_sequential(ctx):
    """Batched prefill of a 512-token prompt (M = 512 through the MFMA GEMM)
    against the same prompt fed one decode step at a time."""
    print("[case] llama32_1b prefill 512 batched vs sequential", flush=True)
    model = synth.build(ctx, "llama32_1b", 3100)
    vocab = synth.CONFIGS["llama32_1b"]["vocab_size"]
    prompt = [int(t) for t in synth.random_tokens(3101, 512, vocab)]
    lb, nb = model.forward(prompt, 0)
    follow_b = model.generate(nb, 512, 8)
    model.reset_cache()
    ls = None
    for i, t in enumerate(prompt):
        ls, ns = model.forward([t], i)
    err = float(np.abs(lb - ls).max())
    print(f"  last-position max-abs {err:.2e}, argmax {nb} vs {ns}")
    assert err <= LOGIT_TOL
    assert nb == ns or top_gap(ls, ns, nb) < LOGIT_TOL
    # the decode that followed the batched prefill is a greedy walk over the
    # sequentially written cache too (teacher forcing on its own tokens)
    tok, pos = nb, 512
    for g in follow_b:
        L, best = model.forward([int(tok)], pos)
        assert g == best or top_gap(L, best, g) < LOGIT_TOL
        tok, pos = int(g), pos + 1
    model.free()


def _greedy(model, prompt, n_gen):
    model.reset_cache()
    _, nxt = model.forward(prompt, 0)
    rest = model.generate(nxt, len(prompt), n_gen - 1)
    return [nxt] + [int(t) for t in rest]


@pytest.mark.parametrize("draft_kind", ["other", "same"])
def test_speculative_equals_greedy(ctx, draft_kind):
    """Greedy speculative decoding emits the target's own greedy tokens,
    whatever the draft proposes; the batched verify and the reference's
    one-by-one verify take the same decisions."""
    print(f"[case] speculative draft={draft_kind}", flush=True)
    tcfg = tiny(TYPE_Q4_0, TYPE_Q4_0, n_layers=3, max_seq=200)
    target = synth.build(ctx, tcfg, 400)
    if draft_kind == "same":
        draft = synth.build(ctx, tcfg, 400)  # identical weights: every draft agrees
    else:
        draft = synth.build(ctx, tiny(TYPE_Q8_0, TYPE_F32, dim=128, hidden_dim=256,
                                      n_heads=2, n_kv_heads=2, vocab_size=700, max_seq=200), 401)
    prompt = [int(t) for t in synth.random_tokens(402, 16, tcfg["vocab_size"])]
    n_gen = 48
    ref = _greedy(target, prompt, n_gen)
    out_b, st_b = speculative_generate(target, draft, prompt, n_gen, 4, eos_ids=(),
                                       batched_verify=True)
    out_s, st_s = speculative_generate(target, draft, prompt, n_gen, 4, eos_ids=(),
                                       batched_verify=False)
    print(f"  batched {st_b}\n  sequential {st_s}")
    assert list(out_s[:n_gen]) == ref
    assert list(out_b) == list(out_s)
    assert (st_b["rounds"], st_b["drafted"], st_b["accepted"]) == \
           (st_s["rounds"], st_s["drafted"], st_s["accepted"])
    assert len(out_b) in (n_gen, n_gen + 1)
    if draft_kind == "same":
        assert st_b["accepted"] == st_b["drafted"]
    target.free()
    draft.free()


def test_speculative_eos_and_budget(ctx):
    """EOS stops decoding at the first emitted EOS (speculative.js:148-166);
    max_tokens bounds the drafts (speculative.js:94)."""
    print("[case] speculative eos/budget", flush=True)
    tcfg = tiny(TYPE_Q8_0, TYPE_Q8_0, max_seq=128)
    target = synth.build(ctx, tcfg, 410)
    draft = synth.build(ctx, tcfg, 410)
    prompt = [int(t) for t in synth.random_tokens(411, 8, tcfg["vocab_size"])]
    ref = _greedy(target, prompt, 20)
    eos = ref[9]
    stop = ref.index(eos)
    for batched in (True, False):
        out, _ = speculative_generate(target, draft, prompt, 20, 4, eos_ids=(eos,),
                                      batched_verify=batched)
        assert list(out) == ref[:stop + 1]
    out, _ = speculative_generate(target, draft, prompt, 3, 4, eos_ids=())
    assert list(out[:3]) == ref[:3] and len(out) <= 4
    target.free()
    draft.free()


def test_speculative_config_shapes(ctx):
    """The M>1 config: Llama-3.2-1B-shaped Q4_0 target, stories15M-shaped
    draft (vocabulary 32000: target tokens enter the draft modulo 32000),
    draft_count 4, verify M = 5."""
    print("[case] speculative llama32_1b target, stories15m draft", flush=True)
    target = synth.build(ctx, "llama32_1b", 3200)
    draft = synth.build(ctx, "stories15m", 3201)
    vocab = synth.CONFIGS["llama32_1b"]["vocab_size"]
    prompt = [int(t) for t in synth.random_tokens(3202, 32, vocab)]
    n_gen = 24
    ref = _greedy(target, prompt, n_gen)
    out_b, st_b = speculative_generate(target, draft, prompt, n_gen, 4, eos_ids=())
    out_s, st_s = speculative_generate(target, draft, prompt, n_gen, 4, eos_ids=(),
                                       batched_verify=False)
    print(f"  batched {st_b}\n  sequential {st_s}")
    assert list(out_s[:n_gen]) == ref
    assert list(out_b) == list(out_s)
    target.free()
    draft.free()


@pytest.mark.parametrize("wt", [TYPE_Q4_0, TYPE_Q8_0])
def test_forward_max_layers_vs_truncated_oracle(ctx, wt):
    """StreamingLlamaRuntime.forward(tokens, pos, {maxLayers}) (llama-streaming.js:
    738-815): the first L layers, then the final norm and head, against the
    oracle's forward with the same limit -- through the batched prefill (a
    prompt of >= 4 tokens) and the captured decode step of L layers (one
    token); then the full forward resumes with the cache the partial calls
    left (later layers unwritten at those positions, as in the reference)."""
    print(f"[case] forward maxLayers vs oracle weights={wt}", flush=True)
    model, ref, cfg = make_pair(ctx, tiny(wt, wt, n_layers=6), 430 + wt)
    prompt = [int(t) for t in synth.random_tokens(431, 12, cfg["vocab_size"])]
    worst = 0.0
    g, _ = model.forward(prompt, 0, max_layers=4)
    assert model.layers_used == 4
    r = ref.forward(prompt, 0, max_layers=4)
    worst = max(worst, float(np.abs(g - r).max()))
    for i, t in enumerate(synth.random_tokens(432, 6, cfg["vocab_size"])):
        L = (4, 2, 4, 0, 9, -1)[i]
        g, nxt = model.forward([int(t)], 12 + i, max_layers=L)
        assert model.layers_used == (6 if L in (0, 9) else max(L, 0))
        r = ref.forward([int(t)], 12 + i, max_layers=L)
        worst = max(worst, float(np.abs(g - r).max()))
        assert nxt == int(np.argmax(g))
    g, _ = model.forward([7, 8, 9, 10, 11], 18)  # full layers over the mixed cache
    r = ref.forward([7, 8, 9, 10, 11], 18)
    worst = max(worst, float(np.abs(g - r).max()))
    print(f"  worst max-abs {worst:.2e}")
    assert worst <= LOGIT_TOL
    model.free()
    ref.close()


@pytest.mark.parametrize("batched", [True, False])
def test_self_speculative_equals_greedy(ctx, batched):
    """SelfSpeculativeDecoder's own scheme (speculative.js:58-204, draft =
    the first draftLayers layers of the target, speculative.js:96-111) in
    greedy mode emits the model's greedy tokens; with draftLayers = nLayers
    the draft is the full model and every draft is accepted."""
    print(f"[case] self-speculative batched={batched}", flush=True)
    tcfg = tiny(TYPE_Q4_0, TYPE_Q4_0, n_layers=4, max_seq=200)
    model = synth.build(ctx, tcfg, 440)
    prompt = [int(t) for t in synth.random_tokens(441, 16, tcfg["vocab_size"])]
    n_gen = 40
    ref = _greedy(model, prompt, n_gen)
    out, st = self_speculative_generate(model, prompt, n_gen, draft_layers=2, draft_count=4,
                                        eos_ids=(), batched_verify=batched)
    print(f"  draft 2 layers: {st}")
    assert list(out[:n_gen]) == ref and len(out) in (n_gen, n_gen + 1)
    assert st["rounds"] > 0 and st["drafted"] >= st["rounds"]
    out, st = self_speculative_generate(model, prompt, n_gen, draft_layers=4, draft_count=4,
                                        eos_ids=(), batched_verify=batched)
    print(f"  draft 4 layers: {st}")
    assert list(out[:n_gen]) == ref
    assert st["accepted"] >= st["drafted"] - 2  # near-ties between batched and single rows
    # the cache after the run equals a plain greedy run's over the same tokens
    n = len(out)
    a, _ = model.forward([int(out[-1])], len(prompt) + n - 1)
    model.reset_cache()
    model.forward(prompt, 0)
    model.forward([int(t) for t in out[:-1]], len(prompt))
    b, _ = model.forward([int(out[-1])], len(prompt) + n - 1)
    assert float(np.abs(a - b).max()) <= LOGIT_TOL
    eos = ref[7]
    out, _ = self_speculative_generate(model, prompt, n_gen, draft_layers=2, eos_ids=(eos,),
                                       batched_verify=batched)
    assert list(out) == ref[:ref.index(eos) + 1]
    with pytest.raises(PbxError):
        self_speculative_generate(model, prompt, n_gen, draft_layers=0)
    with pytest.raises(PbxError):
        self_speculative_generate(model, prompt, 190, draft_layers=2)  # beyond max_seq
    model.free()


def _spec_replay(ref, prompt, max_tokens, draft_layers, draft_count):
    """SelfSpeculativeDecoder.generate (speculative.js:58-204) in greedy mode
    over the oracle: draft with forward([t], pos, {maxLayers}) and argmax,
    roll the cache back, verify one token at a time with the full model,
    accept the agreeing prefix, take the verifier's token at the first
    disagreement (rolling back past it) or a bonus token.  Returns the
    generated tokens, the stats the reference counts and the smallest
    top-2 logit gap of any decision (a near-tie could flip on the GPU)."""
    ref.rollback(0)
    out, pos, gaps = list(prompt), len(prompt), []

    def pick(logits):
        srt = np.sort(logits)
        gaps.append(float(srt[-1] - srt[-2]))
        return oracle.argmax(logits)

    nxt = pick(ref.forward(prompt, 0))
    out.append(nxt)
    generated, rounds, drafted, accepted_all = 1, 0, 0, 0
    while generated < max_tokens:
        draft, dpos = [nxt], pos
        for d in range(draft_count):
            if generated + d >= max_tokens:
                break
            draft.append(pick(ref.forward([draft[-1]], dpos, max_layers=draft_layers)))
            dpos += 1
        nd = len(draft) - 1
        if nd == 0:
            break
        drafted += nd
        rounds += 1
        ref.rollback(pos)
        acc = 0
        for d in range(nd):
            vp = pick(ref.forward([draft[d]], pos + d))
            out.append(vp)
            generated += 1
            if vp == draft[d + 1]:
                acc += 1
            else:
                ref.rollback(pos + d + 2)
                break
        if acc == nd:
            b = pick(ref.forward([draft[-1]], pos + nd))
            out.append(b)
            generated += 1
            pos += nd + 1
            nxt = b
        else:
            pos += acc + 1
            nxt = out[-1]
        accepted_all += acc
    return out[len(prompt):], dict(rounds=rounds, drafted=drafted, accepted=accepted_all), min(gaps)


@pytest.mark.parametrize("batched", [True, False])
def test_self_speculative_stats_match_reference_replay(ctx, batched):
    """The self-draft statistics, not just the tokens: the GPU's
    self-speculative run (draft = the first 2 of 4 layers, 4 drafts a
    round) against a replay of speculative.js:58-204 over the oracle with
    the same weights.  Rounds, drafted and accepted counts (the reference's
    acceptanceRate) and every emitted token are equal; a wrong draft chain
    (layer limit, cache left stale by a rollback) changes them even where
    the greedy output stays the same.  Weights N(0, 0.05): with 0.02 the
    layers barely move the residual stream and every draft is accepted;
    here 28 of 47 are, over 12 rounds (the replay's smallest top-2 gap is
    1.9e-2, far above the logit tolerance)."""
    print(f"[case] self-speculative stats vs oracle replay batched={batched}", flush=True)
    tcfg = tiny(TYPE_Q4_0, TYPE_Q4_0, n_layers=4, max_seq=200, weight_std=0.05)
    model, ref, tcfg = make_pair(ctx, tcfg, 440)
    prompt = [int(t) for t in synth.random_tokens(441, 16, tcfg["vocab_size"])]
    n_gen = 40
    want, want_st, gap = _spec_replay(ref, prompt, n_gen, 2, 4)
    out, st = self_speculative_generate(model, prompt, n_gen, draft_layers=2, draft_count=4,
                                        eos_ids=(), batched_verify=batched)
    got = {k: st[k] for k in ("rounds", "drafted", "accepted")}
    print(f"  GPU {got} vs replay {want_st}; smallest decision gap {gap:.2e}")
    assert gap > LOGIT_TOL, "a near-tie decision: pick another seed"
    assert list(out) == want
    assert got == want_st
    model.free()
    ref.close()


def test_speculative_errors(ctx):
    print("[case] speculative errors", flush=True)
    cfg = tiny(TYPE_Q4_0, TYPE_Q4_0, max_seq=64)
    a = synth.build(ctx, cfg, 420)
    b = synth.build(ctx, cfg, 421)
    with pytest.raises(PbxError):
        speculative_generate(a, a, [1, 2, 3], 4)            # shared cache
    with pytest.raises(PbxError):
        speculative_generate(a, b, [1, 2, 3], 4, draft_count=0)
    with pytest.raises(PbxError):
        speculative_generate(a, b, [1, 2, 3], 60)           # beyond max_seq
    with pytest.raises(PbxError):
        a.forward_batch([1, cfg["vocab_size"]], 0)
    with pytest.raises(PbxError):
        a.forward_batch([1, 2], cfg["max_seq"] - 1)
    a.free()
    b.free()


@pytest.mark.parametrize("wt", [TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_1, TYPE_F16])
@pytest.mark.parametrize("n", [256, 300, 512])
def test_gate_up_swiglu_epilogue(ctx, monkeypatch, wt, n):
    """The batched forward's gate|up GEMM with silu(gate) * up in its epilogue
    (hidden 8192: 64-row tiles at 256 and 300 rows -- the last tile partly
    padding --, 128-row tiles at 512, no K split)
    gives bit-identical logits to the same GEMM storing gate and up for the
    separate SwiGLU pass (PBX_GEMM_SWIGLU=0), and the oracle's logits within
    the usual tolerance (llama.js:326-336)."""
    cfg = dict(dim=512, hidden_dim=8192, n_layers=1, n_heads=8, n_kv_heads=2, vocab_size=512,
               max_seq=n + 8, weight_type=wt, embed_type=TYPE_Q8_0, rope_theta=500000.0)
    print(f"[case] swiglu epilogue wt={wt} n={n}", flush=True)
    model, ref, cfg = make_pair(ctx, cfg, 7000 + wt)
    prompt = [int(t) for t in synth.random_tokens(7100 + n, n, cfg["vocab_size"])]
    monkeypatch.delenv("PBX_GEMM_SWIGLU", raising=False)
    l_sw, _ = model.forward(prompt, 0)
    monkeypatch.setenv("PBX_GEMM_SWIGLU", "0")
    model.reset_cache()
    l_sep, _ = model.forward(prompt, 0)
    assert np.array_equal(l_sw, l_sep)
    err = float(np.abs(l_sw - ref.forward(prompt, 0)).max())
    print(f"  bit-identical to the separate pass; oracle max-abs {err:.2e}", flush=True)
    assert err <= LOGIT_TOL
    model.free()
    ref.close()
