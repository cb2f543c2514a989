"""End-to-end parity of the on-GPU decode step against the llama.js forward
restated in the oracle (llama.js:204-371, llama-streaming.js:505-606).

Bars: logits within 2e-3 max-abs of the oracle at every checked position;
greedy tokens identical to the oracle's argmax (a mismatch is accepted only
where the oracle's own top logits are closer than that tolerance).
"""
import numpy as np
import pytest

import oracle
from purebee_amd import PbxError, synth
from purebee_amd.native import TYPE_F16, TYPE_F32, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q6_K, TYPE_Q8_0
from tests.e2e_util import LOGIT_TOL, check_greedy, make_pair

pytestmark = pytest.mark.gpu

# Switches that select other decode kernels at model creation; the tests
# that check which kernels a step launches clear them first, so they hold
# whatever the caller's environment selects.
PATH_SWITCHES = ("PBX_FFN", "PBX_QKV_ATTN", "PBX_ATTN_O", "PBX_GEMV_INT", "PBX_SMALL_STEP")


@pytest.fixture
def default_paths(monkeypatch):
    for k in PATH_SWITCHES:
        monkeypatch.delenv(k, raising=False)
    return monkeypatch


def tiny(weight_type, embed_type, **kw):
    cfg = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=1000,
               max_seq=64, weight_type=weight_type, embed_type=embed_type, rope_theta=10000.0)
    cfg.update(kw)
    return cfg


def run_prompt_then_greedy(ctx, cfg, n_prompt, n_gen, seed):
    model, ref, cfg = make_pair(ctx, cfg, seed)
    prompt = synth.random_tokens(seed + 1, n_prompt, cfg["vocab_size"])
    # prefill: the reference processes the prompt in one forward (llama.js:465)
    ref_logits = ref.forward(prompt, 0)
    logits, nxt = model.forward(prompt, 0)
    err = float(np.abs(logits - ref_logits).max())
    assert err <= LOGIT_TOL, f"prefill logits max-abs {err:.2e}"
    assert nxt == int(np.argmax(logits))
    first = oracle.argmax(ref_logits)
    if nxt != first:
        assert ref_logits[first] - ref_logits[nxt] < LOGIT_TOL
    # greedy decode on the GPU, then walk it through the oracle
    toks, last = model.generate(nxt, n_prompt, n_gen, want_logits=True)
    exact, ties = check_greedy(ref, toks, nxt, n_prompt)
    # the oracle has now consumed the same tokens: compare the final logits
    ref_last = ref.forward([int(toks[-1])], n_prompt + n_gen)
    gpu_last, _ = model.forward([int(toks[-1])], n_prompt + n_gen)
    err2 = float(np.abs(gpu_last - ref_last).max())
    assert err2 <= LOGIT_TOL, f"final logits max-abs {err2:.2e}"
    model.free()
    ref.close()
    return exact, ties, err, err2


@pytest.mark.parametrize("wt,et", [(TYPE_Q4_0, TYPE_Q4_0), (TYPE_Q8_0, TYPE_Q8_0),
                                   (TYPE_Q8_0, TYPE_F32), (TYPE_F32, TYPE_F32),
                                   (TYPE_Q4_1, TYPE_Q4_1), (TYPE_Q4_0, TYPE_Q6_K),
                                   (TYPE_F16, TYPE_F16)])
def test_tiny_model_prefill_and_greedy(ctx, wt, et):
    print(f"[case] tiny model weights={wt} embed={et}", flush=True)
    exact, ties, e1, e2 = run_prompt_then_greedy(ctx, tiny(wt, et), 8, 24, seed=50 + wt)
    print(f"  exact={exact} ties={ties} prefill_err={e1:.1e} final_err={e2:.1e}")
    assert exact >= 22


def test_untied_head_and_small_head_dim(ctx):
    print("[case] untied head, head_dim 48", flush=True)
    cfg = tiny(TYPE_Q8_0, TYPE_F32, dim=288, hidden_dim=768, n_heads=6, n_kv_heads=6,
               output_type=TYPE_Q4_0)
    exact, ties, e1, e2 = run_prompt_then_greedy(ctx, cfg, 5, 12, seed=77)
    assert exact >= 10


def test_stories15m_shape(ctx):
    """config: stories15M-shaped, Q8_0 layers, f32 embedding / LM head, at its
    workload's full length: a 16-token prompt, then 128 greedy steps, every
    step's choice walked through the oracle."""
    print("[case] stories15m 16-token prompt + 128 greedy", flush=True)
    exact, ties, e1, e2 = run_prompt_then_greedy(ctx, "stories15m", 16, 128, seed=1000)
    print(f"  exact={exact} ties={ties} prefill_err={e1:.1e} final_err={e2:.1e}")
    assert exact >= 126


def test_smollm2_shape(ctx):
    """config: SmolLM2-135M-shaped, GQA 9/3, tied Q8_0 embedding, at its
    workload's full length: a 32-token prompt, then 256 greedy steps."""
    print("[case] smollm2 32-token prompt + 256 greedy", flush=True)
    exact, ties, e1, e2 = run_prompt_then_greedy(ctx, "smollm2_135m", 32, 256, seed=2000)
    print(f"  exact={exact} ties={ties} prefill_err={e1:.1e} final_err={e2:.1e}")
    assert exact >= 252


def test_llama1b_shape(ctx):
    """config: Llama-3.2-1B-shaped Q4_0 (tied 128256x2048 Q4_0 head, theta 5e5)."""
    print("[case] llama32_1b 8-token prompt + 16 greedy", flush=True)
    exact, ties, e1, e2 = run_prompt_then_greedy(ctx, "llama32_1b", 8, 16, seed=3000)
    print(f"  exact={exact} ties={ties} prefill_err={e1:.1e} final_err={e2:.1e}")
    assert exact >= 15


def test_llama1b_shape_q4_1(ctx):
    """Llama-3.2-1B shapes with Q4_1 layer matrices and a tied Q4_1 head
    (the wide GEMV kernels and the row-batched prefill on Q4_1)."""
    print("[case] llama32_1b q4_1 6-token prompt + 8 greedy", flush=True)
    cfg = dict(synth.CONFIGS["llama32_1b"], weight_type=TYPE_Q4_1, embed_type=TYPE_Q4_1)
    exact, ties, e1, e2 = run_prompt_then_greedy(ctx, cfg, 6, 8, seed=3100)
    print(f"  exact={exact} ties={ties} prefill_err={e1:.1e} final_err={e2:.1e}")
    assert exact >= 7


def test_teacher_forced_logits_every_step(ctx):
    print("[case] teacher-forced per-step logits", flush=True)
    model, ref, cfg = make_pair(ctx, tiny(TYPE_Q4_0, TYPE_Q4_0, n_layers=3), 91)
    toks = synth.random_tokens(92, 20, cfg["vocab_size"])
    worst = 0.0
    for p, t in enumerate(toks):
        g, _ = model.forward([int(t)], p)
        r = ref.forward([int(t)], p)
        worst = max(worst, float(np.abs(g - r).max()))
    assert worst <= LOGIT_TOL, worst
    model.free()
    ref.close()


def test_cache_rollback_and_reset(ctx):
    """rollbackCache / resetCache semantics (llama-streaming.js:828-862):
    after rolling back to p, re-running positions >= p reproduces the logits."""
    print("[case] rollback/reset", flush=True)
    model, ref, cfg = make_pair(ctx, tiny(TYPE_Q8_0, TYPE_Q8_0), 93)
    toks = [int(t) for t in synth.random_tokens(94, 12, cfg["vocab_size"])]
    for p, t in enumerate(toks):          # one token per forward: the decode step
        a, _ = model.forward([t], p)
    model.forward([5, 6, 7], 12)          # extend past 12 ...
    model.rollback(12)                    # ... and drop it again
    b, _ = model.forward([toks[-1]], 11)  # re-run position 11
    assert np.array_equal(a, b)
    model.reset_cache()
    for p, t in enumerate(toks):
        c, _ = model.forward([t], p)
    assert np.array_equal(a, c)
    # the prompt in one call (the batched forward) equals the same tokens fed
    # one at a time, and is itself deterministic
    model.reset_cache()
    d, _ = model.forward(toks, 0)
    assert float(np.abs(a - d).max()) <= 1e-4
    model.reset_cache()
    e, _ = model.forward(toks, 0)
    assert np.array_equal(d, e)
    model.free()
    ref.close()


@pytest.mark.parametrize("mode,heads,kv,steps", [
    ("split", 64, 64, 160),   # 4 splits: 160 positions take two tiles per split
    ("head", 64, 64, 160),    # head_dim 32
    ("head", 32, 8, 560),     # head_dim 64, GQA 4:1, past one 512-position chunk
])
def test_attention_kernels_match_one_workgroup_per_head(ctx, monkeypatch, mode, heads, kv, steps):
    """The decode attention kernels against the one-workgroup-per-head kernel
    and the oracle: split-position attention (KV group x position split,
    online softmax over 32-position tiles, combine kernel) and the per-head
    flash-decoding kernel (eight waves of 64 positions merged in LDS, chunks
    of 512 positions)."""
    print(f"[case] attention {mode} vs per-head, {heads}/{kv} heads, {steps} positions", flush=True)
    cfg = tiny(TYPE_Q8_0, TYPE_Q8_0, dim=2048, hidden_dim=256, n_layers=1, n_heads=heads,
               n_kv_heads=kv, vocab_size=512, max_seq=max(256, steps + 8))
    monkeypatch.setenv("PBX_ATTENTION", mode)
    under, ref, cfg = make_pair(ctx, cfg, 97)
    monkeypatch.setenv("PBX_ATTENTION", "decode")
    one = synth.build(ctx, cfg, 97)
    monkeypatch.delenv("PBX_ATTENTION")
    toks = [int(t) for t in synth.random_tokens(98, steps, cfg["vocab_size"])]
    worst = 0.0
    for p, t in enumerate(toks):
        a, _ = under.forward([t], p)
        b, _ = one.forward([t], p)
        worst = max(worst, float(np.abs(a - b).max()))
    r = ref.forward(toks, 0)
    err = float(np.abs(a - r).max())
    print(f"  {mode} vs per-head max-abs {worst:.2e}, vs oracle {err:.2e}")
    assert worst <= 1e-4
    assert err <= LOGIT_TOL
    under.free()
    one.free()
    ref.close()


@pytest.mark.parametrize("ipt,qa", [(1, True), (2, True), (1, False), (2, False), (4, False)])
def test_fused_attention_o_matches_separate_o(ctx, default_paths, ipt, qa):
    """Decode with the o projection fused into the cached head attention
    (workgroup (head, part) adds W_o[rows, head] o_h for its 256 * ipt rows
    into a 64-bit 2^-32 fixed-point update; the gate|up GEMV adds the update
    to its input, the down GEMV folds it into the residual and clears it)
    against the same model with the separate o GEMV and against the oracle,
    over 100 positions (past the attention's two speculative 32-position
    slots) on two layers.  qa: the q|k|v GEMV in the same launch
    (pbx_qkvr_attn_o_c1: the attention workgroups wait for the GEMV's
    epoch-tagged q, k and v cells of their head)."""
    monkeypatch = default_paths
    print(f"[case] fused attention + o, ipt {ipt}, q|k|v in the launch {qa}, 2048/8192, "
          f"32/8 heads, 100 positions", flush=True)
    cfg = tiny(TYPE_Q4_0, TYPE_Q4_0, dim=2048, hidden_dim=8192, n_layers=2, n_heads=32,
               n_kv_heads=8, vocab_size=512, max_seq=256)
    monkeypatch.setenv("PBX_ATTN_O", str(ipt))
    monkeypatch.setenv("PBX_QKV_ATTN", "1" if qa else "0")
    fused, ref, cfg = make_pair(ctx, cfg, 101)
    monkeypatch.setenv("PBX_ATTN_O", "0")
    plain = synth.build(ctx, cfg, 101)
    monkeypatch.delenv("PBX_ATTN_O")
    monkeypatch.delenv("PBX_QKV_ATTN")
    toks = [int(t) for t in synth.random_tokens(102, 100, cfg["vocab_size"])]
    worst = 0.0
    for p, t in enumerate(toks):
        a, _ = fused.forward([t], p)
        b, _ = plain.forward([t], p)
        worst = max(worst, float(np.abs(a - b).max()))
    r = ref.forward(toks, 0)
    err = float(np.abs(a - r).max())
    kern = {k for _, k, _, _ in fused.profile(toks[-1], len(toks), 1)}
    plain_kern = {k for _, k, _, _ in plain.profile(toks[-1], len(toks), 1)}
    print(f"  fused vs separate max-abs {worst:.2e}, vs oracle {err:.2e}")
    assert (f"pbx_qkvr_attn_o_r{4 * ipt}c{ipt}" if qa else f"pbx_attention_o_c{ipt}") in kern
    # with both joins (q|k|v + attention, 512-row o parts) the FFN is one
    # launch too; otherwise gate|up reads the pending update itself
    ffn = "pbx_ffn_q4_d2048_h8192" if qa and ipt == 2 else "pbx_dk_q4_i8x8b1w8p4_gua"
    assert ffn in kern
    assert "pbx_attention_head_c" in plain_kern
    assert worst <= 1e-4
    assert err <= LOGIT_TOL
    fused.free()
    plain.free()
    ref.close()


def test_fused_qkv_attention_long_context(ctx, default_paths):
    """The q|k|v GEMV and the attention + o projection in one launch past
    512 cached positions, where the newest position falls in the
    attention's second 512-position chunk (its k and v come from the
    GEMV's cells there too): a 1-layer model prefilled with 520 tokens,
    then 12 decode steps, against the same model launching the two kernels
    separately, and the greedy tokens of 13 on-device steps (an 8-step and a
    4-step graph launch, then one step) against it."""
    monkeypatch = default_paths
    print("[case] q|k|v + attention in one launch, 1 layer, positions 520..531", flush=True)
    cfg = tiny(TYPE_Q4_0, TYPE_Q4_0, dim=2048, hidden_dim=8192, n_layers=1, n_heads=32,
               n_kv_heads=8, vocab_size=512, max_seq=1024)
    fused = synth.build(ctx, cfg, 111)
    monkeypatch.setenv("PBX_QKV_ATTN", "0")
    plain = synth.build(ctx, cfg, 111)
    monkeypatch.delenv("PBX_QKV_ATTN")
    toks = [int(t) for t in synth.random_tokens(112, 532, cfg["vocab_size"])]
    fused.forward(toks[:520], 0, want_logits=False)
    plain.forward(toks[:520], 0, want_logits=False)
    worst = 0.0
    for p in range(520, 532):
        a, _ = fused.forward([toks[p]], p)
        b, _ = plain.forward([toks[p]], p)
        assert np.isfinite(a).all()
        worst = max(worst, float(np.abs(a - b).max()))
    ga = fused.generate(toks[-1], 531, 13)
    gb = plain.generate(toks[-1], 531, 13)
    kern = {k for _, k, _, _ in fused.profile(toks[-1], 531, 1)}
    print(f"  max-abs {worst:.2e}; greedy {list(ga)} / {list(gb)}")
    assert any(k.startswith("pbx_qkvr_attn_o_") for k in kern)
    assert worst <= 1e-4
    assert list(ga) == list(gb)
    fused.free()
    plain.free()


def test_non_finite_activation_propagates(ctx):
    """A token whose embedding row holds a Q4_0 block with a +inf scale: the
    reference's activations for it are then +-inf and NaN (inf * 0 for the
    block's zero codes), so its logits and those of every later position
    (whose attention reads its K/V) are NaN (llama.js:204-371).  The decode
    step must give NaN there, through the attention with the o projection
    fused (a non-finite product sets the residual element to NaN instead of
    entering the fixed-point update), and so must the 5-row verify, through
    the down projection split over K slices (a non-finite slice marks its
    cell); the rows before the poisoned one stay finite and at the logit
    tolerance."""
    print("[case] non-finite embedding: decode step and 5-row verify", flush=True)
    from purebee_amd.native import T_TOKEN_EMBD
    cfg = tiny(TYPE_Q4_0, TYPE_Q4_0, dim=2048, hidden_dim=8192, n_layers=2, n_heads=32,
               n_kv_heads=8, vocab_size=512, max_seq=64)
    bad = 7
    spec = synth.tensor_specs(cfg)[0]
    assert spec[0] == T_TOKEN_EMBD
    emb = np.array(synth.make_tensor(spec, 103, 0), np.uint8, copy=True)
    row_bytes = (cfg["dim"] // 32) * 18
    emb[bad * row_bytes: bad * row_bytes + 2] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)
    emb_f = oracle.dequant(TYPE_Q4_0, emb, cfg["vocab_size"] * cfg["dim"])
    assert np.isinf(emb_f[bad * cfg["dim"]: (bad + 1) * cfg["dim"]]).any()
    toks = [1, 2, bad, 3, 4]
    for mode in ("decode", "verify"):
        model, ref, cfg = make_pair(ctx, cfg, 103)
        model.set_tensor(T_TOKEN_EMBD, -1, emb)
        ref.set(T_TOKEN_EMBD, -1, emb_f)
        r = [ref.forward([t], p) for p, t in enumerate(toks)]
        if mode == "decode":
            g = [model.forward([t], p)[0] for p, t in enumerate(toks)]
        else:
            lg, _ = model.forward_batch(toks, 0)
            g = list(lg)
        for p in range(len(toks)):
            if p < 2:
                # the LM head is the tied embedding: the poisoned token's own
                # logit is non-finite in every row, the others are finite
                keep = np.arange(cfg["vocab_size"]) != bad
                assert not np.isfinite(r[p][bad]) and not np.isfinite(g[p][bad]), f"{mode} {p}"
                assert np.isfinite(r[p][keep]).all(), f"oracle row {p}"
                assert np.isfinite(g[p][keep]).all(), f"{mode} row {p}"
                err = float(np.abs(g[p][keep] - r[p][keep]).max())
                assert err <= LOGIT_TOL, f"{mode} row {p}: {err:.2e}"
            else:
                assert np.isnan(r[p]).all(), f"oracle row {p}"
                assert np.isnan(g[p]).all(), f"{mode} row {p}: {np.isfinite(g[p]).sum()} finite"
        print(f"  {mode}: rows 0-1 finite, rows 2-4 NaN")
        model.free()
        ref.close()


def test_handoff_wait_timeout_is_reported(ctx, default_paths):
    """The bounded wait of the joined q|k|v + attention launch: when the
    cells it waits for never carry its tag (forced from the host by the test
    hook, which offsets the tag the attention workgroups expect and caps
    their polls at 64), every kernel still exits, and forward, generate and
    the layer-limited forward fail with PBX_ETIMEOUT instead of returning
    NaN logits or tokens picked from them.  With the hook removed the same
    positions give the logits of an untouched run again, bit for bit."""
    print("[case] forced hand-off timeout: forward / generate report PBX_ETIMEOUT", flush=True)
    from purebee_amd.native import ETIMEOUT
    cfg = tiny(TYPE_Q4_0, TYPE_Q4_0, dim=2048, hidden_dim=8192, n_layers=2, n_heads=32,
               n_kv_heads=8, vocab_size=512, max_seq=64)
    model = synth.build(ctx, cfg, 121)
    toks = [int(t) for t in synth.random_tokens(122, 6, cfg["vocab_size"])]
    good = [model.forward([t], p)[0] for p, t in enumerate(toks)]
    kern = {k for _, k, _, _ in model.profile(toks[-1], len(toks), 1)}
    assert any(k.startswith("pbx_qkvr_attn_o_") for k in kern)
    model.rollback(4)
    model.test_handoff(1, 1, 64)
    with pytest.raises(PbxError) as e:
        model.forward([toks[4]], 4)
    assert e.value.code == ETIMEOUT and "gave up" in str(e.value)
    with pytest.raises(PbxError) as e:
        model.generate(toks[4], 4, 3)
    assert e.value.code == ETIMEOUT
    # only layer 1 waits: a forward through the first layer alone succeeds
    model.rollback(4)
    lg, _ = model.forward([toks[4]], 4, max_layers=1)
    assert np.isfinite(lg).all()
    model.test_handoff(-1, 0, 0)
    model.rollback(4)
    again = [model.forward([t], 4 + i)[0] for i, t in enumerate(toks[4:])]
    assert np.array_equal(again[0], good[4]) and np.array_equal(again[1], good[5])
    print("  timeouts reported; normal launch restored bit for bit")
    model.free()


def test_small_step_matches_per_layer_launches(ctx, default_paths):
    """Small Q8_0 models run every layer of a decode step in one launch
    (pbx_small_step_q8: the phases of a layer hand their outputs on through
    tagged cells).  stories15M-shaped, after a 16-token prompt: the step's
    kernels are that launch, the LM head and the argmax; 24 greedy steps give
    the tokens of the per-layer launches (a model made with PBX_SMALL_STEP=0)
    and the last step's logits agree within 5e-4 (the dot products are summed
    in another order); a forward through the first 3 layers
    (llama-streaming.js maxLayers) agrees as well."""
    monkeypatch = default_paths
    print("[case] stories15m small-step launch vs per-layer launches", flush=True)
    cfg = synth.CONFIGS["stories15m"]
    small = synth.build(ctx, cfg, 1300)
    monkeypatch.setenv("PBX_SMALL_STEP", "0")
    per = synth.build(ctx, cfg, 1300)
    monkeypatch.delenv("PBX_SMALL_STEP")
    prompt = [int(t) for t in synth.random_tokens(1301, 16, cfg["vocab_size"])]
    _, n1 = small.forward(prompt, 0)
    _, n2 = per.forward(prompt, 0)
    assert n1 == n2
    kern = [k for _, k, _, _ in small.profile(n1, 16, 1)]
    assert kern[0] == "pbx_small_step_q8" and len(kern) == 3, kern
    assert "pbx_small_step_q8" not in [k for _, k, _, _ in per.profile(n2, 16, 1)]
    small.rollback(16)
    per.rollback(16)
    t1, l1 = small.generate(n1, 16, 24, want_logits=True)
    t2, l2 = per.generate(n2, 16, 24, want_logits=True)
    err = float(np.abs(np.asarray(l1) - np.asarray(l2)).max())
    print(f"  24 steps: max-abs logit difference {err:.2e}")
    assert list(t1) == list(t2) and err <= 5e-4
    a, _ = small.forward([int(t1[-1])], 40, max_layers=3)
    b, _ = per.forward([int(t2[-1])], 40, max_layers=3)
    err3 = float(np.abs(a - b).max())
    print(f"  3 of 6 layers: {err3:.2e}")
    assert err3 <= 5e-4
    small.free()
    per.free()


def test_small_step_wait_timeout_is_reported(ctx, default_paths):
    """The bounded waits of the small-model step: with the test hook skewing
    the tag that layer 1's waits expect (64 polls each), every workgroup still
    finishes and forward and generate fail with PBX_ETIMEOUT; a forward
    through layer 0 alone succeeds, and without the hook the logits are those
    of an untouched run, bit for bit."""
    print("[case] small-step forced wait timeout", flush=True)
    from purebee_amd.native import ETIMEOUT
    cfg = tiny(TYPE_Q8_0, TYPE_Q8_0, n_layers=2)
    model = synth.build(ctx, cfg, 131)
    toks = [int(t) for t in synth.random_tokens(132, 6, cfg["vocab_size"])]
    good = [model.forward([t], p)[0] for p, t in enumerate(toks)]
    assert "pbx_small_step_q8" in {k for _, k, _, _ in model.profile(toks[-1], len(toks), 1)}
    model.rollback(4)
    model.test_handoff(1, 1, 64)
    with pytest.raises(PbxError) as e:
        model.forward([toks[4]], 4)
    assert e.value.code == ETIMEOUT and "gave up" in str(e.value)
    with pytest.raises(PbxError) as e:
        model.generate(toks[4], 4, 3)
    assert e.value.code == ETIMEOUT
    model.rollback(4)
    lg, _ = model.forward([toks[4]], 4, max_layers=1)
    assert np.isfinite(lg).all()
    model.test_handoff(-1, 0, 0)
    model.rollback(4)
    again = [model.forward([t], 4 + i)[0] for i, t in enumerate(toks[4:])]
    assert np.array_equal(again[0], good[4]) and np.array_equal(again[1], good[5])
    print("  timeouts reported; normal launch restored bit for bit")
    model.free()


@pytest.mark.parametrize("wt,et,dim,hidden,vocab", [(TYPE_Q4_0, TYPE_Q4_0, 2048, 1024, 40000),
                                                    (TYPE_Q4_0, TYPE_Q6_K, 2048, 1024, 40000),
                                                    (TYPE_Q8_0, TYPE_Q8_0, 2048, 1024, 512),
                                                    (TYPE_Q4_0, TYPE_Q4_0, 4096, 8192, 512),
                                                    (TYPE_Q8_0, TYPE_Q8_0, 4096, 4096, 512)])
def test_integer_limb_kernels_match_float_kernels(ctx, monkeypatch, wt, et, dim, hidden, vocab):
    """The GEMVs on integer limbs (v_dot4 over a fixed-point activation)
    against the float-unpack kernels and the oracle: gate|up for Q4_0 and
    Q8_0, and for Q4_0 also qkv, o, down and the lm head (K = 2048: a loop
    over 1250 row tiles in 512 workgroups; a Q6_K tied head on its own
    loop), with one, two and four 64-block groups per lane (K = 2048, 4096,
    8192)."""
    print(f"[case] integer-limb vs float kernels, type {wt}, embed {et}, dim {dim}, "
          f"hidden {hidden}, vocab {vocab}", flush=True)
    heads = dim // 128
    cfg = tiny(wt, et, dim=dim, hidden_dim=hidden, n_layers=1, n_heads=heads,
               n_kv_heads=heads // 4, vocab_size=vocab, max_seq=64)
    fast, ref, cfg = make_pair(ctx, cfg, 99)
    monkeypatch.setenv("PBX_GEMV_INT", "0")
    slow = synth.build(ctx, cfg, 99)
    monkeypatch.delenv("PBX_GEMV_INT")
    toks = [int(t) for t in synth.random_tokens(100, 20, cfg["vocab_size"])]
    worst = 0.0
    for p, t in enumerate(toks):
        a, _ = fast.forward([t], p)
        b, _ = slow.forward([t], p)
        worst = max(worst, float(np.abs(a - b).max()))
    r = ref.forward(toks, 0)
    err = float(np.abs(a - r).max())
    print(f"  int vs float max-abs {worst:.2e}, vs oracle {err:.2e}")
    assert worst <= 1e-4
    assert err <= LOGIT_TOL
    fast.free()
    slow.free()
    ref.close()


def test_q6k_head_copy_follows_rewrites(ctx):
    """A Q6_K head at K = 2048 runs on a lane-packed copy of its codes: a
    head rewritten after the step was built (copy made) gives the same
    logits as a model that held the new head from the start."""
    print("[case] q6_k head copy after a rewrite", flush=True)
    from purebee_amd.native import T_TOKEN_EMBD
    cfg = tiny(TYPE_Q4_0, TYPE_Q6_K, dim=2048, hidden_dim=1024, n_layers=1, n_heads=16,
               n_kv_heads=4, vocab_size=4096, max_seq=16)
    specs = synth.tensor_specs(cfg)
    i = next(k for k, s in enumerate(specs) if s[0] == T_TOKEN_EMBD)
    new = synth.make_tensor(specs[i], 77, i)
    a = synth.build(ctx, cfg, 41)
    a.forward([3], 0)  # builds the step and the copy of the old head
    a.set_tensor(T_TOKEN_EMBD, -1, new)
    b = synth.build(ctx, cfg, 41)
    b.set_tensor(T_TOKEN_EMBD, -1, new)
    la, na = a.forward([5], 0)
    lb, nb = b.forward([5], 0)
    assert np.array_equal(la, lb) and na == nb
    a.free()
    b.free()


def test_model_argument_errors(ctx):
    print("[case] model errors", flush=True)
    cfg = tiny(TYPE_Q4_0, TYPE_Q4_0)
    m = synth.Model(ctx, cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["n_heads"],
                    cfg["n_kv_heads"], cfg["vocab_size"], cfg["max_seq"], TYPE_Q4_0, TYPE_Q4_0)
    with pytest.raises(PbxError) as e:
        m.forward([1, 2], 0)  # nothing uploaded yet
    assert "not set" in str(e.value)
    m.free()
    model, ref, cfg = make_pair(ctx, cfg, 95)
    with pytest.raises(PbxError):
        model.forward([cfg["vocab_size"]], 0)
    with pytest.raises(PbxError):
        model.forward([1], cfg["max_seq"])
    with pytest.raises(PbxError):
        model.generate(1, cfg["max_seq"] - 2, 5)
    with pytest.raises(PbxError):
        synth.Model(ctx, 100, 512, 1, 4, 2, 1000, 64, TYPE_Q4_0, TYPE_Q4_0)  # dim % 32
    model.free()
    ref.close()


def test_gpu_matches_reference_llama_js_fixture(ctx):
    """The GPU decode step against logits the reference's own LlamaRuntime
    produced (tests/golden/llama_tiny.json), f32 weights."""
    from tests.golden import llama_fixture as lf
    print("[case] llama.js golden fixture", flush=True)
    fx = lf.load()
    c = fx["config"]
    m = synth.Model(ctx, c["dim"], c["hiddenDim"], c["nLayers"], c["nHeads"], c["nKvHeads"],
                    c["vocabSize"], c["seqLen"], TYPE_F32, TYPE_F32, rope_theta=c["ropeTheta"])
    for tid, layer, w in lf.weights(fx):
        m.set_tensor(tid, layer, w)
    for st in fx["steps"]:
        logits, nxt = m.forward(st["tokens"], st["pos"])
        want = np.asarray(st["logits"], np.float32)
        assert np.abs(logits - want).max() <= LOGIT_TOL, (st["pos"], np.abs(logits - want).max())
        assert nxt == st["argmax"]
    m.free()
