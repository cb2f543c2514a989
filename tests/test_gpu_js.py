"""The JavaScript drop-ins on the GPU, driven through Node.js exactly as the
reference's callers would use them:

* js/hip-q4.js      -- wasm-q4.js surface (q4_0_matvec, q4_1_matvec, matvec
                       dispatch, lmHead) on raw GGUF Q4_0 / Q4_1 / Q8_0 blocks;
* js/engine-hip.js  -- ExecutionEngine.tensorMulAdd / tensorMulAddQ8 /
                       tensorMul (f32 [K,N] Tensors and quantize.js's
                       QuantizedTensor);
* js/llama-hip.js   -- the resident model: forward / generate / rollback and
                       the greedy speculative decoder.

Inputs and expected outputs are computed here (the oracle, or the C ABI's
own model for end-to-end tokens), passed to Node through files, and the
results read back.  Bars as elsewhere: matvec 1e-3 relative L2, logits 2e-3.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle
import purebee_amd as pb
from purebee_amd import synth
from purebee_amd.native import TYPE_Q4_0, TYPE_Q8_0, speculative_generate
from tests.conftest import rel_l2

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(shutil.which("node") is None, reason="node not installed")]

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "purebee_amd", "js")

PRELUDE = """
const fs = require('fs');
const path = require('path');
const dir = process.argv[2];
const rd = (n, T) => { const b = fs.readFileSync(path.join(dir, n));
  return new T(b.buffer.slice(b.byteOffset, b.byteOffset + b.length)); };
const wr = (n, a) => fs.writeFileSync(path.join(dir, n), Buffer.from(a.buffer, a.byteOffset, a.byteLength));
const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json')));
"""


def run_node(tmp_path, script, meta):
    (tmp_path / "meta.json").write_text(json.dumps(meta))
    (tmp_path / "t.js").write_text(PRELUDE + script)
    r = subprocess.run(["node", str(tmp_path / "t.js"), str(tmp_path)], capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stdout


def test_hip_q4_module_matvec_and_dispatch(tmp_path):
    print("[case] js hip-q4 q4_0_matvec / matvec / lmHead", flush=True)
    N, K = 2048, 2048
    w = pb.synth_normal(501, N * K, 0, 0.02).reshape(N, K)
    raw4 = pb.quantize_q4_0(w)
    raw8 = pb.quantize_q8_0(w)
    raw41 = pb.quantize_q4_1(w)
    x = pb.synth_normal(502, K)
    emb = pb.synth_normal(503, 1000 * K, 0, 0.02)
    raw4.tofile(tmp_path / "w4.bin")
    raw8.tofile(tmp_path / "w8.bin")
    raw41.tofile(tmp_path / "w41.bin")
    x.tofile(tmp_path / "x.bin")
    emb.tofile(tmp_path / "emb.bin")
    out = run_node(tmp_path, f"""
const q = require({os.path.join(JS, 'hip-q4.js')!r});
if (!q.init()) throw new Error('init failed');
const x = rd('x.bin', Float32Array), w4 = rd('w4.bin', Uint8Array), w8 = rd('w8.bin', Uint8Array);
const xcopy = Float32Array.from(x);
const y4 = q.q4_0_matvec(x, w4, meta.N, meta.K);
const y4b = q.q4_0_matvec(x, w4, meta.N, meta.K);   // resident second call
const y8 = q.matvec(x, w8, 8, meta.N, meta.K);
const w41 = rd('w41.bin', Uint8Array);
const y41 = q.q4_1_matvec(x, w41, meta.N, meta.K);
const y41d = q.matvec(x, w41, 3, meta.N, meta.K);   // quantizedMatvec type 3
let rep41 = true; for (let i = 0; i < y41.length; i++) if (y41[i] !== y41d[i]) rep41 = false;
wr('y41.bin', y41);
const lm = q.lmHead(x, rd('emb.bin', Float32Array), 1000, meta.K);
wr('y4.bin', y4); wr('y8.bin', y8); wr('lm.bin', lm);
let errs = [];
try {{ q.matvec(x, w4, 1, meta.N, meta.K); }} catch (e) {{ errs.push(e.message); }}
try {{ q.matvec(x, w4, 6, meta.N, meta.K); }} catch (e) {{ errs.push(e.message); }}
let same = true; for (let i = 0; i < x.length; i++) if (x[i] !== xcopy[i]) same = false;
let rep = true; for (let i = 0; i < y4.length; i++) if (y4[i] !== y4b[i]) rep = false;
console.log(JSON.stringify({{errs, same, rep, rep41, supported: q.supported}}));
""", {"N": N, "K": K})
    res = json.loads(out.strip().splitlines()[-1])
    assert res["same"], "input mutated"
    assert res["rep"], "second (resident) call differs"
    assert res["rep41"], "q4_1_matvec and matvec(type 3) differ"
    assert len(res["errs"]) == 2 and all(res["errs"]), res["errs"]
    y4 = np.fromfile(tmp_path / "y4.bin", np.float32)
    y8 = np.fromfile(tmp_path / "y8.bin", np.float32)
    lm = np.fromfile(tmp_path / "lm.bin", np.float32)
    assert rel_l2(y4, oracle.q4_0_matvec_js(x, raw4, N, K)) <= 1e-3
    assert rel_l2(y8, oracle.matvec(TYPE_Q8_0, x, raw8, N, K)) <= 1e-3
    y41 = np.fromfile(tmp_path / "y41.bin", np.float32)
    assert rel_l2(y41, oracle.q4_1_matvec_js(x, raw41, N, K)) <= 1e-3
    ref_lm = emb.reshape(1000, K).astype(np.float64) @ x.astype(np.float64)
    assert rel_l2(lm, ref_lm) <= 1e-3


def test_engine_adapter_linear_ops(tmp_path):
    """tensorMulAdd / tensorMul on f32 [K,N] Tensors and tensorMulAddQ8 on a
    quantize.js QuantizedTensor, through HipEngine and install()."""
    print("[case] js engine-hip tensorMulAdd / tensorMulAddQ8", flush=True)
    M, K, N = 5, 288, 768
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    W = rng.normal(0, 0.02, (K, N)).astype(np.float32)    # reference [K,N]
    b = rng.normal(0, 1, N).astype(np.float32)
    q, sc = pb.quantize_q8_ref(W)                           # quantize.js layout
    x.tofile(tmp_path / "x.bin")
    W.tofile(tmp_path / "W.bin")
    b.tofile(tmp_path / "b.bin")
    q.tofile(tmp_path / "q.bin")
    sc.tofile(tmp_path / "s.bin")
    run_node(tmp_path, f"""
const eng = require({os.path.join(JS, 'engine-hip.js')!r});
const T = eng.PlainTensor;
const fake = {{ engine: {{}} }};
const hip = eng.install(fake);
const x = new T('x', [meta.M, meta.K], rd('x.bin', Float32Array));
const W = new T('W', [meta.K, meta.N], rd('W.bin', Float32Array));
const b = new T('b', [meta.N], rd('b.bin', Float32Array));
fake.engine.cacheWeight(W);
const y = fake.engine.tensorMulAdd(x, W, b, 'y');
const z = fake.engine.tensorMul(x, W, 'z');
const Wq = {{ type: 'q8_0', shape: [meta.K, meta.N], data: rd('q.bin', Int8Array), scales: rd('s.bin', Float32Array) }};
const yq = fake.engine.tensorMulAddQ8(x, Wq, b, 'yq');
if (y.shape[0] !== meta.M || y.shape[1] !== meta.N || y.name !== 'y') throw new Error('bad tensor');
let threw = false;
try {{ fake.engine.tensorMulAdd(new T('bad', [meta.M, meta.K + 1]), W, null, 'o'); }} catch (e) {{ threw = true; }}
if (!threw) throw new Error('dimension mismatch not thrown');
wr('y.bin', y.data); wr('z.bin', z.data); wr('yq.bin', yq.data);
console.log(JSON.stringify(hip.stats));
""", {"M": M, "K": K, "N": N})
    y = np.fromfile(tmp_path / "y.bin", np.float32).reshape(M, N)
    z = np.fromfile(tmp_path / "z.bin", np.float32).reshape(M, N)
    yq = np.fromfile(tmp_path / "yq.bin", np.float32).reshape(M, N)
    ref = x.astype(np.float64) @ W.astype(np.float64)
    assert rel_l2(z, ref) <= 1e-5
    assert rel_l2(y, ref + b) <= 1e-5
    refq = oracle.matmul_q8_ref(x, q, sc, N, b)
    assert rel_l2(yq, refq) <= 1e-3


def test_simd_module_init_and_streaming_weight_cycle(tmp_path):
    """js/hip-simd.js, the wasm-simd.js surface (wasm-simd.js:527-535), and
    the init contracts, driven as their callers drive them:
    * hip-q4 init() runs the wasm-q4.js:673-704 KAT on the GPU (wasm-q4.js
      647-668) and hip-simd init() the wasm-simd.js:365-385 one;
    * allocWeights + matmulCached (x W + bias) and matmul_general against
      numpy in double;
    * llama-streaming.js:367-392 per layer: resetWeights(), allocWeights of
      the embedding again, engine.cacheWeight of the layer's weights, LINEAR
      through tensorMulAdd -- the device memory held stays one layer's
      weights (resetWeights frees them), getStats reads as the reference's,
      and a pointer from before a reset is refused."""
    print("[case] js hip-simd surface, init KATs, streaming weight cycle", flush=True)
    K, N, M = 512, 384, 3
    rng = np.random.default_rng(7)
    ws = [rng.normal(0, 0.05, (K, N)).astype(np.float32) for _ in range(4)]
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    bias = rng.normal(0, 1, N).astype(np.float32)
    for i, w in enumerate(ws):
        w.tofile(tmp_path / f"w{i}.bin")
    x.tofile(tmp_path / "x.bin")
    bias.tofile(tmp_path / "b.bin")
    out = run_node(tmp_path, f"""
const simd = require({os.path.join(JS, 'hip-simd.js')!r});
const q = require({os.path.join(JS, 'hip-q4.js')!r});
const eng = require({os.path.join(JS, 'engine-hip.js')!r});
const K = meta.K, N = meta.N, M = meta.M;
const W = [0, 1, 2, 3].map(i => rd('w' + i + '.bin', Float32Array));
const x = rd('x.bin', Float32Array), b = rd('b.bin', Float32Array);
const okq = q.init(), kat = q.selfTest(), ok = simd.init();
const st0 = simd.getStats();
const p = simd.allocWeights(W[0]);
const c1 = new Float32Array(M * N); simd.matmulCached(x, M, K, p, N, b, c1); wr('cached.bin', c1);
const c2 = new Float32Array(M * N); simd.matmul_general(x, M, K, W[0], N, c2); wr('general.bin', c2);
const st1 = simd.getStats();
const hip = new eng.HipEngine();
hip.initWasm();
const emb = {{ name: 'token_embedding', shape: [K, N], data: W[0] }};
const res = [];
for (let l = 1; l <= 3; l++) {{
  simd.resetWeights();
  emb._wasmPtr = simd.allocWeights(emb.data);
  const t = {{ name: 'layer.w', shape: [K, N], data: W[l] }};
  hip.cacheWeight(t);
  const y = hip.tensorMulAdd({{ shape: [M, K], data: x }}, t, {{ data: b }}, 'y');
  wr('layer' + l + '.bin', y.data);
  res.push(parseFloat(simd.getStats().residentMB));
}}
let stale = false;
const old = emb._wasmPtr;
simd.resetWeights();
try {{ simd.matmulCached(x, M, K, old, N, null, c1); }} catch (e) {{ stale = /not a live/.test(e.message); }}
console.log(JSON.stringify({{ okq, kat, ok, st0, st1, res, stale, final: simd.getStats(), wasm: hip.wasmStats }}));
""", {"K": K, "N": N, "M": M})
    r = json.loads(out.strip().splitlines()[-1])
    assert r["okq"] and r["kat"] and r["ok"]
    assert r["st0"]["weightsMB"] == "0.0" and r["st0"]["scratchMB"] == "4.0"
    assert r["st1"]["weightsMB"] == f"{K * N * 4 / 2**20:.1f}"
    want = x.astype(np.float64) @ ws[0].astype(np.float64)
    got_c = np.fromfile(tmp_path / "cached.bin", np.float32).reshape(M, N)
    got_g = np.fromfile(tmp_path / "general.bin", np.float32).reshape(M, N)
    assert rel_l2(got_c.ravel(), (want + bias).ravel()) <= 1e-5
    assert rel_l2(got_g.ravel(), want.ravel()) <= 1e-5
    for l in (1, 2, 3):
        y = np.fromfile(tmp_path / f"layer{l}.bin", np.float32).reshape(M, N)
        ref = x.astype(np.float64) @ ws[l].astype(np.float64) + bias
        assert rel_l2(y.ravel(), ref.ravel()) <= 1e-5
    # each layer: the layer weight resident, the embedding's copy deferred
    assert max(r["res"]) <= K * N * 4 / 2**20 + 0.1, r["res"]
    assert r["stale"]
    assert r["final"]["residentMB"] == "0.0" and r["final"]["weightsMB"] == "0.0"
    assert r["wasm"]["supported"]


def test_llama_runtime_and_speculative_decoder(ctx, tmp_path):
    """HipLlamaRuntime loaded tensor by tensor under GGUF names: forward
    logits and greedy tokens match the same weights through the C ABI, and
    HipSpeculativeDecoder emits the greedy tokens."""
    print("[case] js llama-hip forward / generate / speculative", flush=True)
    cfg = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=1000,
               max_seq=128, weight_type=TYPE_Q4_0, embed_type=TYPE_Q4_0, rope_theta=10000.0)
    names = {0: "token_embd.weight", 2: "output_norm.weight", 3: "attn_norm.weight",
             4: "ffn_norm.weight", 5: "attn_q.weight", 6: "attn_k.weight", 7: "attn_v.weight",
             8: "attn_output.weight", 9: "ffn_gate.weight", 10: "ffn_up.weight",
             11: "ffn_down.weight"}
    files = []

    def keep(spec, data):
        tid, layer, N, K, t = spec
        nm = names[tid] if layer < 0 else f"blk.{layer}.{names[tid]}"
        fn = f"t{len(files)}.bin"
        np.ascontiguousarray(data).tofile(tmp_path / fn)
        files.append([nm, fn, "f32" if data.dtype == np.float32 else "u8"])

    model = synth.build(ctx, cfg, 600, keep)
    prompt = [int(t) for t in synth.random_tokens(601, 12, cfg["vocab_size"])]
    logits, nxt = model.forward(prompt, 0)
    greedy = [nxt] + [int(t) for t in model.generate(nxt, 12, 19)]
    model.reset_cache()
    draft = synth.build(ctx, cfg, 600)
    spec, _ = speculative_generate(model, draft, prompt, 20, 4, eos_ids=())
    assert list(spec[:20]) == greedy
    model.free()
    draft.free()
    out = run_node(tmp_path, f"""
const {{ HipLlamaRuntime, HipSpeculativeDecoder }} = require({os.path.join(JS, 'llama-hip.js')!r});
const c = meta.cfg;
const mk = () => {{
  const rt = new HipLlamaRuntime({{ dim: c.dim, hiddenDim: c.hidden_dim, nLayers: c.n_layers, nHeads: c.n_heads,
    nKvHeads: c.n_kv_heads, vocabSize: c.vocab_size, seqLen: c.max_seq, ropeTheta: c.rope_theta,
    weightType: 'q4_0', embedType: 'q4_0' }});
  for (const [nm, fn, ty] of meta.files) rt.loadTensor(nm, rd(fn, ty === 'f32' ? Float32Array : Uint8Array));
  return rt;
}};
const rt = mk();
const logits = rt.forward(meta.prompt, 0);
wr('logits.bin', logits);
const gen = rt.generate(meta.prompt, 20, {{ greedy: true, eosId: -1 }});
const genEos = rt.generate(meta.prompt, 20, {{ greedy: true, eosId: meta.eos }});
rt.rollbackCache(5);
const all = rt.forwardAll(meta.prompt.slice(5), 5);
wr('all.bin', all.logits);
const dr = mk();
const sd = new HipSpeculativeDecoder(rt, dr, {{ draftCount: 4 }});
const sp = sd.generate(meta.prompt, 20, {{ eosIds: [] }});
const sampled = rt.generate(meta.prompt, 4, {{ eosId: -1 }}).tokens.slice(meta.prompt.length);
console.log(JSON.stringify({{ gen: gen.tokens.slice(meta.prompt.length), genEos: genEos.tokens.slice(meta.prompt.length),
  genEosCount: genEos.generated, spec: sp.tokens.slice(meta.prompt.length),
  acc: sp.acceptanceRate, sampled, argmax: rt.argmax(logits) }}));
rt.free(); dr.free();
""", {"cfg": cfg, "files": files, "prompt": prompt, "eos": greedy[6]})
    res = json.loads(out.strip().splitlines()[-1])
    lj = np.fromfile(tmp_path / "logits.bin", np.float32)
    assert float(np.abs(lj - logits).max()) <= 2e-3
    assert res["argmax"] == int(np.argmax(lj))
    assert res["gen"] == greedy
    # llama.js:475-489: the loop stops at the first EOS, which is the last token
    stop = greedy.index(greedy[6]) + 1
    assert res["genEos"] == greedy[:stop] and res["genEosCount"] == stop
    assert res["spec"][:20] == greedy
    assert len(res["sampled"]) == 4 and all(0 <= t < cfg["vocab_size"] for t in res["sampled"])
    allj = np.fromfile(tmp_path / "all.bin", np.float32).reshape(-1, cfg["vocab_size"])
    assert allj.shape[0] == len(prompt) - 5
    assert float(np.abs(allj[-1] - logits).max()) <= 2e-3


def test_llama_runtime_from_gguf(ctx, tmp_path):
    """HipLlamaRuntime.fromGGUF: the build's GGUF reader from Node; the model
    equals the one the C ABI loads from the same file."""
    print("[case] js llama-hip fromGGUF", flush=True)
    from purebee_amd.native import Model, TYPE_Q6_K
    from tests.test_gpu_gguf import tiny, write_model
    cfg = tiny(TYPE_Q4_0, TYPE_Q6_K)
    path = tmp_path / "m.gguf"
    write_model(path, cfg, seed=21, n_tokens=1000)
    m = Model.from_gguf(ctx, path, max_seq=64)
    prompt = [int(t) for t in synth.random_tokens(22, 6, 1000)]
    logits, nxt = m.forward(prompt, 0)
    m.free()
    out = run_node(tmp_path, f"""
const {{ HipLlamaRuntime }} = require({os.path.join(JS, 'llama-hip.js')!r});
const rt = HipLlamaRuntime.fromGGUF(meta.path, {{ maxSeq: 64 }});
const logits = rt.forward(meta.prompt, 0);
wr('logits.bin', logits);
let threw = false;
try {{ HipLlamaRuntime.fromGGUF(meta.path + '.missing'); }} catch (e) {{ threw = /cannot open/.test(e.message); }}
console.log(JSON.stringify({{ cfg: rt.config, threw }}));
rt.free();
""", {"path": str(path), "prompt": prompt})
    res = json.loads(out.strip().splitlines()[-1])
    lj = np.fromfile(tmp_path / "logits.bin", np.float32)
    assert np.array_equal(lj, logits)
    c = res["cfg"]
    assert (c["dim"], c["hiddenDim"], c["nLayers"], c["nHeads"], c["nKvHeads"], c["vocabSize"]) == \
        (256, 512, 2, 4, 2, 1000)
    assert c["seqLen"] == 64 and c["embedType"] == TYPE_Q6_K and res["threw"]


def test_streaming_runtime_max_layers_sampling_self_spec(ctx, tmp_path):
    """HipStreamingLlamaRuntime through Node, as StreamingLlamaRuntime's callers
    use it (llama-streaming.js:738-970, speculative.js:58-204):
    * forward(tokens, pos, {maxLayers: 4}) -> {logits, layersUsed: 4}, logits
      within 2e-3 of the oracle's forward truncated to 4 layers (prefill and
      decode steps), and the full forward afterwards;
    * generate() with sampling: a seeded draw source gives the same tokens as
      forward + sample() step by step;
    * HipSelfSpeculativeDecoder (draft = the first 2 layers) in greedy mode
      emits the greedy tokens; with sampling it emits maxTokens tokens."""
    print("[case] js streaming runtime maxLayers / sampling / self-speculative", flush=True)
    from tests.e2e_util import make_pair
    cfg = dict(dim=256, hidden_dim=512, n_layers=6, n_heads=4, n_kv_heads=2, vocab_size=1000,
               max_seq=96, weight_type=TYPE_Q4_0, embed_type=TYPE_Q4_0, rope_theta=10000.0)
    names = {0: "token_embd.weight", 2: "output_norm.weight", 3: "attn_norm.weight",
             4: "ffn_norm.weight", 5: "attn_q.weight", 6: "attn_k.weight", 7: "attn_v.weight",
             8: "attn_output.weight", 9: "ffn_gate.weight", 10: "ffn_up.weight",
             11: "ffn_down.weight"}
    files = []

    def keep(spec, data):
        tid, layer, N, K, t = spec
        nm = names[tid] if layer < 0 else f"blk.{layer}.{names[tid]}"
        fn = f"t{len(files)}.bin"
        np.ascontiguousarray(data).tofile(tmp_path / fn)
        files.append([nm, fn, "f32" if data.dtype == np.float32 else "u8"])

    model = synth.build(ctx, cfg, 650, keep)
    model.free()
    _, ref, _ = make_pair(ctx, cfg, 650)
    prompt = [int(t) for t in synth.random_tokens(651, 12, cfg["vocab_size"])]
    steps = [(int(t), L) for t, L in zip(synth.random_tokens(652, 4, 1000), (4, 4, 0, 2))]
    want = [ref.forward(prompt, 0, max_layers=4)]
    for i, (t, L) in enumerate(steps):
        want.append(ref.forward([t], 12 + i, max_layers=L))
    ref.close()
    out = run_node(tmp_path, f"""
const {{ HipStreamingLlamaRuntime, HipSelfSpeculativeDecoder, sampleTopK }} =
  require({os.path.join(JS, 'llama-hip.js')!r});
const c = meta.cfg;
const seeded = (s) => () => {{ s = (s * 16807) % 2147483647; return (s - 1) / 2147483646; }};
const rt = new HipStreamingLlamaRuntime({{ dim: c.dim, hiddenDim: c.hidden_dim, nLayers: c.n_layers,
  nHeads: c.n_heads, nKvHeads: c.n_kv_heads, vocabSize: c.vocab_size, seqLen: c.max_seq,
  ropeTheta: c.rope_theta, weightType: 'q4_0', embedType: 'q4_0' }});
for (const [nm, fn, ty] of meta.files) rt.loadTensor(nm, rd(fn, ty === 'f32' ? Float32Array : Uint8Array));
const used = [];
let r = rt.forward(meta.prompt, 0, {{ maxLayers: 4 }});
used.push(r.layersUsed); wr('l0.bin', r.logits);
meta.steps.forEach(([t, L], i) => {{
  r = rt.forward([t], 12 + i, L ? {{ maxLayers: L }} : {{}});
  used.push(r.layersUsed); wr('l' + (i + 1) + '.bin', r.logits);
}});
// sampled generate vs forward + sample with the same draws
rt.random = seeded(7);
const gen = rt.generate(meta.prompt, 10, {{ temperature: 0.7, topK: 20, eosId: -1 }});
const rnd = seeded(7);
rt.resetCache();
let lg = rt.forward(meta.prompt, 0).logits, pos = meta.prompt.length;
const manual = [];
for (let i = 0; i < 10; i++) {{
  const t = sampleTopK(lg, 20, 0.7, rnd, false);
  manual.push(t);
  if (i < 9) lg = rt.forward([t], pos++).logits;
}}
const greedy = rt.generate(meta.prompt, 24, {{ greedy: true, eosId: -1 }});
const sd = new HipSelfSpeculativeDecoder(rt, {{ draftLayers: 2, draftCount: 4 }});
const sg = sd.generate(meta.prompt, 24, {{ greedy: true, eosIds: [] }});
const ss = sd.generate(meta.prompt, 16, {{ eosIds: [], temperature: 0.7 }});
console.log(JSON.stringify({{ used, gen: gen.tokens.slice(meta.prompt.length), manual,
  avgLayers: gen.avgLayers, greedy: greedy.tokens.slice(meta.prompt.length),
  sg: sg.tokens.slice(meta.prompt.length), ss: ss.tokens.slice(meta.prompt.length),
  stats: sd.stats }}));
rt.free();
""", {"cfg": cfg, "files": files, "prompt": prompt, "steps": steps})
    res = json.loads(out.strip().splitlines()[-1])
    print(f"  {res['stats']}")
    assert res["used"] == [4, 4, 4, 6, 2]
    worst = 0.0
    for i, w in enumerate(want):
        got = np.fromfile(tmp_path / f"l{i}.bin", np.float32)
        worst = max(worst, float(np.abs(got - w).max()))
    print(f"  maxLayers logits worst max-abs {worst:.2e}")
    assert worst <= 2e-3
    assert res["gen"] == res["manual"] and len(res["gen"]) == 10
    assert res["avgLayers"] == "6.0"
    assert res["sg"][:24] == res["greedy"]
    assert len(res["ss"]) in (16, 17) and all(0 <= t < 1000 for t in res["ss"])
