"""The host-side sampler of the JS runtimes (js/llama-hip.js sampleTopK)
against a full-sort restatement of the reference's top-k / temperature
sampling (llama.js:394-423: scaled logits in a Float32Array;
llama-streaming.js:868-896: in doubles): identical token for every draw,
on vectors with many tied values, for both scalings.  CPU only (the module
loads the GPU addon only when a runtime is constructed)."""
import json
import os
import shutil
import subprocess

import pytest

pytestmark = pytest.mark.skipif(shutil.which("node") is None, reason="node not installed")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "purebee_amd", "js", "llama-hip.js")

SCRIPT = """
const { sampleTopK } = require(%r);
// restatement: scale, stable sort of every (value, index) pair by value
// descending, softmax over the first topK, first cumulative sum >= r
function fullSort(logits, topK, temp, r, f32) {
  const pairs = [];
  for (let i = 0; i < logits.length; i++) {
    const v = logits[i] / temp;
    pairs.push({ v: f32 ? Math.fround(v) : v, i });
  }
  pairs.sort((a, b) => (b.v - a.v) || (a.i - b.i));
  const top = pairs.slice(0, topK);
  const ex = top.map((p) => Math.exp(p.v - top[0].v));
  const sum = ex.reduce((a, b) => a + b, 0);
  let c = 0;
  for (let i = 0; i < top.length; i++) { c += ex[i] / sum; if (r <= c) return top[i].i; }
  return top[0].i;
}
let s = 12345;
const rnd = () => { s = (s * 16807) %% 2147483647; return (s - 1) / 2147483646; };
let bad = 0, n = 0;
for (let trial = 0; trial < 400; trial++) {
  const len = 1 + Math.floor(rnd() * 4000);
  const L = new Float32Array(len);
  const spread = trial %% 2 ? 16 : 4096;   // few distinct values -> many ties
  for (let i = 0; i < len; i++) L[i] = (Math.floor(rnd() * spread) - spread / 2) / 64;
  const k = 1 + Math.floor(rnd() * 80);
  const T = 0.05 + 1.5 * rnd();
  for (const f32 of [true, false]) {
    for (const r of [rnd(), 0, 1, 0.5]) {
      n++;
      if (sampleTopK(L, k, T, () => r, f32) !== fullSort(L, k, T, r, f32)) bad++;
    }
  }
}
console.log(JSON.stringify({ bad, n }));
"""


def test_sample_top_k_matches_full_sort(tmp_path):
    p = tmp_path / "s.js"
    p.write_text(SCRIPT % JS)
    r = subprocess.run(["node", str(p)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["n"] == 3200 and res["bad"] == 0, res
