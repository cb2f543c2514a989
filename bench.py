#!/usr/bin/env python3
"""Benchmark: Llama-3.2-1B-shaped Q4_0 decode at batch 1 on one MI355X.

Default workload ("decode"): a Llama-3.2-1B-shaped model (dim 2048, 16
layers, 32/8 heads, head_dim 64, FFN 8192 SwiGLU, vocab 128256, tied Q4_0
embedding, RoPE theta 5e5) with seeded N(0, 0.02) weights quantised to Q4_0,
resident in HBM.  A 128-token random prompt is run, then one timed step is one
greedy decode token (every layer's matvecs, attention over the KV cache,
LM head, argmax) replayed on the GPU from a captured graph; the default 256
steps take the KV cache from 128 to 384 positions.

Workload "matvec": the per-token quantized-matvec pass alone (16 layers x
q/k/v/o/gate/up/down + LM head) through the plain instruction.

Workload "m-gt-1": only the M>1 measurements of the default line (batched
512-token prefill, the MFMA GEMM at M=512, M=5 verify, speculative decoding).

Workload "small": only the stories15M-shaped (16-token prompt + 128 steps)
and SmolLM2-135M-shaped (32 + 256) Q8_0 decode legs of the default line.

Prints one JSON line: the bench contract plus `roofline` (the kernel with the
largest share of a step: its algorithmic bytes over its mean execution time
inside decode steps, from HIP events that the kernel's own dispatch stamps),
`kernels` (per role), `seam` (the synchronous host-buffer instruction as
llama-streaming.js calls it) and `cpu_baseline` (the restated reference CPU
path on a bounded sample of the same work, timed on this host's cores).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor figure
METRIC = "Llama-3.2-1B Q4 decode tok/s @1 GPU; Q4 matvec HBM GB/s vs peak"
PROMPT = 128


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4_bytes(N, K):
    return N * K // 32 * 18


def host_threads():
    """Threads for the CPU baseline: the CPUs this process may run on, at most
    16 (one GPU's share of the host CPUs of an 8-GPU node)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(host, cfg, seconds):
    """Restated reference CPU path on the same weights: wasm-q4.js Q4_0 kernel
    in SSE under the thread-pool.js row split for the 7 matvecs of each layer,
    and the single-threaded f32 LM head (wasmQ4.lmHead) over the exactly
    dequantised tied embedding.  Attention and norms (<1% of the reference's
    per-token time) are left out of the sample.  Timed with the host's
    threads (value) and with one thread (t1_value)."""
    import oracle
    from purebee_amd import native as N_
    threads = host_threads()
    d, h, L, V = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    emb = oracle.dequant_q4_0(host[(N_.T_TOKEN_EMBD, -1)], V * d)
    x = {d: np.random.default_rng(1).normal(0, 1, d).astype(np.float32),
         h: np.random.default_rng(2).normal(0, 1, h).astype(np.float32)}
    mats = [(N_.T_ATTN_Q, d, d), (N_.T_ATTN_K, -1, d), (N_.T_ATTN_V, -1, d),
            (N_.T_ATTN_OUTPUT, d, d), (N_.T_FFN_GATE, h, d), (N_.T_FFN_UP, h, d),
            (N_.T_FFN_DOWN, d, h)]
    kv = cfg["n_kv_heads"] * (d // cfg["n_heads"])

    def timed(pool, budget, cap):
        def one_token():
            for l in range(L):
                for tid, n, k in mats:
                    n = kv if n < 0 else n
                    pool.q4_0_matvec(x[k], host[(tid, l)], n, k)
            oracle.cpu_lm_head(x[d], emb, V, d)

        one_token()
        t0 = time.perf_counter()
        one_token()
        per = time.perf_counter() - t0
        n = max(2, min(cap, int(budget / max(per, 1e-3))))
        t0 = time.perf_counter()
        for _ in range(n):
            one_token()
        return n, time.perf_counter() - t0

    pool = oracle.CpuPool(threads)
    n, dt = timed(pool, seconds, 60)
    pool.close()
    pool1 = oracle.CpuPool(1)
    n1, dt1 = timed(pool1, seconds * 0.75, 20)
    pool1.close()
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "host_cpus": os.cpu_count(), "t1_value": round(n1 / dt1, 3),
            "sample": f"{n} decode tokens of Q4_0 matvec work (16 layers x 7 matvecs, "
                      f"{threads} threads) + single-threaded f32 LM head, {dt:.1f}s; "
                      f"t1_value: {n1} tokens on 1 thread, {dt1:.1f}s"}


def cpu_matvec_shapes(host_threads_n):
    """The restated reference CPU kernel (wasm-q4.js:118-267 in SSE, the
    thread-pool.js:174-227 row split, the per-call copy) on each Llama-1B
    Q4_0 matvec shape: median of 10 calls after 3 warm-ups, GB/s of the
    algorithmic bytes (weights + x + y)."""
    import oracle
    pool = oracle.CpuPool(host_threads_n)
    res = {}
    for name, N, K in (("q_o", 2048, 2048), ("k_v", 512, 2048), ("gate_up", 8192, 2048),
                       ("down", 2048, 8192), ("lm_head", 128256, 2048)):
        raw = oracle.quantize_q4_0(oracle.synth_normal(70 + N + K, N * K, 0.0, 0.02).reshape(N, K))
        x = np.random.default_rng(K).normal(0, 1, K).astype(np.float32)
        out = np.empty(N, np.float32)
        ts = []
        for i in range(13):
            t0 = time.perf_counter()
            pool.q4_0_matvec(x, raw, N, K, out)
            ts.append(time.perf_counter() - t0)
        t = sorted(ts[3:])[5]
        by = q4_bytes(N, K) + 4 * (N + K)
        res[name] = {"N": N, "K": K, "us": round(t * 1e6, 1), "GBps": round(by / t / 1e9, 3)}
    pool.close()
    log("cpu matvec shapes (" + str(host_threads_n) + " threads): " +
        ", ".join(f"{k} {v['GBps']:.2f} GB/s" for k, v in res.items()))
    return {"threads": host_threads_n, "kind": "port", "shapes": res}


def cpu_stories_decode(seconds):
    """Config 1's path in the reference, restated: per token, 6 layers x 7
    matmul_q8 calls (quantize.js:224-266 on QuantizedTensor [K,N], as LINEAR
    -> tensorMulAddQ8 runs them, engine.js:259-269) and the f32 LM head over
    the 32000 x 288 embedding (llama.js:353-367), on one thread as the
    reference's main JS thread runs them.  Attention and norms (a small
    share of its time) are left out of the sample."""
    import oracle
    d, h, L, V = 288, 768, 6, 32000
    rng = np.random.default_rng(5)
    mats = []
    for K, N in ((d, d), (d, d), (d, d), (d, d), (d, h), (d, h), (h, d)):
        q, sc = oracle.quantize_q8_ref(rng.normal(0, 0.02, (K, N)).astype(np.float32))
        mats.append((K, N, q, sc))
    emb = rng.normal(0, 0.02, V * d).astype(np.float32)
    xs = {K: rng.normal(0, 1, (1, K)).astype(np.float32) for K in (d, h)}

    def one_token():
        for _ in range(L):
            for K, N, q, sc in mats:
                oracle.matmul_q8_ref(xs[K], q, sc, N)
        oracle.cpu_lm_head(xs[d][0], emb, V, d)

    one_token()
    t0 = time.perf_counter()
    one_token()
    per = time.perf_counter() - t0
    n = max(3, min(2000, int(seconds / max(per, 1e-4))))
    t0 = time.perf_counter()
    for _ in range(n):
        one_token()
    dt = time.perf_counter() - t0
    log(f"cpu stories15M q8 decode (restated llama.js path, 1 thread): {n / dt:.1f} tok/s")
    return {"value": round(n / dt, 2), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"{n} decode tokens: 6 layers x 7 matmul_q8 (M=1) + f32 LM head 32000x288, "
                      f"{dt:.1f}s"}


def run_small_decode(pb, synth, name, n_prompt, n_gen):
    """Configs 1 and 3: greedy decode of n_gen tokens after a random
    n_prompt-token prompt, timed over the whole generate call (HIP events on
    the model's stream), plus the per-kernel times of 16 steps launched
    kernel by kernel and the roofline of the step's largest kernel."""
    cfg = synth.CONFIGS[name]
    ctx = pb.Context(0)
    model = synth.build(ctx, cfg, seed=1000)
    prompt = synth.random_tokens(7, n_prompt, cfg["vocab_size"])
    model.forward(prompt, 0, want_logits=False)
    model.reset_cache()
    t0 = time.perf_counter()
    _, nxt = model.forward(prompt, 0, want_logits=False)
    prefill_s = time.perf_counter() - t0
    model.generate(nxt, n_prompt, 16)
    model.rollback(n_prompt)
    ctx.sync()
    ctx.timer_start()
    model.generate(nxt, n_prompt, n_gen)
    ms = ctx.timer_stop() / n_gen
    model.rollback(n_prompt)
    prof = model.profile(nxt, n_prompt, 16)
    roles = {}
    for role, kern, us, by in prof:
        r = roles.setdefault(role, {"kernel": kern, "launches_per_step": 0, "us_per_step": 0.0,
                                    "bytes_per_step": 0.0})
        r["launches_per_step"] += 1
        r["us_per_step"] += us
        r["bytes_per_step"] += by
    for r in roles.values():
        r["us_per_launch_in_step"] = round(r["us_per_step"] / r["launches_per_step"], 3)
        r["GBps"] = round(r["bytes_per_step"] / r["us_per_step"] / 1e3, 1) if r["us_per_step"] else 0.0
        r["us_per_step"] = round(r["us_per_step"], 2)
        r["bytes_per_step"] = round(r["bytes_per_step"])
    dom_name, dom = max(roles.items(), key=lambda kv: kv[1]["us_per_step"])
    gbps = dom["bytes_per_step"] / dom["us_per_step"] / 1e3
    step_bytes = sum(r["bytes_per_step"] for r in roles.values())
    log(f"{name}: decode {n_gen} steps (KV {n_prompt}->{n_prompt + n_gen}) {ms * 1e3:.1f} us/token, "
        f"{1e3 / ms:.1f} tok/s; largest kernel {dom_name} ({dom['kernel']}) "
        f"{dom['us_per_launch_in_step']:.2f} us a launch, {gbps:.0f} GB/s")
    out = {"workload": f"{name}-shaped {'q8_0'} greedy decode, batch 1, {n_prompt}-token prompt "
                       f"then {n_gen} steps",
           "tok_per_s": round(1e3 / ms, 2), "ms_per_token": round(ms, 5),
           "prefill_ms": round(prefill_s * 1e3, 3), "bytes_per_step": step_bytes,
           "effective_GBps": round(step_bytes / ms / 1e6, 1),
           "roofline": {"bound": "hbm", "kernel": f"{dom['kernel']} ({dom_name})",
                        "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbps / HBM_PEAK_GBS, 4),
                        "us_per_launch": dom["us_per_launch_in_step"]},
           "kernels": roles}
    model.free()
    ctx.close()
    return out


COPY_BYTES = 256 << 20


def measure_copy(ctx, reps=8):
    """Achievable HBM bandwidth of a plain copy kernel (pbx_dev_copy) over
    buffers larger than the 256 MB MALL; counted as read + write bytes.  The
    same launches calibrate the FETCH_SIZE / WRITE_SIZE counters."""
    a, b = ctx.alloc(COPY_BYTES), ctx.alloc(COPY_BYTES)
    ctx.dev_copy(b.ptr, a.ptr, COPY_BYTES)
    ctx.sync()
    ctx.timer_start()
    for i in range(reps):
        src, dst = (a, b) if i % 2 == 0 else (b, a)
        ctx.dev_copy(dst.ptr, src.ptr, COPY_BYTES)
    ms = ctx.timer_stop()
    a.free()
    b.free()
    return {"bytes": COPY_BYTES, "GBps": 2 * COPY_BYTES * reps / ms / 1e6}


def load_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary
    (profiles/traffic_decode.json, written by --summarize-pmc), or None."""
    path = os.path.join(ROOT, "profiles", "traffic_decode.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    k = t.get("kernels", {}).get(kernel)
    return None if k is None else k.get("hbm_bytes_per_launch")


def summarize_pmc(fetch_csv, write_csv, out_path):
    """Mean FETCH_SIZE / WRITE_SIZE per dispatch and kernel from two
    rocprofv3 --pmc counter_collection CSVs, scaled by the factor that makes
    the plain copy kernel read and write exactly its known bytes."""
    import csv

    def per_kernel(path, counter):
        acc = {}
        with open(path) as f:
            for r in csv.DictReader(f):
                if r.get("Counter_Name") != counter:
                    continue
                name = r["Kernel_Name"].split("(")[0].strip()
                key = (name, r.get("Dispatch_Id"))
                acc[key] = acc.get(key, 0.0) + float(r["Counter_Value"])
        out = {}
        for (name, _), v in acc.items():
            s = out.setdefault(name, [0.0, 0])
            s[0] += v
            s[1] += 1
        return {k: v[0] / v[1] for k, v in out.items()}

    fetch = per_kernel(fetch_csv, "FETCH_SIZE")
    write = per_kernel(write_csv, "WRITE_SIZE")
    copy_kib = COPY_BYTES / 1024.0
    f_scale = copy_kib / fetch["pbx_copy16"] if fetch.get("pbx_copy16") else None
    w_scale = copy_kib / write["pbx_copy16"] if write.get("pbx_copy16") else None
    kernels = {}
    for k in sorted(set(fetch) | set(write)):
        fk, wk = fetch.get(k), write.get(k)
        entry = {"fetch_kib_raw": fk, "write_kib_raw": wk}
        if fk is not None and wk is not None and f_scale and w_scale:
            entry["hbm_bytes_per_launch"] = round((fk * f_scale + wk * w_scale) * 1024)
        kernels[k] = entry
    res = {"copy_kernel_bytes_each_way": COPY_BYTES, "fetch_scale": f_scale,
           "write_scale": w_scale, "kernels": kernels}
    with open(out_path, "w") as f:
        json.dump(res, f, indent=1)
    return res


def run_decode(args, pb, synth):
    cfg = synth.CONFIGS["llama32_1b"]
    ctx = pb.Context(0)
    dev, cus = ctx.device_info()
    log(f"device {dev}, {cus} CUs")
    host = {}
    t0 = time.time()

    def keep(spec, data):
        tid, layer, N, K, t = spec
        if t == pb.TYPE_Q4_0:
            host[(tid, layer)] = data

    model = synth.build(ctx, cfg, seed=1000, keep=keep)
    info = model.info()
    log(f"model built + uploaded in {time.time() - t0:.1f}s, {info['device_bytes'] / 1e9:.2f} GB resident")

    copy = measure_copy(ctx)
    log(f"plain copy kernel: {copy['GBps']:.0f} GB/s ({copy['bytes'] / 2**20:.0f} MiB read + written)")

    prompt = synth.random_tokens(7, PROMPT, cfg["vocab_size"])
    # the first forward also pays one-time costs (batch buffers, first launches);
    # time the second one over the same prompt
    model.forward(prompt, 0, want_logits=False)
    model.reset_cache()
    ctx.sync()
    t0 = time.perf_counter()
    _, nxt = model.forward(prompt, 0, want_logits=False)
    prefill_s = time.perf_counter() - t0
    log(f"prefill {PROMPT} tokens (one batched forward, warm): {prefill_s * 1e3:.1f} ms")

    def time_decode(steps):
        model.rollback(PROMPT)
        ctx.sync()
        ctx.timer_start()
        t = model.generate(nxt, PROMPT, steps)
        return ctx.timer_stop() / steps, t

    model.generate(nxt, PROMPT, args.warmup)
    ms_per_step, toks = time_decode(args.steps)
    log(f"decode {args.steps} steps: {ms_per_step * 1e3:.1f} us/token, {1e3 / ms_per_step:.1f} tok/s "
        f"(graph={model.info()['graph']})")
    # the workload's full length (KV 128 -> 384), reported beside the timed steps
    ms256 = ms_per_step if args.steps == 256 else time_decode(256)[0]
    log(f"decode 256 steps (KV {PROMPT}->{PROMPT + 256}): {ms256 * 1e3:.1f} us/token, "
        f"{1e3 / ms256:.1f} tok/s")
    model.rollback(PROMPT)

    # per-kernel execution times inside decode steps: the same steps launched
    # kernel by kernel, each kernel's start / stop events stamped by its own
    # dispatch (the durations a kernel trace of these launches reports)
    n_prof = 16
    prof = model.profile(nxt, PROMPT, n_prof)
    model.rollback(PROMPT)
    roles = {}
    for role, kern, us, by in prof:
        r = roles.setdefault(role, {"kernel": kern, "launches_per_step": 0,
                                    "kernel_us_per_step": 0.0, "bytes_per_step": 0.0})
        r["launches_per_step"] += 1
        r["kernel_us_per_step"] += us
        r["bytes_per_step"] += by
    kernel_sum = sum(r["kernel_us_per_step"] for r in roles.values())
    for role, r in roles.items():
        n = r["launches_per_step"]
        r["us_per_launch_in_step"] = r["kernel_us_per_step"] / n
        r["bytes_per_launch"] = r["bytes_per_step"] / n
        r["GBps"] = r["bytes_per_step"] / r["kernel_us_per_step"] / 1e3 if r["kernel_us_per_step"] else 0.0
        # the graph-replayed step's time split over the roles in proportion
        # to their execution times (the shares add up to ms_per_step)
        r["share_of_step_us"] = ms_per_step * 1e3 * r["kernel_us_per_step"] / kernel_sum
        log(f"{role:8s} {r['kernel']:24s} x{n:3d}: {r['us_per_launch_in_step']:7.2f} us/launch in step, "
            f"{r['GBps']:7.0f} GB/s, {r['kernel_us_per_step']:7.1f} us/step")
    log(f"kernel execution sum {kernel_sum:.1f} us per step (kernel by kernel); "
        f"graph step {ms_per_step * 1e3:.1f} us")
    # the roofline kernel: the role with the largest share of a step, whatever
    # it computes
    dom_name, dom = max(roles.items(), key=lambda kv: kv[1]["kernel_us_per_step"])
    us_in = dom["us_per_launch_in_step"]
    gbps = dom["bytes_per_launch"] / us_in / 1e3
    roofline = {"bound": "hbm", "kernel": f"{dom['kernel']} ({dom_name})",
                "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbps / HBM_PEAK_GBS, 4),
                "traffic": load_traffic(dom["kernel"]),
                "bytes_per_launch": round(dom["bytes_per_launch"]),
                "us_per_launch": round(us_in, 3),
                "timing": f"mean execution of the {dom['launches_per_step']} launches in each of "
                          f"{n_prof} decode steps at KV {PROMPT + 1}..{PROMPT + n_prof} "
                          "(kernel by kernel; dispatch-stamped HIP events)"}
    if dom_name in ("attn", "attn_o", "qkv_attn_o"):
        # bytes of a launch with attention: the matvec weights and activations
        # plus K and V of every cached position (8 * kv_dim bytes each); the
        # matvec-only figure leaves the cache out
        kv = cfg["n_kv_heads"] * (cfg["dim"] // cfg["n_heads"])
        kv_bytes = 8 * kv * (PROMPT + (n_prof + 1) / 2)
        mv = dom["bytes_per_launch"] - kv_bytes
        roofline.update({"bytes_kv_per_launch": round(kv_bytes),
                         "bytes_matvec_only": round(mv),
                         "achieved_matvec_only": round(mv / us_in / 1e3, 1),
                         "frac_matvec_only": round(mv / us_in / 1e3 / HBM_PEAK_GBS, 4)})
        log(f"dominant {dom_name} ({dom['kernel']}): {us_in:.2f} us in step, {gbps:.0f} GB/s "
            f"with KV, {mv / us_in / 1e3:.0f} GB/s matvec bytes only")
    # the largest GEMV also timed back to back over all layers' weights (the
    # gate/up set, 302 MB, exceeds the 256 MB MALL)
    gemv_roles = {k: v for k, v in roles.items() if k in ("qkv", "o", "gate_up", "down", "lm_head")}
    if gemv_roles:
        g_name, g = max(gemv_roles.items(), key=lambda kv: kv[1]["kernel_us_per_step"])
        us_b2b, by, nl = model.bench_role(g_name, max(2, 640 // g["launches_per_step"]))
        model.rollback(PROMPT)
        log(f"largest GEMV {g_name} ({g['kernel']}): {g['us_per_launch_in_step']:.2f} us in step; "
            f"back to back {us_b2b:.2f} us, {by / us_b2b / 1e3:.0f} GB/s")
        roofline["largest_gemv"] = {
            "kernel": f"{g['kernel']} ({g_name})", "us_per_launch": round(g["us_per_launch_in_step"], 3),
            "bytes_per_launch": round(g["bytes_per_launch"]),
            "frac": round(g["bytes_per_launch"] / g["us_per_launch_in_step"] / 1e3 / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(g["kernel"]),
            "us_back_to_back": round(us_b2b, 3),
            "frac_back_to_back": round(by / us_b2b / 1e3 / HBM_PEAK_GBS, 4)}
    step_bytes = sum(r["bytes_per_step"] for r in roles.values())
    seam = run_seam(ctx, pb, cfg, host) if host else None
    matvec_shapes = None if args.no_matvec_shapes else run_matvec_shapes(ctx, pb)
    m_gt_1 = None if args.no_m_gt_1 else run_m_gt_1(ctx, model, cfg, pb, synth)
    next_rows = None
    if not args.no_m_gt_1:
        next_rows = {"q4_1_matvec": run_q4_1(ctx, pb), "gemm_types": run_gemm_types(ctx, pb),
                     "gguf": run_gguf(ctx, pb, synth)}
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the restated reference CPU path ...")
        cpu = cpu_baseline(host, cfg, args.cpu_seconds)
        log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} threads")
        cpu["matvec_shapes"] = cpu_matvec_shapes(cpu["cores"])
    small = None
    if not args.no_small_configs:
        small = {"stories15m": run_small_decode(pb, synth, "stories15m", 16, 128),
                 "smollm2_135m": run_small_decode(pb, synth, "smollm2_135m", 32, 256)}
        if not args.no_cpu_baseline:
            small["stories15m"]["cpu_baseline"] = cpu_stories_decode(args.cpu_seconds * 0.5)
    out = {
        "metric": METRIC,
        "value": round(1e3 / ms_per_step, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights (int4 codes, fp16 block scales); each 32-element block of a "
                 "GEMV's input rounded to 22-bit fixed point on a power-of-two block scale "
                 "(three int8 limbs, exact int32 dots); fp32 block combine, accumulation, "
                 "norms, attention and KV cache",
        "data": "synthetic: seeded N(0,0.02) weights quantised to Q4_0, random prompt tokens",
        "config": {"workload": "llama-3.2-1b-shaped q4_0 greedy decode, batch 1, "
                               f"{PROMPT}-token prompt then {args.steps} steps "
                               f"(KV {PROMPT}->{PROMPT + args.steps})",
                   "model": "llama-3.2-1b-shaped (random init)",
                   "global_batch": 1, "seq_len": PROMPT + args.steps,
                   "bytes_per_step": round(step_bytes),
                   "effective_GBps": round(step_bytes / ms_per_step / 1e6, 1),
                   "prefill_ms": round(prefill_s * 1e3, 2), "device": dev,
                   "copy_kernel_GBps": round(copy["GBps"], 1),
                   "decode_256": {"kv": f"{PROMPT}->{PROMPT + 256}",
                                  "us_per_token": round(ms256 * 1e3, 2),
                                  "tok_per_s": round(1e3 / ms256, 2)},
                   "kernel_us_per_step": round(kernel_sum, 2),
                   "first_tokens": [int(t) for t in toks[:8]]},
        "roofline": roofline,
        "kernels": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in roles.items()},
        "seam": seam,
        "matvec_shapes": matvec_shapes,
        "m_gt_1": m_gt_1,
        "next_rows": next_rows,
        "small_configs": small,
        "cpu_baseline": cpu,
    }
    model.free()
    ctx.close()
    return out


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA, vendor figure


def run_seam(ctx, pb, cfg, host, tokens=8):
    """The synchronous instruction seam StreamingLlamaRuntime goes through
    (quantizedMatvec, llama-streaming.js:168-177, called 7 times a layer by
    _runLayerQ4, llama-streaming.js:505-606) plus the LM head: one pbx_linear
    call per matvec with host activations in and host outputs back, 113 calls
    a token for Llama-3.2-1B, on the same Q4_0 weights uploaded as separate
    matrices.  Reports the matvec time a token spends in that seam."""
    from purebee_amd import native as N_
    d, h, L, V = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = cfg["n_kv_heads"] * (d // cfg["n_heads"])
    shapes = [(N_.T_ATTN_Q, d, d), (N_.T_ATTN_K, kv, d), (N_.T_ATTN_V, kv, d),
              (N_.T_ATTN_OUTPUT, d, d), (N_.T_FFN_GATE, h, d), (N_.T_FFN_UP, h, d),
              (N_.T_FFN_DOWN, d, h)]
    ws = [(ctx.upload(pb.TYPE_Q4_0, n, k, host[(tid, l)]), k) for l in range(L) for tid, n, k in shapes]
    ws.append((ctx.upload(pb.TYPE_Q4_0, V, d, host[(N_.T_TOKEN_EMBD, -1)]), d))
    xs = {k: np.random.default_rng(k).normal(0, 1, k).astype(np.float32) for k in (d, h)}

    def one_token():
        for w, k in ws:
            ctx.linear(w, xs[k])

    one_token()
    t0 = time.perf_counter()
    for _ in range(tokens):
        one_token()
    dt = (time.perf_counter() - t0) / tokens
    for w, _ in ws:
        w.free()
    calls = len(ws)
    log(f"seam: {calls} host-buffer pbx_linear calls a token, {dt * 1e3:.2f} ms/token "
        f"({dt / calls * 1e6:.1f} us a call), {1 / dt:.1f} tok/s of matvec work")
    return {"calls_per_token": calls, "ms_per_token": round(dt * 1e3, 3),
            "us_per_call": round(dt / calls * 1e6, 2), "tok_per_s": round(1 / dt, 2),
            "note": "matvecs only (q, k, v, o, gate, up, down per layer + LM head), host buffers, "
                    "synchronous; attention and norms are not in this leg"}


def run_m_gt_1(ctx, model, cfg, pb, synth):
    """The M>1 path on the same model: a 512-token batched prefill, the MFMA
    GEMM alone at the prefill shape, and speculative decoding with M=5
    verifies (4 drafts from a stories15M-shaped Q8_0 model + 1)."""
    d, h, V = cfg["dim"], cfg["hidden_dim"], cfg["vocab_size"]
    res = {}
    prompt = synth.random_tokens(11, 512, V)
    times = []
    for _ in range(3):
        model.reset_cache()
        ctx.sync()
        t0 = time.perf_counter()
        model.forward(prompt, 0, want_logits=False)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[1]
    # useful FLOPs of a prefill: 2 * params per token for the layer matrices,
    # the LM head on the last row only, attention 4 * hd per (query, key) pair
    L, kvd = cfg["n_layers"], cfg["n_kv_heads"] * (d // cfg["n_heads"])
    layer_params = L * (d * (d + 2 * kvd) + d * d + 2 * h * d + d * h)
    flops = 2.0 * 512 * layer_params + 2.0 * V * d + L * cfg["n_heads"] * 4 * (d // cfg["n_heads"]) * 512 * 513 / 2
    res["prefill"] = {"tokens": 512, "ms": round(t * 1e3, 3), "tok_per_s": round(512 / t, 1),
                      "useful_TFLOPs": round(flops / t / 1e12, 2)}
    log(f"prefill 512 tokens (batched, MFMA): {t * 1e3:.2f} ms, {512 / t:.0f} tok/s, "
        f"{flops / t / 1e12:.1f} TFLOP/s useful")
    # the GEMM alone: gate|up (16384 x 2048, Q4_0) at M = 512, prep + MFMA
    N, K, M = 2 * h, d, 512
    raw = pb.quantize_q4_0(pb.synth_normal(77, N * K, 0, 0.02).reshape(N, K))
    w = ctx.upload(pb.TYPE_Q4_0, N, K, raw)
    dx = ctx.alloc(M * K * 4).upload(np.random.default_rng(5).normal(0, 1, M * K).astype(np.float32))
    dy = ctx.alloc(M * N * 4)
    ctx.bench_linear([w], [dx.ptr], [dy.ptr], M, 3)
    reps = 20
    ms = ctx.bench_linear([w], [dx.ptr], [dy.ptr], M, reps) / reps
    tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    res["gemm"] = {"shape": f"M={M} N={N} K={K} q4_0 (gate|up)", "kernel": "pbx_gemm_q4_big",
                   "us_per_launch": round(ms * 1e3, 2), "achieved": round(tf, 2),
                   "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                   "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                   "note": "useful 2*M*N*K; the kernel issues two fp16 MFMAs (activation hi + lo) "
                           "per useful product"}
    log(f"gemm {res['gemm']['shape']}: {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s useful "
        f"({100 * tf / MFMA_F16_PEAK_TFLOPS:.1f}% of {MFMA_F16_PEAK_TFLOPS:.0f})")
    w.free(), dx.free(), dy.free()
    # verify: M = 5 forward after a 128-token prompt, then speculative decoding
    draft = synth.build(ctx, "stories15m", seed=2000)
    vp = synth.random_tokens(12, PROMPT, V)
    model.reset_cache()
    model.forward(vp, 0, want_logits=False)
    rows = synth.random_tokens(13, 5, V)
    model.forward_batch(rows, PROMPT, want_logits=False)
    ctx.sync()
    n_ver = 64
    t0 = time.perf_counter()
    for i in range(n_ver):
        model.forward_batch(rows, PROMPT, want_logits=False)
    tv = (time.perf_counter() - t0) / n_ver
    wbytes = model.info()["device_bytes"]  # resident weights + caches: an upper bound
    step_bytes = sum(q4_bytes(*s[2:4]) for s in synth.tensor_specs(cfg) if s[4] == pb.TYPE_Q4_0)
    res["verify"] = {"M": 5, "ms": round(tv * 1e3, 3),
                     "weight_GBps": round(step_bytes / tv / 1e9, 1),
                     "frac_hbm": round(step_bytes / tv / 1e9 / HBM_PEAK_GBS, 4),
                     "weight_bytes": step_bytes, "resident_bytes": wbytes}
    log(f"verify M=5: {tv * 1e3:.3f} ms per forward, {step_bytes / tv / 1e9:.0f} GB/s of weights")
    out, st = pb.speculative_generate(model, draft, vp, 64, 4, eos_ids=())
    res["speculative"] = {"draft": "stories15m-shaped q8_0 (vocab 32000)", "draft_count": 4,
                          "tokens": int(len(out)), "rounds": st["rounds"],
                          "accepted": st["accepted"], "drafted": st["drafted"],
                          "decode_ms": round(st["decode_ms"], 2),
                          "tok_per_s": round((len(out) - 1) / (st["decode_ms"] / 1e3), 1)}
    log(f"speculative: {len(out)} tokens in {st['rounds']} rounds, accepted {st['accepted']}/"
        f"{st['drafted']}, {res['speculative']['tok_per_s']} tok/s")
    draft.free()
    model.reset_cache()
    return res


def run_q4_1(ctx, pb):
    """The Q4_1 matvec (quantizedMatvec type 3) through the plain
    instruction at the Llama-3.2-1B FFN shapes, beside Q4_0 on the same
    shapes.  Each timed pass rotates through 32 distinct weights (over 300 MB,
    more than the last-level cache), so every launch streams its weight from
    HBM.  Algorithmic bytes per launch: the GGUF blocks (20 B per 32 weights
    for Q4_1, 18 B for Q4_0) plus the fp32 activation and output vectors."""
    res = {}
    rng = np.random.default_rng(41)
    for name, N, K in (("ffn_gate", 8192, 2048), ("ffn_down", 2048, 8192)):
        base = pb.synth_normal(4100 + N, N * K, 0, 0.02).reshape(N, K)
        dx = ctx.alloc(K * 4).upload(rng.normal(0, 1, K).astype(np.float32))
        dy = ctx.alloc(N * 4)
        for t, qname, bpb, quant in ((pb.TYPE_Q4_1, "q4_1", 20, pb.quantize_q4_1),
                                     (pb.TYPE_Q4_0, "q4_0", 18, pb.quantize_q4_0)):
            ws = []
            for i in range(32):
                # distinct weights: roll the columns of one quantised base
                ws.append(ctx.upload(t, N, K, quant(np.roll(base, 32 * i, axis=1))))
            ctx.bench_linear(ws, [dx.ptr] * 32, [dy.ptr] * 32, 1, 2)
            reps = 10
            us = ctx.bench_linear(ws, [dx.ptr] * 32, [dy.ptr] * 32, 1, reps) / reps / 32 * 1e3
            b = N * K // 32 * bpb + 4 * (N + K)
            res[f"{name}_{qname}"] = {"N": N, "K": K, "us_per_launch": round(us, 2),
                                      "achieved_GBps": round(b / us / 1e3, 1),
                                      "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                                      "algorithmic_bytes": b}
            log(f"{qname} matvec {name} {N}x{K}: {us:.2f} us, {b / us / 1e3:.0f} GB/s")
            for w in ws:
                w.free()
        dx.free(), dy.free()
    return res


def run_matvec_shapes(ctx, pb):
    """The plain instruction (q4_0_matvec / quantizedMatvec, M = 1) on each
    Llama-3.2-1B matvec shape with Q4_0 weights: N(0, 0.02) quantised, x from
    N(0, 1).  Each shape's launches rotate through distinct device copies of
    the weight totalling >= 600 MB (beyond the 256 MB last-level cache).
    `us_per_launch`: the rotation captured as one HIP graph and replayed
    (>= 100 launches streaming, no host launch gaps); `launched_us`: the same
    launches issued one by one from the host; `single_us`: one launch between
    two events, the latency a lone call sees.  Algorithmic bytes:
    N*K/32*18 + 4K + 4N."""
    res = {}
    rng = np.random.default_rng(7)
    for name, N, K in (("q_o", 2048, 2048), ("k_v", 512, 2048), ("gate_up", 8192, 2048),
                       ("down", 2048, 8192), ("lm_head", 128256, 2048)):
        raw = pb.quantize_q4_0(pb.synth_normal(5000 + N + K, N * K, 0, 0.02).reshape(N, K))
        b = q4_bytes(N, K) + 4 * (N + K)
        copies = min(256, -(-600_000_000 // b))
        ws = [ctx.upload(pb.TYPE_Q4_0, N, K, raw) for _ in range(copies)]
        dx = ctx.alloc(K * 4).upload(rng.normal(0, 1, K).astype(np.float32))
        dy = ctx.alloc(N * 4)
        reps = max(2, -(-100 // copies))
        xs, ys = [dx.ptr] * copies, [dy.ptr] * copies
        ctx.bench_linear(ws, xs, ys, 1, 1)
        us = ctx.bench_linear(ws, xs, ys, 1, reps, graph=True) / reps / copies * 1e3
        launched = ctx.bench_linear(ws, xs, ys, 1, reps) / reps / copies * 1e3
        single = min(ctx.bench_linear([ws[i]], [dx.ptr], [dy.ptr], 1, 1) * 1e3
                     for i in range(min(8, copies)))
        res[name] = {"N": N, "K": K, "us_per_launch": round(us, 2),
                     "launched_us": round(launched, 2), "single_us": round(single, 2),
                     "achieved_GBps": round(b / us / 1e3, 1),
                     "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "algorithmic_bytes": b,
                     "rotated_copies": copies}
        log(f"q4_0 matvec {name} {N}x{K}: {us:.2f} us in a graph ({b / us / 1e3:.0f} GB/s, "
            f"{b / us / 1e3 / HBM_PEAK_GBS:.3f} of peak), {launched:.2f} us launched one by one, "
            f"{single:.2f} us alone")
        for w in ws:
            w.free()
        dx.free(), dy.free()
    return res


FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA, vendor figure


def run_gemm_types(ctx, pb):
    """The MFMA GEMM per weight type at M = 512 on a 2048 x 2048 matrix,
    timed back to back with HIP events: F32 on the fp32 MFMA, F16 / Q4_1 /
    Q4_0 on the fp16 MFMA (two issues per useful product, activations hi +
    lo).  Useful FLOPs 2*M*N*K."""
    res = {}
    M, N, K = 512, 2048, 2048
    W = pb.synth_normal(4300, N * K, 0, 0.02).reshape(N, K)
    dx = ctx.alloc(M * K * 4).upload(np.random.default_rng(6).normal(0, 1, M * K).astype(np.float32))
    dy = ctx.alloc(M * N * 4)
    for name, t, data, peak in (("f32", pb.TYPE_F32, W, FP32_MFMA_PEAK_TFLOPS),
                                ("f16", pb.TYPE_F16, pb.to_f16_bytes(W), MFMA_F16_PEAK_TFLOPS),
                                ("q4_1", pb.TYPE_Q4_1, pb.quantize_q4_1(W), MFMA_F16_PEAK_TFLOPS),
                                ("q4_0", pb.TYPE_Q4_0, pb.quantize_q4_0(W), MFMA_F16_PEAK_TFLOPS)):
        w = ctx.upload(t, N, K, data)
        ctx.bench_linear([w], [dx.ptr], [dy.ptr], M, 3)
        reps = 20
        us = ctx.bench_linear([w], [dx.ptr], [dy.ptr], M, reps) / reps * 1e3
        tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
        res[name] = {"M": M, "N": N, "K": K, "us_per_call": round(us, 2), "TFLOPs": round(tf, 2),
                     "peak": peak, "frac": round(tf / peak, 4)}
        log(f"gemm {name} M={M} N={N} K={K}: {us:.1f} us, {tf:.1f} TFLOP/s "
            f"({100 * tf / peak:.1f}% of {peak:.0f})")
        w.free()
    dx.free(), dy.free()
    return res


def run_gguf(ctx, pb, synth):
    """The file -> device path: a Llama-3.2-1B-shaped GGUF file as llama.cpp
    lays out a Q4_0 model (Q4_0 layer matrices, tied Q6_K token embedding,
    F32 norms) is written to a temporary directory, loaded with
    pbx_model_load_gguf (mmap, one pinned upload per tensor) and decoded
    greedily with the Q6_K LM head."""
    import tempfile
    cfg = dict(synth.CONFIGS["llama32_1b"], embed_type=pb.TYPE_Q6_K, max_seq=512)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "llama32_1b_q4_0.gguf")
        t0 = time.perf_counter()
        size = synth.write_gguf(path, cfg, seed=1000)
        log(f"gguf: wrote {size / 1e9:.2f} GB in {time.perf_counter() - t0:.1f}s")
        t0 = time.perf_counter()
        model = pb.Model.from_gguf(ctx, path, max_seq=512)
        ctx.sync()
        load_s = time.perf_counter() - t0
    log(f"gguf: loaded in {load_s * 1e3:.0f} ms ({size / load_s / 1e9:.2f} GB/s file to HBM)")
    prompt = synth.random_tokens(7, PROMPT, cfg["vocab_size"])
    _, nxt = model.forward(prompt, 0, want_logits=False)
    steps = 64
    model.generate(nxt, PROMPT, 8)
    model.rollback(PROMPT)
    ctx.sync()
    ctx.timer_start()
    model.generate(nxt, PROMPT, steps)
    ms = ctx.timer_stop() / steps
    model.rollback(PROMPT)
    us, by, _ = model.bench_role("lm_head", 8)
    log(f"gguf decode: {ms * 1e3:.1f} us/token, {1e3 / ms:.1f} tok/s; Q6_K lm head "
        f"{us:.1f} us, {by / us / 1e3:.0f} GB/s")
    model.free()
    return {"file_bytes": size, "load_ms": round(load_s * 1e3, 1),
            "load_GBps": round(size / load_s / 1e9, 2),
            "decode_tok_per_s": round(1e3 / ms, 1), "decode_us_per_token": round(ms * 1e3, 1),
            "lm_head_q6_k": {"us_per_launch": round(us, 2), "bytes_per_launch": round(by),
                             "GBps": round(by / us / 1e3, 1),
                             "frac_hbm": round(by / us / 1e3 / HBM_PEAK_GBS, 4)},
            "layout": "q4_0 layer matrices, tied q6_k token_embd, f32 norms (llama.cpp Q4_0)"}


def run_pmc_probe(args, pb, synth):
    """A short run for hardware-counter passes (rocprofv3 --pmc serialises
    every dispatch): the calibration copies and two decode steps of the same
    model.  Prints its progress."""
    cfg = synth.CONFIGS["llama32_1b"]
    ctx = pb.Context(0)
    log("probe: building model")
    model = synth.build(ctx, cfg, seed=1000)
    log("probe: calibration copies")
    measure_copy(ctx, reps=2)
    log("probe: prompt + 2 decode steps")
    _, nxt = model.forward(synth.random_tokens(7, 4, cfg["vocab_size"]), 0, want_logits=False)
    model.generate(nxt, 4, 2)
    ctx.sync()
    log("probe: done")
    model.free()
    ctx.close()
    return None


def run_matvec(args, pb, synth):
    """Per-token Q4_0 matvec pass through the plain instruction."""
    cfg = synth.CONFIGS["llama32_1b"]
    d, h, L, V = cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["vocab_size"]
    kv = cfg["n_kv_heads"] * (d // cfg["n_heads"])
    shapes = [("q", d, d), ("k", kv, d), ("v", kv, d), ("o", d, d), ("gate", h, d), ("up", h, d),
              ("down", d, h)]
    ctx = pb.Context(0)
    dev, _ = ctx.device_info()
    ops = []
    seed = 1000
    for l in range(L):
        for i, (name, N, K) in enumerate(shapes):
            raw = pb.quantize_q4_0(pb.synth_normal(seed + 16 * l + i, N * K, 0, 0.02).reshape(N, K))
            ops.append((name, N, K, ctx.upload(pb.TYPE_Q4_0, N, K, raw)))
    raw = pb.quantize_q4_0(pb.synth_normal(seed + 999, V * d, 0, 0.02).reshape(V, d))
    ops.append(("lm_head", V, d, ctx.upload(pb.TYPE_Q4_0, V, d, raw)))
    xb = {K: ctx.alloc(K * 4).upload(np.random.default_rng(K).normal(0, 1, K).astype(np.float32))
          for K in (d, h)}
    yb = ctx.alloc(V * 4)
    W = [w for (_, _, _, w) in ops]
    X = [xb[K].ptr for (_, _, K, _) in ops]
    Y = [yb.ptr] * len(ops)
    ctx.bench_linear(W, X, Y, 1, args.warmup)
    ms = ctx.bench_linear(W, X, Y, 1, args.steps)
    ms_per_step = ms / args.steps
    step_bytes = sum(q4_bytes(N, K) + 4 * (N + K) for (_, N, K, _) in ops)
    # the LM head alone, its launches separated by the 547 MB of layer weights
    sel = [w for (n, _, _, w) in ops if n == "lm_head"]
    t = ctx.bench_linear(sel, [xb[d].ptr], [yb.ptr], 1, 20) / 20
    b = q4_bytes(V, d) + 4 * (V + d)
    roofline = {"bound": "hbm", "kernel": "pbx_gemv_q4_0_wide_r16 (lm head)",
                "achieved": round(b / t / 1e6, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(b / t / 1e6 / HBM_PEAK_GBS, 4), "traffic": None}
    ctx.close()
    return {"metric": METRIC, "value": round(1e3 / ms_per_step, 2), "unit": "tok/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "q4_0 weights (int4 codes, fp16 block scales); each 32-element block of "
                     "the input rounded to 22-bit fixed point (three int8 limbs, exact int32 "
                     "dots); fp32 block combine and accumulation",
            "data": "synthetic: seeded N(0,0.02) weights quantised to Q4_0",
            "config": {"workload": "llama-3.2-1b-shaped q4_0 decode matvec pass only",
                       "bytes_per_step": step_bytes, "device": dev},
            "roofline": roofline, "cpu_baseline": None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--workload", choices=("decode", "matvec", "pmc-probe", "m-gt-1", "small"),
                    default="decode")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-m-gt-1", action="store_true",
                    help="skip the prefill / verify / speculative measurements")
    ap.add_argument("--no-small-configs", action="store_true",
                    help="skip the stories15M and SmolLM2 decode legs")
    ap.add_argument("--no-matvec-shapes", action="store_true",
                    help="skip the isolated matvec shapes (their timing captures HIP graphs, "
                         "which rocprofv3's kernel tracer can fault on)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/traffic_decode.json from two rocprofv3 --pmc runs")
    args = ap.parse_args()
    if args.summarize_pmc:
        res = summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1],
                            os.path.join(ROOT, "profiles", "traffic_decode.json"))
        print(json.dumps(res, indent=1))
        return
    if args.gpus != 1:
        print("bench.py: this backend runs on one GPU; runs over several GPUs are not "
              "supported", file=sys.stderr)
        sys.exit(2)
    if args.workload == "decode" and PROMPT + args.steps > 1024:
        print("bench.py: --steps must keep the KV cache within 1024 positions", file=sys.stderr)
        sys.exit(2)
    import purebee_amd as pb
    from purebee_amd import synth
    if args.workload == "pmc-probe":
        run_pmc_probe(args, pb, synth)
        return
    if args.workload == "small":
        res = {"stories15m": run_small_decode(pb, synth, "stories15m", 16, 128),
               "smollm2_135m": run_small_decode(pb, synth, "smollm2_135m", 32, 256)}
        print(json.dumps({"workload": "stories15M and SmolLM2-shaped q8_0 decode",
                          "small_configs": res}), flush=True)
        return
    if args.workload == "m-gt-1":
        cfg = synth.CONFIGS["llama32_1b"]
        ctx = pb.Context(0)
        model = synth.build(ctx, cfg, seed=1000)
        res = run_m_gt_1(ctx, model, cfg, pb, synth)
        model.free()
        ctx.close()
        print(json.dumps({"workload": "llama-3.2-1b-shaped q4_0, M>1 path", "m_gt_1": res}), flush=True)
        return
    out = run_decode(args, pb, synth) if args.workload == "decode" else run_matvec(args, pb, synth)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
