#!/usr/bin/env python3
"""Benchmark: Llama-3.2-1B-shaped Q4_0 decode matvecs on one MI355X.

Workload "matvec" (default): one step is the quantized-matvec pass of one
Llama-3.2-1B decode token at batch 1: for each of 16 layers the seven
projections q/k/v/o (2048x2048, 512x2048 x2, 2048x2048), gate/up
(8192x2048 x2) and down (2048x8192), then the tied 128256x2048 LM head, all
Q4_0, every layer with its own synthetic weights (SplitMix64/Box-Muller
N(0, 0.02), quantised d = absmax/8) so the 695 MB per step stream from HBM
rather than from the 256 MB MALL.  Activations are N(0,1).  Inputs are
resident in HBM before the timed region.

Prints one JSON line (the bench contract) with a roofline entry for the
kernel that takes the largest share of a step (HIP events on the context's
stream) and the restated reference CPU path timed on a bounded sample.
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

DIM, HIDDEN, LAYERS, KV_DIM, VOCAB = 2048, 8192, 16, 512, 128256
LAYER_SHAPES = [("q", DIM, DIM), ("k", KV_DIM, DIM), ("v", KV_DIM, DIM), ("o", DIM, DIM),
                ("gate", HIDDEN, DIM), ("up", HIDDEN, DIM), ("down", DIM, HIDDEN)]


def q4_bytes(N, K):
    """Algorithmic bytes of one Q4_0 matvec: weights + x + y."""
    return N * K // 32 * 18 + 4 * K + 4 * N


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_model(pb, ctx, seed=1000):
    """Quantised weights for every layer, uploaded once; host copies kept
    for the CPU baseline."""
    ops, host = [], {}
    t0 = time.time()
    for layer in range(LAYERS):
        for i, (name, N, K) in enumerate(LAYER_SHAPES):
            w = pb.synth_normal(seed + layer * 16 + i, N * K, 0.0, 0.02).reshape(N, K)
            raw = pb.quantize_q4_0(w)
            ops.append((name, N, K, ctx.upload(pb.TYPE_Q4_0, N, K, raw)))
            host[(layer, name)] = raw
    w = pb.synth_normal(seed + 999, VOCAB * DIM, 0.0, 0.02).reshape(VOCAB, DIM)
    raw = pb.quantize_q4_0(w)
    del w
    ops.append(("lm_head", VOCAB, DIM, ctx.upload(pb.TYPE_Q4_0, VOCAB, DIM, raw)))
    host["lm_head"] = raw
    log(f"weights generated+uploaded in {time.time() - t0:.1f}s")
    return ops, host


def cpu_baseline(host, seconds):
    """Restated reference CPU path (wasm-q4.js kernel in SSE + thread-pool.js
    row split, f32 LM head through wasmQ4.lmHead on the exactly dequantised
    embedding) on the same per-token matvec pass, for a bounded sample."""
    import oracle
    threads = min(16, os.cpu_count() or 1)
    pool = oracle.CpuPool(threads)
    emb = oracle.dequant_q4_0(host["lm_head"], VOCAB * DIM)
    xs = {K: np.asarray(np.random.default_rng(K).normal(0, 1, K), np.float32) for K in (DIM, HIDDEN)}
    outs = {}

    def one_token():
        for layer in range(LAYERS):
            for name, N, K in LAYER_SHAPES:
                outs[name] = pool.q4_0_matvec(xs[K], host[(layer, name)], N, K,
                                              outs.get(name) if name in outs else None)
        oracle.cpu_lm_head(xs[DIM], emb, VOCAB, DIM)

    one_token()  # warm-up
    t0 = time.perf_counter()
    one_token()
    per = time.perf_counter() - t0
    n = max(1, min(60, int(seconds / max(per, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(n):
        one_token()
    dt = time.perf_counter() - t0
    pool.close()
    return {"value": n / dt, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} tokens of the per-token Q4_0 matvec pass (16 layers x 7 matvecs on "
                      f"{threads} threads + single-threaded f32 LM head), {dt:.1f}s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this backend runs on one GPU; multi-GPU runs are not part of this "
              "build (see DESIGN.md for how the path would shard)", file=sys.stderr)
        sys.exit(2)

    import purebee_amd as pb
    ctx = pb.Context(0)
    dev, cus = ctx.device_info()
    log(f"device {dev}, {cus} CUs")
    ops, host = build_model(pb, ctx)
    xbuf = {K: ctx.alloc(K * 4).upload(np.random.default_rng(K).normal(0, 1, K).astype(np.float32))
            for K in (DIM, HIDDEN)}
    ybuf = ctx.alloc(VOCAB * 4)
    W = [w for (_, _, _, w) in ops]
    X = [xbuf[K].ptr for (_, _, K, _) in ops]
    Y = [ybuf.ptr for _ in ops]

    # warm-up, then the timed steps: HIP events on the context's stream
    ctx.bench_linear(W, X, Y, 1, args.warmup)
    ctx.sync()
    ms = ctx.bench_linear(W, X, Y, 1, args.steps)
    ms_per_step = ms / args.steps
    step_bytes = sum(q4_bytes(N, K) for (_, N, K, _) in ops)
    log(f"step {ms_per_step * 1e3:.1f} us, {step_bytes / ms_per_step / 1e6:.0f} GB/s aggregate")

    # per-kernel timing: each shape class over all its instances (distinct buffers)
    kernels = {}
    for cls, names in (("qo_2048x2048", ("q", "o")), ("kv_512x2048", ("k", "v")),
                       ("gateup_8192x2048", ("gate", "up")), ("down_2048x8192", ("down",)),
                       ("lmhead_128256x2048", ("lm_head",))):
        sel = [(N, K, w) for (n, N, K, w) in ops if n in names]
        Ws = [w for (_, _, w) in sel]
        Xs = [xbuf[K].ptr for (_, K, _) in sel]
        reps = max(1, 400 // len(sel))
        ctx.bench_linear(Ws, Xs, [ybuf.ptr] * len(sel), 1, 3)
        t = ctx.bench_linear(Ws, Xs, [ybuf.ptr] * len(sel), 1, reps)
        per_launch_us = t * 1e3 / (reps * len(sel))
        N, K, _ = sel[0]
        b = q4_bytes(N, K)
        kernels[cls] = {"N": N, "K": K, "launches_per_step": len(sel), "us_per_launch": per_launch_us,
                        "bytes_per_launch": b, "GBps": b / per_launch_us / 1e3,
                        "us_per_step": per_launch_us * len(sel)}
        log(f"{cls}: {per_launch_us:.2f} us/launch, {b / per_launch_us / 1e3:.0f} GB/s")
    dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]["us_per_step"])
    roofline = {"bound": "hbm", "kernel": dom_name, "achieved": round(dom["GBps"], 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4),
                "traffic": None}

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the restated reference CPU path ...")
        cpu = cpu_baseline(host, args.cpu_seconds)
        log(f"cpu baseline {cpu['value']:.2f} tok/s on {cpu['cores']} threads")

    out = {
        "metric": "Llama-3.2-1B Q4 decode tok/s @1 GPU; Q4 matvec HBM GB/s vs peak",
        "value": round(1e3 / ms_per_step, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights, fp32 activations/accumulation",
        "data": "synthetic (seeded N(0,0.02) weights quantised to Q4_0, N(0,1) activations)",
        "config": {"workload": "llama-3.2-1b q4_0 decode matvec pass: 16 layers x "
                               "(q,k,v,o,gate,up,down) + tied 128256x2048 lm head, batch 1",
                   "bytes_per_step": step_bytes,
                   "aggregate_GBps": round(step_bytes / ms_per_step / 1e6, 1),
                   "device": dev},
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
