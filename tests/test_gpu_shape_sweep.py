"""Seeded random shapes through the instruction (pbx_linear, llama-streaming.js:168-177 /
engine.js:180-269): every weight type the boundary takes, odd N and K (any number of
32-blocks, Q6_K in 256-blocks), 1..40 activation rows (the GEMV kernels below 4 rows, the MFMA
GEMM from 4) with and without bias, through host buffers and device pointers.  Each row within
1e-5 relative L2 of the oracle's double-accumulated matvec (the same bar as the fixed-shape
tests), so the kernel and shape selection is exercised away from the model shapes."""
import numpy as np
import pytest

import oracle
import purebee_amd as pb
from tests.conftest import rel_l2, synth_matrix

pytestmark = pytest.mark.gpu

TYPES = [pb.TYPE_Q4_0, pb.TYPE_Q8_0, pb.TYPE_Q4_1, pb.TYPE_F16, pb.TYPE_Q6_K, pb.TYPE_F32]


def weight_bytes(t, W):
    if t == pb.TYPE_F32:
        return W
    if t == pb.TYPE_F16:
        return W.astype(np.float16).view(np.uint8).ravel()
    return {pb.TYPE_Q4_0: oracle.quantize_q4_0, pb.TYPE_Q4_1: oracle.quantize_q4_1,
            pb.TYPE_Q8_0: oracle.quantize_q8_0, pb.TYPE_Q6_K: oracle.quantize_q6_k}[t](W)


def reference(t, x, raw, W, N, K):
    if t == pb.TYPE_F32:
        return oracle.f32_matvec(x, W)
    return oracle.matvec(t, x, raw, N, K)


def draw(case):
    rng = np.random.default_rng(91000 + case)
    t = TYPES[case % len(TYPES)]
    if t == pb.TYPE_Q6_K:
        K = 256 * int(rng.integers(1, 17))
    else:
        K = 32 * int(rng.integers(1, 257))
    N = int(rng.integers(1, 2600))
    M = int(rng.choice([1, 1, 2, 3, 4, 5, 7, 8, 16, 33, 40]))
    # keep the oracle's work (N K M multiply-adds in C) to a few hundred million
    while N * K * M > 3e8 and M > 1:
        M //= 2
    return t, N, K, M, bool(rng.random() < 0.5), bool(rng.random() < 0.3)


@pytest.mark.parametrize("case", range(48))
def test_random_shape_linear(ctx, case):
    t, N, K, M, bias, dev = draw(case)
    print(f"[case] sweep {case}: type={t} N={N} K={K} M={M} bias={bias} device={dev}", flush=True)
    W = synth_matrix(5 * N + 3 * K + case, N, K)
    raw = weight_bytes(t, W)
    X = pb.synth_normal(7 * N + K + case, M * K).reshape(M, K)
    b = pb.synth_normal(N + case, N) if bias else None
    w = ctx.upload(t, N, K, raw)
    if dev:
        dx = ctx.alloc(M * K * 4).upload(X)
        dy = ctx.alloc(M * N * 4)
        db = ctx.alloc(N * 4).upload(b) if bias else None
        ctx.linear_dev(w, dx.ptr, M, dy.ptr, db.ptr if bias else None)
        Y = dy.download(np.float32, M * N).reshape(M, N)
        for buf in (dx, dy, db):
            if buf is not None:
                buf.free()
    else:
        Y = ctx.linear(w, X, b).reshape(M, N)
    worst = 0.0
    for m in range(M):
        ref = reference(t, X[m], raw, W, N, K) + (b if bias else 0.0)
        worst = max(worst, rel_l2(Y[m], ref))
    print(f"  worst rel L2 vs oracle {worst:.2e}", flush=True)
    assert worst < 1e-5
    w.free()
