"""pbx_linear_dev_noalloc (the entry point that allocates nothing; its GEMM
workspace is a static device array) against pbx_linear_dev on the same
inputs: identical outputs, for two calls in a row, the second with a
smaller input, over the GEMV (M < 4) and MFMA GEMM (split K) paths and the
f32 path; a shape beyond the workspace limit is refused."""
import ctypes

import numpy as np
import pytest

import oracle
import purebee_amd as pb
from tests.conftest import rel_l2, synth_matrix

pytestmark = pytest.mark.gpu


def run_both(ctx, w, K, N, M, bias):
    X = pb.synth_normal(17 * M + K, M * K).reshape(M, K)
    dx = ctx.alloc(M * K * 4).upload(X)
    db = ctx.alloc(N * 4).upload(bias) if bias is not None else None
    dy1, dy2 = ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
    ctx.linear_dev(w, dx.ptr, M, dy1.ptr, db.ptr if db else None)
    ctx.linear_dev_noalloc(w, dx.ptr, M, dy2.ptr, db.ptr if db else None)
    ctx.sync()
    y1 = dy1.download(np.float32, M * N).reshape(M, N)
    y2 = dy2.download(np.float32, M * N).reshape(M, N)
    for b in (dx, db, dy1, dy2):
        if b is not None:
            b.free()
    return X, y1, y2


@pytest.mark.parametrize("t,N,K,Ms", [
    (pb.TYPE_Q4_0, 2048, 2048, (512, 64)),   # MFMA GEMM, then a smaller split-K GEMM
    (pb.TYPE_Q4_0, 16384, 2048, (5, 2)),     # skinny GEMM, then the GEMV
    (pb.TYPE_Q8_0, 576, 1536, (33, 4)),
    (pb.TYPE_F32, 1024, 512, (100, 8)),      # f32 MFMA with split-K partials
])
def test_noalloc_equals_linear_dev(ctx, t, N, K, Ms):
    print(f"[case] noalloc type={t} N={N} K={K} M={Ms}", flush=True)
    W = synth_matrix(N + 3 * K + t, N, K)
    data = W if t == pb.TYPE_F32 else {pb.TYPE_Q4_0: oracle.quantize_q4_0,
                                       pb.TYPE_Q8_0: oracle.quantize_q8_0}[t](W)
    w = ctx.upload(t, N, K, data)
    bias = pb.synth_normal(N + 7, N)
    for i, M in enumerate(Ms):
        X, y1, y2 = run_both(ctx, w, K, N, M, bias if i == 0 else None)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), (M, np.abs(y1 - y2).max())
        m = M - 1
        ref = (oracle.f32_matvec(X[m], W) if t == pb.TYPE_F32
               else oracle.matvec(t, X[m], data, N, K)) + (bias if i == 0 else 0)
        assert rel_l2(y2[m], ref) < 1e-3
    w.free()


def test_noalloc_rejects_shapes_beyond_the_workspace(ctx):
    print("[case] noalloc workspace limit", flush=True)
    N, K, M = 256, 8192, 4096   # fp16 activation pair alone: 2 * 4096 * 8192 * 2 B = 128 MiB
    w = ctx.upload(pb.TYPE_Q4_0, N, K, oracle.quantize_q4_0(synth_matrix(5, N, K)))
    dx, dy = ctx.alloc(M * K * 4), ctx.alloc(M * N * 4)
    with pytest.raises(pb.PbxError, match="workspace"):
        ctx.linear_dev_noalloc(w, dx.ptr, M, dy.ptr)
    dx.free(), dy.free(), w.free()


def test_noalloc_allocates_nothing_and_captures(ctx):
    """On a fresh context, the no-allocation entry point goes first, on a
    split-K MFMA GEMM shape (fp16 activation pair, row scales and partials
    all in the static workspace): the context's grown workspace stays 0.
    The same call is then captured into a HIP graph in global capture mode
    (which fails if anything in it allocates or synchronises) and the graph
    replayed three times, with the program's own work and synchronisations
    between the replays; every replay equals the eager result bit for bit.
    pbx_linear_dev afterwards gives the same result and does grow its
    workspace."""
    print("[case] noalloc on a fresh context: no growth, global-mode graph capture", flush=True)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [ctypes.c_void_p]
    hip.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    N, K, M = 2048, 2048, 64
    W = synth_matrix(91, N, K)
    raw = oracle.quantize_q4_0(W)
    with pb.Context(0) as fresh:
        assert fresh.workspace_info()[0] == 0
        w = fresh.upload(pb.TYPE_Q4_0, N, K, raw)
        X = pb.synth_normal(92, M * K).reshape(M, K)
        dx = fresh.alloc(M * K * 4).upload(X)
        dy = [fresh.alloc(M * N * 4) for _ in range(3)]
        fresh.linear_dev_noalloc(w, dx.ptr, M, dy[0].ptr)
        fresh.sync()
        grown, static = fresh.workspace_info()
        assert grown == 0 and static == pb.native.NOALLOC_WORKSPACE_BYTES, (grown, static)
        eager = dy[0].download(np.float32, M * N)
        ref = oracle.matvec(pb.TYPE_Q4_0, X[M - 1], raw, N, K)
        assert rel_l2(eager.reshape(M, N)[M - 1], ref) < 1e-3
        stream = ctypes.c_void_p(fresh.stream())
        assert hip.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
        fresh.linear_dev_noalloc(w, dx.ptr, M, dy[1].ptr)
        graph, gexec = ctypes.c_void_p(), ctypes.c_void_p()
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert hip.hipGraphInstantiate(ctypes.byref(gexec), graph, None, None, 0) == 0
        for rep in range(3):
            dy[1].upload(np.full(M * N, np.nan, np.float32))
            assert hip.hipGraphLaunch(gexec, stream) == 0
            fresh.sync()
            got = dy[1].download(np.float32, M * N)
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), rep
            fresh.linear_dev_noalloc(w, dx.ptr, 3, dy[2].ptr)  # eager work between replays
            fresh.sync()
        hip.hipGraphExecDestroy(gexec)
        hip.hipGraphDestroy(graph)
        assert fresh.workspace_info()[0] == 0
        fresh.linear_dev(w, dx.ptr, M, dy[2].ptr)
        fresh.sync()
        assert np.array_equal(dy[2].download(np.float32, M * N).view(np.uint32), eager.view(np.uint32))
        assert fresh.workspace_info()[0] > 0
        for b in (dx, *dy):
            b.free()
        w.free()
