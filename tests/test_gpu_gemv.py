"""GPU parity of the quantized matvec instruction through the C ABI.

Bars (stated per test):
  * dequantised weights: bit-exact against the oracle (gguf.js:239-286);
  * matvec / matmul outputs: relative L2 <= 1e-3 against the oracle's
    double-accumulated restatement (llama-streaming.js:72-104 for Q4_0).
"""
import numpy as np
import pytest

import oracle
import purebee_amd as pb
from tests.conftest import rel_l2, synth_matrix

pytestmark = pytest.mark.gpu

TOL = 1e-3  # relative L2, matvec outputs

# (N, K) shapes of the configurations: Llama-3.2-1B, SmolLM2-135M, stories15M
LLAMA1B = [(2048, 2048), (512, 2048), (8192, 2048), (2048, 8192)]
SMOLLM2 = [(576, 576), (192, 576), (1536, 576), (576, 1536)]
STORIES = [(288, 288), (768, 288), (288, 768)]
EDGE = [(1, 32), (7, 64), (65, 96), (1000, 1056), (129, 2080), (3, 16384), (63, 4064)]


QUANT = [pb.TYPE_Q4_0, pb.TYPE_Q4_1, pb.TYPE_Q8_0]


def quantize(t, w):
    return {pb.TYPE_Q4_0: oracle.quantize_q4_0, pb.TYPE_Q4_1: oracle.quantize_q4_1,
            pb.TYPE_Q8_0: oracle.quantize_q8_0}[t](w)


def dequant(t, raw, n):
    return {pb.TYPE_Q4_0: oracle.dequant_q4_0, pb.TYPE_Q4_1: oracle.dequant_q4_1,
            pb.TYPE_Q8_0: oracle.dequant_q8_0}[t](raw, n)


@pytest.mark.parametrize("t", QUANT)
@pytest.mark.parametrize("N,K", LLAMA1B[:2] + SMOLLM2[:2] + STORIES[:2] + EDGE[:4])
def test_dequant_bit_exact(ctx, t, N, K):
    print(f"[case] dequant type={t} N={N} K={K}", flush=True)
    raw = quantize(t, synth_matrix(100 + N + K, N, K))
    w = ctx.upload(t, N, K, raw)
    got = ctx.dequant(w)
    ref = dequant(t, raw, N * K).reshape(N, K)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    w.free()


def test_reference_q4_kat(ctx):
    """wasm-q4.js:673-704 on the GPU path: [32, 128] within 0.1."""
    print("[case] q4 KAT", flush=True)
    raw = np.zeros(36, np.uint8)
    raw[0:2] = [0x00, 0x3C]
    raw[2:18] = 0x99
    raw[18:20] = [0x00, 0x40]
    raw[20:36] = 0xAA
    w = ctx.upload(pb.TYPE_Q4_0, 2, 32, raw)
    y = ctx.linear(w, np.ones(32, np.float32))
    assert abs(y[0] - 32.0) < 0.1 and abs(y[1] - 128.0) < 0.1
    assert y[0] == 32.0 and y[1] == 128.0
    w.free()


@pytest.mark.parametrize("t", QUANT)
@pytest.mark.parametrize("N,K", LLAMA1B + SMOLLM2 + STORIES + EDGE)
def test_matvec_parity(ctx, t, N, K):
    print(f"[case] matvec type={t} N={N} K={K}", flush=True)
    raw = quantize(t, synth_matrix(7 * N + K, N, K))
    x = pb.synth_normal(N ^ K, K)
    w = ctx.upload(t, N, K, raw)
    y = ctx.linear(w, x)
    ref = oracle.matvec(t, x, raw, N, K)
    assert y.shape == (N,)
    assert rel_l2(y, ref) <= TOL, rel_l2(y, ref)
    # fp32 accumulation in a different order: in practice far below the bar
    assert rel_l2(y, ref) < 1e-5
    w.free()


def test_lm_head_q4_0_llama(ctx):
    """The tied 128256 x 2048 Q4_0 embedding as LM head (the largest GEMV)."""
    N, K = 128256, 2048
    print(f"[case] lm head q4_0 N={N} K={K}", flush=True)
    raw = pb.quantize_q4_0(synth_matrix(4242, N, K))
    x = pb.synth_normal(17, K)
    w = ctx.upload(pb.TYPE_Q4_0, N, K, raw)
    y = ctx.linear(w, x)
    ref = oracle.q4_0_matvec_js(x, raw, N, K)
    assert rel_l2(y, ref) <= TOL
    assert int(np.argmax(y)) == int(np.argmax(ref))
    w.free()


@pytest.mark.parametrize("N,K", [(32000, 288), (49152, 576), (300, 2048), (5, 64)])
def test_f32_matvec_lm_head(ctx, N, K):
    """f32 weights: the reference LM head of llama.js:359-367 / batch_dot."""
    print(f"[case] f32 matvec N={N} K={K}", flush=True)
    W = synth_matrix(N + 3 * K, N, K)
    x = pb.synth_normal(5, K)
    w = ctx.upload(pb.TYPE_F32, N, K, W)
    y = ctx.linear(w, x)
    assert rel_l2(y, oracle.f32_matvec(x, W)) <= TOL
    assert rel_l2(y, oracle.batch_dot_wasm(x, W)) < 1e-5
    assert np.array_equal(ctx.dequant(w), W)
    w.free()


def q4_1_special_blocks():
    """Q4_1 rows of 64 columns covering the scale corner cases: d = 0
    (constant block: every element is m), negative and positive minima, a
    subnormal d, and the largest finite fp16 m.  Row r, block b."""
    cases = [(0x0000, 0x3C00), (0x3C00, 0xC800), (0x2E66, 0x2E66), (0x0001, 0x8000),
             (0x0200, 0x7BFF), (0x4000, 0x0000), (0x3555, 0xB555), (0x1400, 0x9400)]
    rng = np.random.default_rng(3)
    raw = np.zeros((len(cases) // 2, 2, 20), np.uint8)
    for i, (d, m) in enumerate(cases):
        blk = raw[i // 2, i % 2]
        blk[0:2] = [d & 0xFF, d >> 8]
        blk[2:4] = [m & 0xFF, m >> 8]
        blk[4:] = rng.integers(0, 256, 16)
    return raw.ravel(), len(cases) // 2, 64


def test_q4_1_special_scales(ctx):
    """Dequant bit-exact and matvec against gguf.js:288-314 /
    llama-streaming.js:115-151 on hand-made scale corner cases."""
    print("[case] q4_1 special scales", flush=True)
    raw, N, K = q4_1_special_blocks()
    w = ctx.upload(pb.TYPE_Q4_1, N, K, raw)
    got = ctx.dequant(w)
    ref = oracle.dequant_q4_1(raw, N * K).reshape(N, K)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    x = pb.synth_normal(5, K)
    y = ctx.linear(w, x)
    assert rel_l2(y, oracle.q4_1_matvec_js(x, raw, N, K)) < 1e-5
    w.free()


def test_q4_1_from_q4_0_kat(ctx):
    """The reference KAT (wasm-q4.js:673-704) rewritten as Q4_1 blocks with
    m = -8d, which encode the same values: [32, 128] exactly."""
    print("[case] q4_1 KAT identity", flush=True)
    raw = np.zeros(40, np.uint8)
    raw[0:4] = [0x00, 0x3C, 0x00, 0xC8]   # d = 1, m = -8
    raw[4:20] = 0x99
    raw[20:24] = [0x00, 0x40, 0x00, 0xCC]  # d = 2, m = -16
    raw[24:40] = 0xAA
    w = ctx.upload(pb.TYPE_Q4_1, 2, 32, raw)
    y = ctx.linear(w, np.ones(32, np.float32))
    assert y[0] == 32.0 and y[1] == 128.0
    w.free()


@pytest.mark.parametrize("M", [2, 7, 64])
def test_q4_1_multi_row(ctx, M):
    """M > 1 on Q4_1 (one GEMV grid row per activation row)."""
    N, K = 1536, 576
    print(f"[case] q4_1 multi-row M={M}", flush=True)
    raw = oracle.quantize_q4_1(synth_matrix(M + 40, N, K))
    X = pb.synth_normal(M, M * K).reshape(M, K)
    w = ctx.upload(pb.TYPE_Q4_1, N, K, raw)
    Y = ctx.linear(w, X)
    for m in range(M):
        assert rel_l2(Y[m], oracle.q4_1_matvec_js(X[m], raw, N, K)) < 1e-5
    w.free()


def gguf_bytes(t, W):
    """W as the GGUF bytes of type t (F16 halves, or oracle-quantised Q6_K)."""
    if t == pb.TYPE_F16:
        return W.astype(np.float16).view(np.uint8).ravel()
    return oracle.quantize_q6_k(W)


EMBED_SHAPES = [(1000, 2048), (300, 576 // 32 * 32), (77, 256), (129, 1024), (64, 8192)]


@pytest.mark.parametrize("t", [pb.TYPE_F16, pb.TYPE_Q6_K])
@pytest.mark.parametrize("N,K", EMBED_SHAPES)
def test_f16_q6_k_dequant_and_matvec(ctx, t, N, K):
    """F16 / Q6_K weights (gguf.js:231-237, 317-364): dequantisation
    bit-exact; the matvec against the reference's route for these types
    (dequantise to f32, then the f32 matvec) at 1e-5 relative L2."""
    if t == pb.TYPE_Q6_K and K % 256:
        K = K // 256 * 256 or 256
    print(f"[case] type={t} N={N} K={K}", flush=True)
    W = synth_matrix(N * 3 + K + t, N, K)
    raw = gguf_bytes(t, W)
    w = ctx.upload(t, N, K, raw)
    got = ctx.dequant(w)
    ref = oracle.dequant(t, raw, N * K).reshape(N, K)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    x = pb.synth_normal(N + K, K)
    y = ctx.linear(w, x)
    assert rel_l2(y, oracle.matvec(t, x, raw, N, K)) < 1e-5
    X = pb.synth_normal(N + K + 1, 3 * K).reshape(3, K)
    Y = ctx.linear(w, X)
    for m in range(3):
        assert rel_l2(Y[m], oracle.matvec(t, X[m], raw, N, K)) < 1e-5
    w.free()


def test_f16_all_patterns_on_gpu(ctx):
    """float16ToFloat32 (gguf.js:55-70) on the GPU over all 65,536 patterns:
    once as one F16 weight (gguf.js:231-237) and once as the fp16 scales of
    65,536 Q8_0 blocks whose codes are +1 / -1 (gguf.js:239-257), so the
    dequantised values are +-f16(pattern).  Bit-exact against the oracle,
    NaN compared by isnan (subnormals, +-0, +-inf included)."""
    print("[case] f16 all patterns (F16 weight, Q8_0 scales)", flush=True)
    bits = np.arange(65536, dtype=np.uint16)
    raw = bits.view(np.uint8).copy()
    w = ctx.upload(pb.TYPE_F16, 64, 1024, raw)
    got = ctx.dequant(w).ravel()
    w.free()
    ref = oracle.dequant_f16(raw, 65536)
    ieee = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(ieee)) and np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.array_equal(ref[~nan].view(np.uint32), ieee[~nan].view(np.uint32))
    blk = np.zeros((65536, 34), np.uint8)
    blk[:, :2] = bits.view(np.uint8).reshape(-1, 2)
    blk[:, 2:18] = 1
    blk[:, 18:] = 0xFF  # int8 -1
    raw8 = blk.ravel()
    w = ctx.upload(pb.TYPE_Q8_0, 2048, 1024, raw8)
    got8 = ctx.dequant(w).reshape(65536, 32)
    w.free()
    ref8 = oracle.dequant_q8_0(raw8, 65536 * 32).reshape(65536, 32)
    nan8 = np.isnan(ref8)
    assert np.array_equal(np.isnan(got8), nan8)
    assert np.array_equal(got8[~nan8].view(np.uint32), ref8[~nan8].view(np.uint32))
    assert np.array_equal(got8[:, 0][~nan].view(np.uint32), ieee[~nan].view(np.uint32))
    assert np.array_equal(got8[:, 31][~nan].view(np.uint32), (-ieee)[~nan].view(np.uint32))


def test_q6_k_rejects_k_not_multiple_of_256(ctx):
    print("[case] q6_k K % 256", flush=True)
    with pytest.raises(pb.PbxError):
        ctx.upload(pb.TYPE_Q6_K, 4, 288, np.zeros(4 * 2 * 210, np.uint8))


@pytest.mark.parametrize("t", QUANT + [pb.TYPE_F32])
def test_bias_and_multi_row(ctx, t):
    N, K, M = 576, 576, 5
    print(f"[case] bias/multi-row type={t}", flush=True)
    W = synth_matrix(31, N, K)
    data = W if t == pb.TYPE_F32 else quantize(t, W)
    X = pb.synth_normal(32, M * K).reshape(M, K)
    bias = pb.synth_normal(33, N)
    w = ctx.upload(t, N, K, data)
    Y = ctx.linear(w, X, bias)
    for m in range(M):
        ref = (oracle.f32_matvec(X[m], W) if t == pb.TYPE_F32
               else oracle.matvec(t, X[m], data, N, K)) + bias
        assert rel_l2(Y[m], ref) <= TOL
    w.free()


@pytest.mark.parametrize("t", [pb.TYPE_Q4_0, pb.TYPE_Q8_0])
@pytest.mark.parametrize("N,K,M,bias", [
    (512, 2048, 3, True),      # 4 waves x 1 row, one 64-block group a lane
    (2048, 2048, 2, False),    # 4 x 2
    (8192, 2048, 1, True),     # 16 x 4 (Q4_0) / 8 x 4 (Q8_0)
    (8192, 4096, 2, True),     # 8 x 4, two groups
    (1000, 3104, 3, False),    # B = 97: the second group's lanes past B masked
    (2048, 8192, 1, True),     # 4 x 2, four groups
    (2048, 7168, 1, True),     # builder-wave kernel with B = 224: its last chunk's
    (2048, 7168, 3, False),    #   blocks past B masked (limbs and scales unwritten)
    (4096, 6400, 2, True),     # B = 200
    (70000, 2048, 1, False),   # tall, no bias: the tile loop (512 workgroups)
    (70000, 2048, 2, True),    # tall with bias: one tile a workgroup
])
def test_integer_limb_instruction(ctx, monkeypatch, t, N, K, M, bias):
    """The instruction's integer-limb kernels (Q4_0 / Q8_0, K = 2048..8192)
    against the oracle and against the float-unpack kernels
    (PBX_GEMV_INT=0), for 1-3 activation rows with and without bias."""
    print(f"[case] integer-limb linear type={t} N={N} K={K} M={M} bias={bias}", flush=True)
    raw = quantize(t, synth_matrix(3 * N + K, N, K))
    X = pb.synth_normal(N + 5 * K, M * K).reshape(M, K)
    b = pb.synth_normal(N + 1, N) if bias else None
    w = ctx.upload(t, N, K, raw)
    Y = ctx.linear(w, X, b)
    monkeypatch.setenv("PBX_GEMV_INT", "0")
    fctx = pb.Context(0)
    monkeypatch.delenv("PBX_GEMV_INT")
    wf = fctx.upload(t, N, K, raw)
    F = fctx.linear(wf, X, b)
    for m in range(M):
        ref = oracle.matvec(t, X[m], raw, N, K) + (b if bias else 0)
        assert rel_l2(Y[m], ref) < 1e-5, (m, rel_l2(Y[m], ref))
        assert rel_l2(Y[m], F[m]) < 1e-5
    wf.free()
    fctx.close()
    w.free()


@pytest.mark.parametrize("t", [pb.TYPE_Q4_0, pb.TYPE_Q8_0])
@pytest.mark.parametrize("N,K", [(512, 2048), (2048, 8192), (70000, 2048)])
def test_integer_limb_non_finite_activations(ctx, monkeypatch, t, N, K):
    """A row of x holding +inf, -inf or NaN: the reference's sums
    (llama-streaming.js:72-104) are then NaN or +-inf in every output; the
    integer-limb kernels (one and several prologue slots, the tile loop)
    must give non-finite outputs exactly where the oracle and the float
    kernels (PBX_GEMV_INT=0) do, and the finite rows of the same call must
    be unaffected."""
    print(f"[case] integer-limb non-finite x type={t} N={N} K={K}", flush=True)
    raw = quantize(t, synth_matrix(7 * N + K, N, K))
    X = pb.synth_normal(N + 3 * K, 4 * K).reshape(4, K)
    X[0, 5] = np.inf
    X[1, K - 1] = -np.inf
    X[2, K // 2] = np.nan
    w = ctx.upload(t, N, K, raw)
    Y = np.stack([ctx.linear(w, X[m]) for m in range(4)])
    Y3 = ctx.linear(w, X[[3, 0, 3]])  # rows of one launch: finite, inf, finite
    monkeypatch.setenv("PBX_GEMV_INT", "0")
    fctx = pb.Context(0)
    monkeypatch.delenv("PBX_GEMV_INT")
    wf = fctx.upload(t, N, K, raw)
    F = np.stack([fctx.linear(wf, X[m]) for m in range(4)])
    for m in range(3):
        ref = oracle.matvec(t, X[m], raw, N, K)
        assert not np.isfinite(ref).any()
        assert not np.isfinite(F[m]).any()
        assert not np.isfinite(Y[m]).any(), (m, np.isfinite(Y[m]).sum())
    ref3 = oracle.matvec(t, X[3], raw, N, K)
    assert rel_l2(Y[3], ref3) < 1e-5
    assert rel_l2(Y3[0], ref3) < 1e-5 and rel_l2(Y3[2], ref3) < 1e-5
    assert not np.isfinite(Y3[1]).any()
    wf.free()
    fctx.close()
    w.free()


@pytest.mark.parametrize("K,N,M", [(288, 288, 1), (288, 768, 1), (768, 288, 3), (64, 100, 2)])
def test_q8_ref_tensor_matches_matmul_q8(ctx, K, N, M):
    """The reference's own QuantizedTensor (quantize.js) through
    tensorMulAddQ8 -> matmul_q8 (quantize.js:224-266)."""
    print(f"[case] q8ref K={K} N={N} M={M}", flush=True)
    Wkn = synth_matrix(K * 7 + N, K, N)
    q, s = oracle.quantize_q8_ref(Wkn)
    X = pb.synth_normal(M + 1, M * K).reshape(M, K)
    X[0, 3] = 0.0  # the skipped-zero branch
    bias = pb.synth_normal(9, N)
    w = ctx.upload_q8ref(K, N, q, s)
    Y = ctx.linear(w, X, bias)
    ref = oracle.matmul_q8_ref(X, q, s, N, bias)
    assert rel_l2(Y, ref) <= TOL
    assert rel_l2(Y, ref) < 1e-5
    assert np.array_equal(ctx.dequant(w).ravel(), oracle.dequant_q8_ref(q, s))
    w.free()


def test_device_pointer_path_and_reuse(ctx):
    """pbx_linear_dev on device buffers; the same resident weight reused."""
    N, K = 2048, 8192
    print("[case] device-pointer path", flush=True)
    raw = pb.quantize_q4_0(synth_matrix(77, N, K))
    w = ctx.upload(pb.TYPE_Q4_0, N, K, raw)
    dx = ctx.alloc(K * 4)
    dy = ctx.alloc(N * 4)
    for seed in (1, 2, 3):
        x = pb.synth_normal(seed, K)
        dx.upload(x)
        ctx.linear_dev(w, dx.ptr, 1, dy.ptr)
        ctx.sync()
        y = dy.download(np.float32, N)
        assert rel_l2(y, oracle.q4_0_matvec_js(x, raw, N, K)) <= TOL
    dx.free()
    dy.free()
    w.free()


def test_error_paths_on_device(ctx):
    print("[case] error paths", flush=True)
    with pytest.raises(pb.PbxError) as e:
        ctx.upload(pb.TYPE_Q4_0, 4, 33, np.zeros(200, np.uint8))
    assert e.value.code == -1 and "K%32" in str(e.value)
    with pytest.raises(pb.PbxError) as e:
        ctx.upload(pb.TYPE_Q4_0, 4, 64, np.zeros(10, np.uint8))
    assert e.value.code == -1 and "needs 144" in str(e.value)
    with pytest.raises(pb.PbxError) as e:
        ctx.upload(5, 4, 64, np.zeros(1000, np.uint8))
    assert e.value.code == -1
    # K beyond the GEMV limit uploads but the launch reports ENOTSUP
    w = ctx.upload(pb.TYPE_Q4_0, 2, 16416, np.zeros(2 * 513 * 18, np.uint8))
    with pytest.raises(pb.PbxError) as e:
        ctx.linear(w, np.zeros(16416, np.float32))
    assert e.value.code == -5
    w.free()
    # a NULL handle is rejected before any HIP call
    with pytest.raises(pb.PbxError) as e:
        ctx._call("pbx_linear", ctx._p, None, np.zeros(32, np.float32).ctypes.data, 1, None,
                  np.zeros(2, np.float32).ctypes.data)
    assert e.value.code == -1


GEMM_SHAPES = [(2048, 2048), (512, 2048), (8192, 2048), (2048, 8192), (576, 576), (1536, 576),
               (576, 1536), (288, 288), (768, 288), (288, 768), (100, 64), (64, 32)]


def weight_bytes(t, W):
    if t == pb.TYPE_F32:
        return W
    if t == pb.TYPE_F16:
        return pb.to_f16_bytes(W)
    return quantize(t, W)


@pytest.mark.parametrize("t", QUANT + [pb.TYPE_F16, pb.TYPE_F32])
@pytest.mark.parametrize("M", [4, 5, 17, 33, 64, 130])
@pytest.mark.parametrize("N,K", GEMM_SHAPES)
def test_mfma_gemm_parity(ctx, t, M, N, K):
    """M >= 4 takes the MFMA path (exact integer weight codes or fp16
    weights, activations as an fp16 pair hi + lo; F32 weights on the fp32
    MFMA; fp32 accumulation): every row within 1e-5 relative L2 of the
    oracle's double-accumulated matvec and of the M=1 GEMV (the matvec bar is
    1e-3; single-fp16 activations would sit near 2e-4)."""
    print(f"[case] gemm type={t} M={M} N={N} K={K}", flush=True)
    tol = 1e-5
    raw = weight_bytes(t, synth_matrix(11 * N + K + M, N, K))
    X = pb.synth_normal(M * 7 + K, M * K).reshape(M, K)
    X[1] *= 1e-3   # rows of very different magnitude: per-row scaling
    X[2] *= 300.0
    bias = pb.synth_normal(3, N)
    w = ctx.upload(t, N, K, raw)
    Y = ctx.linear(w, X, bias)
    assert Y.shape == (M, N)
    rows = range(M) if M <= 17 else [0, 1, 2, M // 2, M - 1]
    worst = 0.0
    for m in rows:
        ref = oracle.matvec(t, X[m], raw, N, K) + bias
        worst = max(worst, rel_l2(Y[m], ref))
    print(f"  worst rel L2 vs oracle {worst:.2e}")
    assert worst <= tol
    # every row against the M=1 GEMV (fp32 path)
    for m in range(M):
        assert rel_l2(Y[m], ctx.linear(w, X[m]) + bias) <= tol
    w.free()


def test_mfma_gemm_prefill_shape(ctx):
    """The prefill shape of the M>1 config: M = 512 on the gate/up matrix."""
    N, K, M = 16384, 2048, 512
    print(f"[case] gemm prefill M={M} N={N} K={K}", flush=True)
    raw = pb.quantize_q4_0(synth_matrix(99, N, K))
    X = pb.synth_normal(98, M * K).reshape(M, K)
    w = ctx.upload(pb.TYPE_Q4_0, N, K, raw)
    Y = ctx.linear(w, X)
    for m in (0, 255, 511):
        assert rel_l2(Y[m], oracle.q4_0_matvec_js(X[m], raw, N, K)) <= TOL
    w.free()
