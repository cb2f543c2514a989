"""Pins the oracle (CPU restatement of the reference arithmetic) against the
reference's own known-answer tests and against what mathematics fixes.

Reference KATs used:
  wasm-q4.js:673-704   Q4_0 matvec self-test: rows -> [32, 128] (also, re-encoded
                       as Q4_1 blocks with m = -8d, the Q4_1 pin)
  wasm-simd.js:367-385 f32 matmul self-test (2x3 . 3x5 identity-like)
  main.js:65-74        TENSOR_MUL [2,3]x[3,2] -> [58, 64, 139, 154]
"""
import numpy as np
import pytest

import oracle
from tests.conftest import rel_l2


def kat_q4_0_raw():
    # wasm-q4.js:681-696: row 0 scale 1.0 (0x3C00), bytes 0x99 -> 32;
    #                     row 1 scale 2.0 (0x4000), bytes 0xAA -> 128.
    raw = np.zeros(36, np.uint8)
    raw[0], raw[1] = 0x00, 0x3C
    raw[2:18] = 0x99
    raw[18], raw[19] = 0x00, 0x40
    raw[20:36] = 0xAA
    return raw


def test_reference_q4_kat_all_restatements():
    x = np.ones(32, np.float32)
    raw = kat_q4_0_raw()
    for fn in (oracle.q4_0_matvec_js, oracle.q4_0_matvec_wasm, oracle.q4_0_matvec_cpu_sse):
        out = fn(x, raw, 2, 32)
        assert abs(out[0] - 32.0) < 0.1 and abs(out[1] - 128.0) < 0.1, (fn.__name__, out)
        # exact, in fact: small integers times powers of two
        assert out[0] == 32.0 and out[1] == 128.0


def test_reference_f32_matmul_kats():
    # wasm-simd.js:367-385
    A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    B = np.zeros((3, 5), np.float32)
    B[0, 0] = B[1, 1] = B[2, 2] = 1
    C = oracle.matmul_f32_axpy(A, B)
    np.testing.assert_allclose(C.ravel(), [1, 2, 3, 0, 0, 4, 5, 6, 0, 0], atol=1e-5)
    # main.js:65-74
    B2 = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    np.testing.assert_allclose(oracle.matmul_f32_axpy(A, B2).ravel(), [58, 64, 139, 154], atol=1e-3)
    # and the bias initialisation of matmulCached (wasm-simd.js:486-494)
    C3 = oracle.matmul_f32_axpy(A, B2, bias=np.array([1, -1], np.float32))
    np.testing.assert_allclose(C3.ravel(), [59, 63, 140, 153], atol=1e-3)


def test_f16_all_patterns_match_ieee():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_wasm_variant_divergences():
    # wasm-q4.js:88-109 flushes exp==0 to +0 and maps exp==31 to a finite value.
    bits = np.arange(65536, dtype=np.uint16)
    ieee = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32_wasm(int(b)) for b in bits], np.float32)
    exp = (bits >> 10) & 0x1F
    normal = (exp > 0) & (exp < 31)
    assert np.array_equal(got[normal].view(np.uint32), ieee[normal].view(np.uint32))
    assert np.all(got[exp == 0] == 0.0)
    e31 = exp == 31
    frac = (bits[e31] & 0x3FF).astype(np.float64)
    sign = np.where(bits[e31] >> 15, -1.0, 1.0)
    np.testing.assert_array_equal(got[e31], (sign * 65536.0 * (1 + frac / 1024)).astype(np.float32))


def test_f64_to_f16_matches_numpy():
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.uniform(0, 1, 4000), rng.uniform(0, 70000, 2000), 10.0 ** rng.uniform(-9, 5, 4000),
        -rng.uniform(0, 10, 1000),
        # exact ties between adjacent halves: 1 + (2k+1)/2048
        1.0 + (2 * np.arange(50) + 1) / 2048.0,
        # ties on the subnormal grid
        (2 * np.arange(50) + 1) * 2.0 ** -25,
        [0.0, 65504.0, 65519.99, 65520.0, 6.103515625e-05, 5.960464477539063e-08],
    ])
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f64_to_f16(v) for v in vals], np.uint16)
    assert np.array_equal(got, ref)


def test_dequant_nibble_order_three_restatements_agree():
    """gguf.js:259-286 (dequant), llama-streaming.js:72-104 (JS matvec) and
    wasm-q4.js:118-267 (WASM matvec) are independent reference codes; with
    x = e_k the two matvecs must return column k of the dequantised matrix."""
    rng = np.random.default_rng(1)
    N, K = 3, 64
    raw = rng.integers(0, 256, N * (K // 32) * 18, dtype=np.uint8)
    for b in range(N * K // 32):  # sane scales (the WASM form flushes subnormals)
        raw[b * 18:b * 18 + 2] = np.frombuffer(np.float16(rng.uniform(0.01, 2)).tobytes(), np.uint8)
    W = oracle.dequant_q4_0(raw, N * K).reshape(N, K)
    for k in range(K):
        e = np.zeros(K, np.float32)
        e[k] = 1
        assert np.array_equal(oracle.q4_0_matvec_js(e, raw, N, K), W[:, k])
        assert np.array_equal(oracle.q4_0_matvec_wasm(e, raw, N, K), W[:, k])
    # element 0 is the low nibble of byte 0, element 16 its high nibble
    d = np.frombuffer(raw[0:2].tobytes(), np.float16)[0].astype(np.float32)
    assert W[0, 0] == np.float32((int(raw[2]) & 15) - 8) * d
    assert W[0, 16] == np.float32((int(raw[2]) >> 4) - 8) * d


def test_dequant_every_byte_value():
    # all 256 qs byte values under one scale; dequant is exact (small int * fp16)
    raw = np.zeros(16 * 18, np.uint8)
    for blk in range(16):
        raw[blk * 18:blk * 18 + 2] = np.frombuffer(np.float16(0.375).tobytes(), np.uint8)
        raw[blk * 18 + 2: blk * 18 + 18] = np.arange(16 * blk, 16 * blk + 16)
    W = oracle.dequant_q4_0(raw, 16 * 32).reshape(16, 32)
    for blk in range(16):
        for j in range(16):
            byte = 16 * blk + j
            assert W[blk, j] == ((byte & 15) - 8) * 0.375
            assert W[blk, j + 16] == ((byte >> 4) - 8) * 0.375
    # Q8_0: all int8 values
    raw8 = np.zeros(8 * 34, np.uint8)
    for blk in range(8):
        raw8[blk * 34:blk * 34 + 2] = np.frombuffer(np.float16(-1.5).tobytes(), np.uint8)
        raw8[blk * 34 + 2:blk * 34 + 34] = np.arange(32 * blk, 32 * blk + 32)
    W8 = oracle.dequant_q8_0(raw8, 256)
    assert np.array_equal(W8, np.arange(256).astype(np.uint8).view(np.int8).astype(np.float32) * -1.5)


def q8_0_from_q4_0(raw0):
    """Q4_0 blocks -> Q8_0 blocks with the same d and int8 codes nibble - 8
    (gguf.js:239-286: both decode to code * d)."""
    b0 = raw0.reshape(-1, 18)
    b8 = np.zeros((b0.shape[0], 34), np.uint8)
    b8[:, :2] = b0[:, :2]
    lo = (b0[:, 2:] & 15).astype(np.int16) - 8
    hi = (b0[:, 2:] >> 4).astype(np.int16) - 8
    b8[:, 2:18] = lo.astype(np.int8).view(np.uint8)
    b8[:, 18:34] = hi.astype(np.int8).view(np.uint8)
    return b8.ravel()


def numpy_dequant_q8_0(raw, N, K):
    """gguf.js:239-257 written independently of the oracle: int8 * fp16 d."""
    blk = raw.reshape(N * K // 32, 34)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32)
    q = blk[:, 2:].copy().view(np.int8).astype(np.float32)
    return (q * d).reshape(N, K)


def test_q8_0_matvec_reference_kat_reencoded():
    """The Q4_0 KAT of wasm-q4.js:673-704 re-encoded as Q8_0 blocks (d = 1
    with int8 1s, d = 2 with int8 2s) must give exactly [32, 128] through the
    Q8_0 checker of every Q8_0 GPU matvec and GEMM test."""
    raw8 = q8_0_from_q4_0(kat_q4_0_raw())
    assert np.array_equal(raw8.reshape(2, 34)[0, 2:].view(np.int8), np.ones(32, np.int8))
    assert np.array_equal(raw8.reshape(2, 34)[1, 2:].view(np.int8), np.full(32, 2, np.int8))
    out = oracle.q8_0_matvec(np.ones(32, np.float32), raw8, 2, 32)
    assert out[0] == 32.0 and out[1] == 128.0


def test_q8_0_matvec_columns_and_exact_product():
    """x = e_k must return column k of the dequantised matrix (bit-exact),
    every int8 value and sign included; a general x must equal the exactly
    rounded dequantised product to within the final fp32 rounding.  A wrong
    block stride, an unsigned code or a per-row scale fails the first."""
    rng = np.random.default_rng(21)
    N, K = 5, 96
    raw = rng.integers(0, 256, N * (K // 32) * 34, dtype=np.uint8)
    for b in range(N * K // 32):
        raw[b * 34:b * 34 + 2] = np.frombuffer(
            np.float16(rng.uniform(-2, 2)).tobytes(), np.uint8)
    raw.reshape(-1, 34)[0, 2:34] = np.arange(-128, 128, 8).astype(np.int8).view(np.uint8)
    W = numpy_dequant_q8_0(raw, N, K)
    for k in range(K):
        e = np.zeros(K, np.float32)
        e[k] = 1
        assert np.array_equal(oracle.q8_0_matvec(e, raw, N, K), W[:, k]), k
    import math
    x = rng.normal(0, 1, K).astype(np.float32)
    out = oracle.q8_0_matvec(x, raw, N, K)
    for n in range(N):
        exact = math.fsum(float(W[n, k]) * float(x[k]) for k in range(K))
        assert abs(float(out[n]) - exact) <= abs(exact) * 2.0 ** -23 + 1e-30, (n, out[n], exact)
    # agrees with the Q4_0 checker on blocks both formats can hold
    raw4 = oracle.quantize_q4_0(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    x = rng.normal(0, 1, K).astype(np.float32)
    assert rel_l2(oracle.q8_0_matvec(x, q8_0_from_q4_0(raw4), N, K),
                  oracle.q4_0_matvec_js(x, raw4, N, K)) < 1e-12


def test_dequant_partial_last_block():
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, 2 * 18, dtype=np.uint8)
    raw[0:2] = raw[18:20] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    full = oracle.dequant_q4_0(raw, 64)
    part = oracle.dequant_q4_0(raw, 40)  # second block truncated to 8 values
    assert np.array_equal(part, full[:40])


def test_matvec_restatements_agree_and_are_linear():
    rng = np.random.default_rng(5)
    N, K = 37, 288
    raw = oracle.quantize_q4_0(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    x1 = rng.normal(0, 1, K).astype(np.float32)
    x2 = rng.normal(0, 1, K).astype(np.float32)
    js = oracle.q4_0_matvec_js(x1, raw, N, K)
    wasm = oracle.q4_0_matvec_wasm(x1, raw, N, K)
    W = oracle.dequant_q4_0(raw, N * K).reshape(N, K).astype(np.float64)
    exact = W @ x1.astype(np.float64)
    assert rel_l2(js, exact) < 1e-7
    assert rel_l2(wasm, exact) < 1e-5
    # linearity in x
    lin = oracle.q4_0_matvec_js(x1 + 2 * x2, raw, N, K)
    assert rel_l2(lin, js + 2 * oracle.q4_0_matvec_js(x2, raw, N, K)) < 1e-6
    # the SSE restatement timed as the CPU baseline is bit-identical to the f32 replay
    assert np.array_equal(oracle.q4_0_matvec_cpu_sse(x1, raw, N, K), wasm)


def q4_1_from_q4_0(raw0):
    """Q4_0 blocks -> Q4_1 blocks with the same d and m = -8d (exact in fp16
    for these scales), which decode to the same values."""
    b0 = raw0.reshape(-1, 18)
    d = b0[:, :2].copy().view(np.float16)
    m = (d.astype(np.float64) * -8).astype(np.float16)
    assert np.array_equal(m.astype(np.float64), d.astype(np.float64) * -8)
    b1 = np.zeros((b0.shape[0], 20), np.uint8)
    b1[:, :2] = d.view(np.uint8)
    b1[:, 2:4] = m.view(np.uint8)
    b1[:, 4:] = b0[:, 2:]
    return b1.ravel()


def test_q4_1_reference_kat_through_q4_0_identity():
    """No KAT for Q4_1 in the reference; the Q4_0 KAT (wasm-q4.js:673-704)
    re-encoded as Q4_1 with m = -8d must give the same [32, 128]."""
    raw1 = q4_1_from_q4_0(kat_q4_0_raw())
    x = np.ones(32, np.float32)
    for fn in (oracle.q4_1_matvec_js, oracle.q4_1_matvec_wasm):
        out = fn(x, raw1, 2, 32)
        assert out[0] == 32.0 and out[1] == 128.0, (fn.__name__, out)
    assert np.array_equal(oracle.dequant_q4_1(raw1, 64), oracle.dequant_q4_0(kat_q4_0_raw(), 64))


def test_q4_1_matches_q4_0_on_equivalent_blocks():
    rng = np.random.default_rng(21)
    N, K = 41, 320
    raw0 = oracle.quantize_q4_0(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    raw1 = q4_1_from_q4_0(raw0)
    x = rng.normal(0, 1, K).astype(np.float32)
    assert np.array_equal(oracle.dequant_q4_1(raw1, N * K), oracle.dequant_q4_0(raw0, N * K))
    ref = oracle.q4_0_matvec_js(x, raw0, N, K)
    assert rel_l2(oracle.q4_1_matvec_js(x, raw1, N, K), ref) < 1e-12
    assert rel_l2(oracle.q4_1_matvec_wasm(x, raw1, N, K), ref) < 1e-5


def test_q4_1_dequant_every_byte_value():
    # gguf.js:288-314: lo(byte j) * d + m at j, hi(byte j) * d + m at j + 16
    raw = np.zeros(16 * 20, np.uint8).reshape(16, 20)
    raw[:, 0:2] = np.frombuffer(np.float16(0.375).tobytes(), np.uint8)
    raw[:, 2:4] = np.frombuffer(np.float16(-1.25).tobytes(), np.uint8)
    raw[:, 4:] = np.arange(256, dtype=np.uint8).reshape(16, 16)
    W = oracle.dequant_q4_1(raw.ravel(), 16 * 32).reshape(16, 32)
    for blk in range(16):
        for j in range(16):
            byte = 16 * blk + j
            assert W[blk, j] == (byte & 15) * 0.375 - 1.25
            assert W[blk, j + 16] == (byte >> 4) * 0.375 - 1.25
    # a short last block is truncated like Q4_0's
    assert np.array_equal(oracle.dequant_q4_1(raw.ravel(), 40), W.ravel()[:40])


def test_q4_1_constant_blocks_closed_form():
    """d = 0: every element is m, so the matvec is m * sum(x) per block."""
    rng = np.random.default_rng(8)
    K = 96
    raw = np.zeros((1, 3, 20), np.uint8)
    mins = [0.5, -3.0, 0.0078125]
    for b, mv in enumerate(mins):
        raw[0, b, 2:4] = np.frombuffer(np.float16(mv).tobytes(), np.uint8)
        raw[0, b, 4:] = rng.integers(0, 256, 16)  # ignored: d = 0
    x = rng.normal(0, 1, K).astype(np.float32)
    exact = sum(mv * x[32 * b:32 * b + 32].astype(np.float64).sum() for b, mv in enumerate(mins))
    assert abs(oracle.q4_1_matvec_js(x, raw.ravel(), 1, K)[0] - exact) <= 1e-6 * abs(exact)
    assert abs(oracle.q4_1_matvec_wasm(x, raw.ravel(), 1, K)[0] - exact) <= 1e-5 * abs(exact)


def test_q4_1_matvec_restatements_agree_and_are_linear():
    rng = np.random.default_rng(6)
    N, K = 37, 288
    raw = oracle.quantize_q4_1(rng.normal(0.01, 0.02, (N, K)).astype(np.float32))
    x1 = rng.normal(0, 1, K).astype(np.float32)
    x2 = rng.normal(0, 1, K).astype(np.float32)
    js = oracle.q4_1_matvec_js(x1, raw, N, K)
    W = oracle.dequant_q4_1(raw, N * K).reshape(N, K).astype(np.float64)
    exact = W @ x1.astype(np.float64)
    assert rel_l2(js, exact) < 1e-6   # the dequantised f32 weights round once
    assert rel_l2(oracle.q4_1_matvec_wasm(x1, raw, N, K), js) < 1e-5
    lin = oracle.q4_1_matvec_js(x1 + 2 * x2, raw, N, K)
    assert rel_l2(lin, js + 2 * oracle.q4_1_matvec_js(x2, raw, N, K)) < 1e-6


def q6k_block(d=1.0, scales=None, ql=None, qh=None):
    blk = np.zeros(210, np.uint8)
    if ql is not None:
        blk[:128] = ql
    if qh is not None:
        blk[128:192] = qh
    blk[192:208] = (np.ones(16, np.int8) if scales is None else np.asarray(scales, np.int8)).view(np.uint8)
    blk[208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    return blk


def test_q6_k_dequant_known_positions():
    """gguf.js:317-364 by single-byte probes: with every code at its zero
    point (ql = 0, qh = 0 gives q = -32) a probe byte moves exactly the
    elements the layout names, by the amount it names."""
    base = oracle.dequant_q6_k(q6k_block(), 256)
    assert np.all(base == -32.0)
    cases = [  # (array, index, value) -> {element: code}
        ("ql", 5, 0x0F, {5: 15}),            # low nibble of ql[l]      -> l
        ("ql", 37, 0x0F, {37: 15}),          # low nibble of ql[l + 32] -> l + 32
        ("ql", 5, 0xF0, {69: 15}),           # high nibble of ql[l]     -> l + 64
        ("ql", 37, 0xA0, {101: 10}),         # high nibble of ql[l+32]  -> l + 96
        ("ql", 64 + 3, 0x01, {131: 1}),      # second half: + 128
        ("qh", 7, 0b11100100, {7: 0, 39: 16, 71: 32, 103: 48}),  # 2-bit fields 0..3
        ("qh", 32 + 31, 0b00000011, {159: 48}),
    ]
    for arr, idx, val, want in cases:
        ql = np.zeros(128, np.uint8)
        qh = np.zeros(64, np.uint8)
        (ql if arr == "ql" else qh)[idx] = val
        out = oracle.dequant_q6_k(q6k_block(ql=ql, qh=qh), 256)
        exp = np.full(256, -32.0, np.float32)
        for e, code in want.items():
            exp[e] = code - 32
        assert np.array_equal(out, exp), (arr, idx, np.nonzero(out != exp))


def test_q6_k_dequant_scales_and_d():
    # element e uses int8 scale e // 16 (is = 8*half + l/16, + 2 per group)
    scales = np.arange(-8, 8, dtype=np.int8) * 3
    out = oracle.dequant_q6_k(q6k_block(d=0.5, scales=scales), 256)
    exp = np.repeat(scales.astype(np.float64), 16) * 0.5 * -32
    assert np.array_equal(out, exp.astype(np.float32))
    # subnormal d, the largest |scale| and the top code: exact in f32
    ql = np.full(128, 0xFF, np.uint8)
    qh = np.full(64, 0xFF, np.uint8)
    out = oracle.dequant_q6_k(q6k_block(d=2.0 ** -20, scales=[-128] * 16, ql=ql, qh=qh), 256)
    assert np.all(out == np.float32(2.0 ** -20 * -128 * 31))
    # a short last block is truncated
    blk = np.concatenate([q6k_block(scales=scales), q6k_block(d=2.0)])
    assert np.array_equal(oracle.dequant_q6_k(blk, 300), oracle.dequant_q6_k(blk, 512)[:300])


def test_f16_dequant_all_patterns():
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.dequant_f16(bits.view(np.uint8), 65536)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_q6_k_quantizer_invariants():
    rng = np.random.default_rng(17)
    w = rng.normal(0, 0.02, (4, 512)).astype(np.float32)
    w[1, :256] = 0
    raw = oracle.quantize_q6_k(w)
    W = oracle.dequant_q6_k(raw, w.size).reshape(-1, 256)
    blocks = w.reshape(-1, 256).astype(np.float64)
    assert np.all(W[2] == 0)   # row 1, block 0: all zero
    d = raw.reshape(-1, 210)[:, 208:210].copy().view(np.float16).astype(np.float64).ravel()
    sc = raw.reshape(-1, 210)[:, 192:208].view(np.int8).astype(np.float64)
    step = d[:, None] * sc                      # per 16-element sub-block
    err = np.abs(W.astype(np.float64) - blocks).reshape(-1, 16, 16)
    # half a step, plus the edge where x / step rounds past 31 (<= one step)
    assert np.all(err <= step[:, :, None] * 1.0 + 1e-12)
    assert np.mean(err <= step[:, :, None] * 0.5 + 1e-12) > 0.99
    # quantise -> dequantise is close in L2
    assert rel_l2(W.ravel(), blocks.ravel()) < 0.05


def test_cpu_pool_partition_matches_single_thread():
    rng = np.random.default_rng(11)
    N, K = 1003, 256
    raw = oracle.quantize_q4_0(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    x = rng.normal(0, 1, K).astype(np.float32)
    ref = oracle.q4_0_matvec_wasm(x, raw, N, K)
    for t in (1, 2, 3, 8):
        pool = oracle.CpuPool(t)
        assert np.array_equal(pool.q4_0_matvec(x, raw, N, K), ref)
        pool.close()


def test_lm_head_restatements():
    rng = np.random.default_rng(2)
    V, D = 2100, 36   # D % 4 != 0 exercises the scalar tail
    E = rng.normal(0, 0.02, (V, D)).astype(np.float32)
    h = rng.normal(0, 1, D).astype(np.float32)
    wasm = oracle.batch_dot_wasm(h, E)
    assert np.array_equal(oracle.cpu_lm_head(h, E, V, D), wasm)
    assert rel_l2(wasm, E.astype(np.float64) @ h) < 1e-6
    assert rel_l2(oracle.f32_matvec(h, E), E.astype(np.float64) @ h) < 1e-7


def test_q8_ref_quantizer_math_round_ties():
    # maxAbs = 127 -> invScale = 1: values land exactly on .5 ties;
    # ECMAScript Math.round sends ties toward +infinity.
    w = np.zeros(32, np.float32)
    w[0] = 127.0
    w[1:6] = [2.5, -2.5, 0.5, -0.5, -126.5]
    q, s = oracle.quantize_q8_ref(w)
    assert s[0] == np.float32(1.0)
    assert list(q[:6]) == [127, 3, -2, 1, 0, -126]


def test_q8_quantizer_invariants():
    rng = np.random.default_rng(9)
    w = rng.normal(0, 0.02, (16, 256)).astype(np.float32)
    w[3, 32:64] = 0  # an all-zero block
    raw = oracle.quantize_q8_0(w).reshape(-1, 34)
    d = raw[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    q = raw[:, 2:].view(np.int8)
    blocks = w.reshape(-1, 32)
    amax = np.abs(blocks).max(1)
    assert np.all(np.abs(q.astype(int)) <= 127)
    nz = amax > 0
    # the absmax element maps to +-127
    idx = np.abs(blocks).argmax(1)
    assert np.all(np.abs(q[np.arange(len(q)), idx][nz].astype(int)) == 127)
    assert np.all(q[~nz] == 0) and np.all(d[~nz] == 0)
    # d = fp16(absmax/127)
    assert np.array_equal(d[nz], (amax[nz].astype(np.float64) / 127).astype(np.float16).astype(np.float32))
    # reconstruction error bounded by half a quantisation step (plus fp16 scale error)
    err = np.abs(q.astype(np.float64) * d[:, None] - blocks)
    assert np.all(err <= (amax / 127 * 0.5 + amax * 1e-3)[:, None] + 1e-12)


def test_q4_quantizer_invariants():
    rng = np.random.default_rng(10)
    w = rng.normal(0, 0.02, (8, 128)).astype(np.float32)
    w[0, :32] = 0
    raw = oracle.quantize_q4_0(w).reshape(-1, 18)
    d = raw[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    W = oracle.dequant_q4_0(raw.ravel(), w.size).reshape(-1, 32)
    blocks = w.reshape(-1, 32)
    amax = np.abs(blocks).max(1)
    assert d[0] == 0 and np.all(W[0] == 0)
    nib_lo = raw[:, 2:] & 15
    nib_hi = raw[:, 2:] >> 4
    assert nib_lo.max() <= 15 and nib_hi.max() <= 15
    assert np.array_equal(d[1:], (amax[1:].astype(np.float64) / 8).astype(np.float16).astype(np.float32))
    # |x - w| <= d/2 (+ fp16 rounding of d), except at the clamped +8 edge (<= d)
    err = np.abs(W - blocks)
    bound = np.broadcast_to((amax / 8)[:, None] * (0.5 + 2e-3) + 8 * np.abs(d - amax / 8)[:, None],
                            err.shape)
    clamped = blocks * (8 / np.where(amax > 0, amax, 1))[:, None] > 7.5
    assert np.all(err[~clamped] <= bound[~clamped] + 1e-9)
    assert np.all(err[clamped] <= 2 * bound[clamped] + 1e-9)


def test_q4_1_quantizer_invariants():
    rng = np.random.default_rng(13)
    w = rng.normal(0.01, 0.02, (8, 128)).astype(np.float32)
    w[0, :32] = 0.25  # a constant block
    raw = oracle.quantize_q4_1(w).reshape(-1, 20)
    d = raw[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    m = raw[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
    blocks = w.reshape(-1, 32).astype(np.float64)
    lo, hi = blocks.min(1), blocks.max(1)
    assert d[0] == 0 and m[0] == 0.25
    assert np.array_equal(d, ((hi - lo) / 15).astype(np.float16).astype(np.float64))
    assert np.array_equal(m, lo.astype(np.float16).astype(np.float64))
    W = oracle.dequant_q4_1(raw.ravel(), w.size).reshape(-1, 32)
    assert np.all(W[0] == 0.25)
    # |x - w| <= d/2 plus the fp16 rounding of d (x15) and of m
    err = np.abs(W - blocks)
    bound = d / 2 + 15 * np.abs(d - (hi - lo) / 15) + np.abs(m - lo) + 1e-9
    assert np.all(err <= bound[:, None] * (1 + 1e-6))


def test_matmul_q8_ref_matches_dequantised_product():
    rng = np.random.default_rng(4)
    K, N, M = 64, 96, 3
    w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
    q, s = oracle.quantize_q8_ref(w)
    A = rng.normal(0, 1, (M, K)).astype(np.float32)
    A[1, 5] = 0.0   # the skipped-zero branch (quantize.js:248)
    bias = rng.normal(0, 1, N).astype(np.float32)
    out = oracle.matmul_q8_ref(A, q, s, N, bias)
    Wd = oracle.dequant_q8_ref(q, s).reshape(K, N).astype(np.float64)
    ref = A.astype(np.float64) @ Wd + bias
    assert rel_l2(out, ref) < 1e-6


def test_product_and_oracle_quantisers_agree():
    """The product's host quantisers (pbx_quantize_*) and the oracle's are
    written independently; their bytes must be identical."""
    import purebee_amd as pb
    rng = np.random.default_rng(12)
    w = rng.normal(0, 0.02, (33, 576)).astype(np.float32)
    w[0, :32] = 0
    assert np.array_equal(pb.quantize_q8_0(w), oracle.quantize_q8_0(w))
    assert np.array_equal(pb.quantize_q4_0(w), oracle.quantize_q4_0(w))
    assert np.array_equal(pb.quantize_q4_1(w), oracle.quantize_q4_1(w))
    w6 = rng.normal(0, 0.02, (5, 512)).astype(np.float32)
    w6[2, :256] = 0
    assert np.array_equal(pb.quantize_q6_k(w6), oracle.quantize_q6_k(w6))
    q1, s1 = pb.quantize_q8_ref(w)
    q2, s2 = oracle.quantize_q8_ref(w)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


def test_synth_generator_product_matches_oracle():
    import purebee_amd as pb
    a = pb.synth_normal(1234, 100001, 0.0, 0.02)
    b = oracle.synth_normal(1234, 100001, 0.0, 0.02)
    assert np.array_equal(a, b)
    z = pb.synth_normal(99, 400000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert not np.array_equal(pb.synth_normal(1, 64), pb.synth_normal(2, 64))
