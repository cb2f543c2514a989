"""Q4_0 block scales across the whole fp16 range through the M > 32 MFMA GEMM
(pbx_linear at M >= 4, llama-streaming.js:168-177 / engine.js:180-269
batched; the block format of gguf.js:259-286).  The kernel multiplies each
block's integer-code product by its fp16 scale in fp32, so fp16 subnormal
scales, tiny, typical and large ones must all come out as the oracle's
double-accumulated matvec.  Rows of every magnitude sit in one matrix and
each weight row's outputs (a column of Y) are compared on their own, so an
inexact small-scale row (a flushed subnormal, a lost low bit) cannot hide
behind the large ones: a column within 1e-4 relative L2 (a column of M
outputs carries more cancellation than a row of N; the fp32 accumulation
leaves ~1e-6), every row of Y within the usual 1e-5."""
import numpy as np
import pytest

import oracle
import purebee_amd as pb
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu

# per-row scale magnitudes: fp16 subnormals (2^-24 .. 2^-15), small normals,
# typical, large
SCALES = [3 * 2.0**-24, 2.0**-18, 2.0**-15 * 1.7, 6.2e-5, 1.3e-3, 0.0123, 0.5, 37.0, 999.0]


def q4_0_rows(seed, N, K, row_scale):
    """Q4_0 bytes (per block: fp16 d, then 16 bytes of nibble codes) with the
    block scales of row n drawn near row_scale(n)."""
    rng = np.random.default_rng(seed)
    B = K // 32
    raw = np.empty((N, B, 18), np.uint8)
    for n in range(N):
        d = (row_scale(n) * rng.uniform(0.5, 1.0, B)).astype(np.float16)
        raw[n, :, :2] = d.view(np.uint8).reshape(B, 2)
        raw[n, :, 2:] = rng.integers(0, 256, (B, 16), dtype=np.uint8)
    return raw.ravel()


def check(ctx, raw, N, K, M, seed):
    X = pb.synth_normal(seed, M * K).reshape(M, K)
    X[1] *= 1e-3
    X[2] *= 300.0
    w = ctx.upload(pb.TYPE_Q4_0, N, K, raw)
    Y = ctx.linear(w, X)
    w.free()
    ref = np.stack([oracle.matvec(pb.TYPE_Q4_0, X[m], raw, N, K) for m in range(M)])
    cols = max(rel_l2(Y[:, n], ref[:, n]) for n in range(N))
    rows = max(rel_l2(Y[m], ref[m]) for m in range(M))
    print(f"  worst column rel L2 {cols:.2e}, worst row {rows:.2e}", flush=True)
    assert cols < 1e-4
    assert rows < 1e-5


@pytest.mark.parametrize("M", [40, 130])
def test_q4_0_scale_range_per_weight_row(ctx, M):
    N, K = 288, 1024
    print(f"[case] q4_0 scale range M={M} N={N} K={K}", flush=True)
    check(ctx, q4_0_rows(M + 17, N, K, lambda n: SCALES[n % len(SCALES)]), N, K, M, 900 + M)


@pytest.mark.parametrize("top", [2.0**-20, 4094.0, 8000.0, 65504.0])
def test_q4_0_largest_scale(ctx, top):
    """Largest scale 2^-20 (every scale an fp16 subnormal) up to fp16's
    largest finite value; a row of each magnitude from top down to 2^-24."""
    N, K, M = 160, 512, 48
    print(f"[case] q4_0 largest scale {top}", flush=True)
    mags = [top * 2.0**-e for e in range(0, 40, 3)]
    raw = q4_0_rows(int(top) + 5, N, K, lambda n: max(mags[n % len(mags)], 2.0**-24))
    # row 0 holds the largest scale itself
    raw.reshape(N, K // 32, 18)[0, 0, :2] = np.array([top], np.float16).view(np.uint8)
    check(ctx, raw, N, K, M, 77)
