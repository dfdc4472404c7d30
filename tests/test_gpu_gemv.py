"""Decode GEMV parity: HIP kernels vs the CPU oracle (fp32, reference loop
order).  Bar: relative L2 <= 1e-3 (north star), plus the reference tests'
own absolute 1e-4 on their cases, and exact equality where the mathematics
fixes the answer (one-hot x returns a dequantised column)."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import (EncodingFailed, InvalidArgument, InvalidMatrixShape,
                            InvalidVectorShape, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0)
from oracle import ref
from oracle import restate_np as rn
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-3
EXEC = {"q8_0": "executeQ8_0Weights", "q4_k": "executeQ4KWeights", "q6_k": "executeQ6KWeights"}
EXEC_B = {"q8_0": "executeBatchedQ8_0Weights", "q4_k": "executeBatchedQ4KWeights",
          "q6_k": "executeBatchedQ6KWeights"}
DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01},
          "q6_k": {"dscale": 0.005}}


def run(gemv, fmt, W, x, M, K):
    return getattr(gemv, EXEC[fmt])(W, x, M, K)


# ---- the reference's own test cases (GEMVTests.swift:459-734) ---------------
def test_reference_q4k_case(gemv):
    M, K = 9, 512
    W = ref.make_q4k_weights(M, K)
    x = (((np.arange(K) % 17) - 8) / 19.0).astype(np.float32)
    y = gemv.executeQ4KWeights(W, x, M, K)
    exp = ref.gemv("q4_k", W, x, M, K)
    assert np.max(np.abs(y - exp)) < 1e-4 and rel_l2(y, exp) < TOL


def test_reference_batched_q4k_case(gemv):
    M, K, T = 7, 512, 3
    W = ref.make_q4k_weights(M, K)
    x = (((np.arange(T * K) % 37) - 18) / 23.0).astype(np.float32)
    yb = gemv.executeBatchedQ4KWeights(W, x, T, M, K).reshape(T, M)
    for t in range(T):
        xt = x[t * K:(t + 1) * K]
        single = gemv.executeQ4KWeights(W, xt, M, K)
        assert np.max(np.abs(yb[t] - single)) < 1e-5
        assert np.max(np.abs(yb[t] - ref.gemv("q4_k", W, xt, M, K))) < 2e-4


@pytest.mark.parametrize("M,K", [(7, 512), (9, 768)])
def test_reference_q6k_cases(gemv, M, K):
    W = ref.make_q6k_weights(M, K)
    x = (((np.arange(K) % 23) - 11) / 29.0).astype(np.float32)
    y = gemv.executeQ6KWeights(W, x, M, K)
    exp = ref.gemv("q6_k", W, x, M, K)
    assert np.max(np.abs(y - exp)) < 1e-4 and rel_l2(y, exp) < TOL


def test_reference_q8_0_case(gemv):
    # FusedKernelTests.swift:89-126 uses unseeded Float.random; seeded here
    rows, cols = 64, 128
    rng = np.random.default_rng(5)
    x = (rng.uniform(-1, 1, cols) * (np.arange(cols) + 1) / cols).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (rows, cols)).astype(np.float32)
    W = np.concatenate([ref.pack_block("q8_0", w.reshape(-1, 32)[i]) for i in range(rows * cols // 32)])
    y = gemv.executeQ8_0Weights(W, x, rows, cols)
    exp = ref.gemv("q8_0", W, x, rows, cols)
    rel = np.abs(y - exp) / np.maximum(np.abs(exp), 1e-6)
    assert np.all(rel < 0.02) and rel_l2(y, exp) < TOL


def test_encoded_gemvs_share_one_stream(ctx, gemv):
    # GEMVTests.swift:662-734: several encodes on one command buffer
    K = 512
    W4, W6 = ref.make_q4k_weights(5, K), ref.make_q6k_weights(4, K)
    x = (((np.arange(K) % 19) - 9) / 23.0).astype(np.float32)
    s = ctx.stream()
    wb4, wb6, xb = ctx.upload(W4), ctx.upload(W6), ctx.upload(x)
    y4, y6 = ctx.alloc(5 * 4), ctx.alloc(4 * 4)
    gemv.encodeQ4KWeights(s, wb4, xb, y4, 5, K)
    gemv.encodeQ6KWeights(s, wb6, xb, y6, 4, K)
    s.synchronize()
    assert np.max(np.abs(y4.download(np.float32) - ref.gemv("q4_k", W4, x, 5, K))) < 1e-4
    assert np.max(np.abs(y6.download(np.float32) - ref.gemv("q6_k", W6, x, 4, K))) < 1e-4
    s.destroy()


# ---- BASELINE shapes, full size ------------------------------------------
BASELINE = [
    ("q8_0", 3072, 1024, 1), ("q8_0", 14336, 4096, 1),
    ("q4_k", 14336, 4096, 2), ("q4_k", 4096, 14336, 2),
    ("q6_k", 151936, 1024, 3), ("q6_k", 128256, 4096, 3),
]


@pytest.mark.parametrize("fmt,M,K,cfg", BASELINE, ids=lambda v: str(v))
def test_baseline_shapes(gemv, fmt, M, K, cfg):
    W = synth.weights(fmt, synth.seed(cfg, 0), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(cfg, 1), K)
    y = run(gemv, fmt, W, x, M, K)
    exp = ref.gemv(fmt, W, x, M, K, threads=ref.max_threads())
    err = rel_l2(y, exp)
    print(f"{fmt} {M}x{K}: rel_l2 = {err:.3e}")
    assert err < TOL


# ---- shape edge cases (row tails, lane-group widths, x from global) --------
SHAPES = [(1, 256), (3, 256), (5, 512), (17, 768), (33, 1280), (100, 2048), (63, 3072),
          (129, 1024), (7, 6144), (11, 16384), (5, 16640), (3, 32768)]


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("M,K", SHAPES)
def test_shapes(gemv, fmt, M, K):
    W = synth.weights(fmt, synth.seed(30, M % 16), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(30, 1), K)
    y = run(gemv, fmt, W, x, M, K)
    assert rel_l2(y, ref.gemv(fmt, W, x, M, K)) < TOL


@pytest.mark.parametrize("M,K", [(5, 96), (9, 160), (4, 32)])
def test_q8_0_odd_block_rows(gemv, M, K):
    """K/32 odd: rows are only 2-byte aligned (generic Q8_0 kernel)."""
    W = synth.q8_0(synth.seed(31, 0), M, K)
    x = synth.normal_f32(synth.seed(31, 1), K)
    y = gemv.executeQ8_0Weights(W, x, M, K)
    assert rel_l2(y, ref.gemv("q8_0", W, x, M, K)) < TOL


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k"])
def test_one_hot_returns_dequantised_column_exactly(gemv, fmt):
    M, K = 50, 1024
    W = synth.weights(fmt, synth.seed(32, 0), M, K, **DSCALE[fmt])
    cols = rn.weights_f32(fmt, W, M, K)
    for j in (0, 1, 17, 31, 32, 100, 255, 256, 511, 640, 1023):
        x = np.zeros(K, np.float32)
        x[j] = 1.0
        y = run(gemv, fmt, W, x, M, K)
        # value equality: a -0.0 weight times 1 summed onto +0.0 gives +0.0
        assert np.array_equal(y, cols[:, j]), j


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("M,K,T", [(300, 1024, 5), (3072, 1024, 4), (2048, 1024, 8), (4096, 1024, 2)])
def test_batched_equals_per_token(gemv, fmt, M, K, T):
    """Batched rows equal per-token rows bit for bit, also at shapes where the
    batch changes the number of rows each lane group computes."""
    W = synth.weights(fmt, synth.seed(33, 0), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(33, 1), T * K)
    yb = getattr(gemv, EXEC_B[fmt])(W, x, T, M, K).reshape(T, M)
    for t in range(T):
        single = run(gemv, fmt, W, x[t * K:(t + 1) * K], M, K)
        assert np.array_equal(yb[t], single)
    exp = ref.gemv(fmt, W, x, M, K, tokens=T).reshape(T, M)
    assert rel_l2(yb, exp) < TOL


def test_linearity(gemv):
    M, K = 256, 2048
    W = synth.q4_k(synth.seed(34, 0), M, K)
    a, b = synth.normal_f32(1, K), synth.normal_f32(2, K)
    ya, yb = gemv.executeQ4KWeights(W, a, M, K), gemv.executeQ4KWeights(W, b, M, K)
    yab = gemv.executeQ4KWeights(W, (2 * a - 0.5 * b).astype(np.float32), M, K)
    assert rel_l2(yab, 2 * ya - 0.5 * yb) < 1e-5


def test_projection_dispatch(ctx, gemv):
    """encodeProjection picks the kernel from the tensor's data type and honours byteOffset."""
    M, K = 64, 512
    x = synth.normal_f32(35, K)
    xb = ctx.upload(x)
    for dtype, fmt in ((TYPE_Q8_0, "q8_0"), (TYPE_Q4_K, "q4_k"), (TYPE_Q6_K, "q6_k")):
        W = synth.weights(fmt, synth.seed(35, dtype), M, K, **DSCALE[fmt])
        pad = 256
        buf = ctx.upload(np.concatenate([np.zeros(pad, np.uint8), W]))
        y = ctx.alloc(M * 4)
        gemv.encodeProjection(None, buf, dtype, xb, y, M, K, byteOffset=pad)
        ctx.synchronize()
        assert rel_l2(y.download(np.float32), ref.gemv(fmt, W, x, M, K)) < TOL


def test_validation_errors(ctx, gemv):
    K, M = 512, 4
    W = ref.make_q4k_weights(M, K)
    x = np.zeros(K, np.float32)
    with pytest.raises(InvalidVectorShape):
        gemv.executeQ4KWeights(W, x[:-1], M, K)
    with pytest.raises(InvalidVectorShape):
        gemv.executeQ4KWeights(W, np.zeros(K + 128, np.float32), M, K + 128)
    with pytest.raises(InvalidMatrixShape):
        gemv.executeQ4KWeights(W[:-1], x, M, K)
    wb, xb, yb = ctx.upload(W), ctx.upload(x), ctx.alloc(M * 4 - 4)
    with pytest.raises(EncodingFailed):
        gemv.encodeQ4KWeights(None, wb, xb, yb, M, K)
    with pytest.raises(InvalidArgument):
        gemv.encodeQ4KWeights(None, wb.view(4, wb.length - 4), xb, ctx.alloc(M * 4), M - 1, K)
    # M = 0 is a no-op
    gemv.encodeQ4KWeights(None, wb, xb, ctx.alloc(4), 0, K)
    ctx.synchronize()
