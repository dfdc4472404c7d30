"""Pins the CPU GEMV/GEMM oracle (oracle/er_oracle.c) without retyping it:
float64 accumulation of independently dequantised weights, one-hot x
extracting a dequantised column exactly, linearity, batched == per token,
and the reference's own test cases (GEMVTests.swift:459-734)."""
import numpy as np
import pytest

from oracle import ref
from oracle import restate_np as rn
from conftest import rel_l2

import edgerunner_amd.synth as synth

FMTS = ["q8_0", "q4_k", "q6_k"]


def _w(fmt, M, K, seed=11):
    return synth.weights(fmt, synth.seed(seed, 0), M, K)


@pytest.mark.parametrize("fmt", FMTS)
def test_gemv_matches_float64(fmt):
    M, K = 33, 1024
    W = _w(fmt, M, K)
    x = synth.normal_f32(synth.seed(11, 1), K)
    y = ref.gemv(fmt, W, x, M, K)
    y64 = rn.gemv_f64(fmt, W, x, M, K).ravel()
    assert rel_l2(y, y64) < 1e-6


@pytest.mark.parametrize("fmt", FMTS)
def test_gemv_one_hot_extracts_column(fmt):
    M, K = 17, 512
    W = _w(fmt, M, K)
    Wd = rn.weights_f32(fmt, W, M, K)
    for j in (0, 1, 31, 32, 255, 256, 300, 511):
        x = np.zeros(K, np.float32)
        x[j] = 1.0
        y = ref.gemv(fmt, W, x, M, K)
        assert np.array_equal(y, Wd[:, j]), j


@pytest.mark.parametrize("fmt", FMTS)
def test_gemv_linearity(fmt):
    M, K = 9, 768
    W = _w(fmt, M, K)
    a = synth.normal_f32(1, K)
    b = synth.normal_f32(2, K)
    ya, yb = ref.gemv(fmt, W, a, M, K), ref.gemv(fmt, W, b, M, K)
    yab = ref.gemv(fmt, W, 2.0 * a - 0.5 * b, M, K)
    assert rel_l2(yab, 2.0 * ya - 0.5 * yb) < 1e-5


@pytest.mark.parametrize("fmt", FMTS)
def test_batched_equals_per_token(fmt):
    M, K, T = 7, 512, 3
    W = _w(fmt, M, K)
    x = ((np.arange(T * K) % 37) - 18) / 23.0
    yb = ref.gemv(fmt, W, x.astype(np.float32), M, K, tokens=T).reshape(T, M)
    for t in range(T):
        assert np.array_equal(yb[t], ref.gemv(fmt, W, x[t * K:(t + 1) * K].astype(np.float32), M, K))


def test_threaded_equals_serial():
    M, K = 64, 1024
    W = _w("q4_k", M, K)
    x = synth.normal_f32(3, K)
    assert np.array_equal(ref.gemv("q4_k", W, x, M, K, threads=1),
                          ref.gemv("q4_k", W, x, M, K, threads=4))


def test_reference_cases_against_float64():
    # GEMVTests.swift:459-478, 556-575, 624-660 (formula fillers + x formulas)
    cases = [
        ("q4_k", ref.make_q4k_weights(9, 512), 9, 512, ((np.arange(512) % 17) - 8) / 19.0),
        ("q6_k", ref.make_q6k_weights(7, 512), 7, 512, ((np.arange(512) % 23) - 11) / 29.0),
        ("q6_k", ref.make_q6k_weights(9, 768), 9, 768, ((np.arange(768) % 23) - 11) / 29.0),
    ]
    for fmt, W, M, K, x in cases:
        y = ref.gemv(fmt, W, x.astype(np.float32), M, K)
        y64 = rn.gemv_f64(fmt, W, x.astype(np.float32), M, K).ravel()
        assert np.max(np.abs(y - y64)) < 1e-4


def test_gemm_oracle_is_per_token_gemv_on_bf16():
    T, N, K = 5, 12, 512
    W = _w("q4_k", N, K)
    X = synth.normal_bf16(5, T * K)
    Y = ref.gemm("q4_k", W, X, T, N, K)
    Xf = (X.astype(np.uint32) << 16).view(np.float32)
    for t in range(T):
        assert np.array_equal(Y[t], ref.gemv("q4_k", W, Xf[t * K:(t + 1) * K], N, K))


def test_argmax_lowest_index_ties():
    v = np.array([1, 5, 3, 5, 5, -1], np.float32)
    assert ref.argmax(v) == 1
    rng = np.random.default_rng(3)
    for _ in range(20):
        v = rng.integers(0, 4, size=50).astype(np.float32)
        assert ref.argmax(v) == int(np.argmax(v))


def test_quantize_q8_0_rows_closed_forms():
    rows, bpr = 3, 4
    src = synth.normal_f32(9, rows * bpr * 32)
    src[32:64] = 0.0                       # a zero block
    dst = ref.quantize_q8_0_rows(src, rows, bpr * 32, 0, bpr)
    blk = dst.reshape(-1, 34)
    q = blk[:, 2:].view(np.int8).astype(np.int32)
    v = src.reshape(-1, 32)
    for b in range(blk.shape[0]):
        amax = np.max(np.abs(v[b]))
        if amax == 0:
            assert np.all(q[b] == 0) and blk[b, 0] == 0 and blk[b, 1] == 0
            continue
        i = int(np.argmax(np.abs(v[b])))
        assert abs(q[b, i]) == 127                       # max |v| maps to +-127
        assert np.all(np.abs(q[b]) <= 127)
        d = np.float32(amax) / np.float32(127)
        assert np.array_equal(q[b], np.clip(np.rint(v[b] / d), -127, 127).astype(np.int32))
        assert (blk[b, 0] | (blk[b, 1].astype(np.uint16) << 8)) == ref.f32_to_f16(float(d))
    # ties go to even: 0.5 * scale rounds to 0, 1.5 * scale to 2
    row = np.zeros(32, np.float32)
    row[0] = 127.0
    row[1] = 0.5
    row[2] = 1.5
    row[3] = -2.5
    q = ref.quantize_q8_0_rows(row, 1, 32, 0, 1)[2:6].view(np.int8)
    assert list(q) == [127, 0, 2, -2]


def test_gelu_tanh_oracle():
    """cpuGeluTanh (GEMVTests.swift:38-47): odd-part identity g(x) - g(-x) = x,
    saturation outside [-10, 10], and the tanh form's known distance (< 2e-3)
    from the exact x * Phi(x)."""
    import math
    xs = np.linspace(-9.5, 9.5, 381).astype(np.float32)
    g = ref.gelu_tanh(xs)
    gm = ref.gelu_tanh(-xs)
    assert np.allclose(g - gm, xs, atol=2e-6)
    exact = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in xs.astype(np.float64)])
    assert np.max(np.abs(g - exact)) < 2e-3
    big = np.array([10.5, 12.0, 1e4], np.float32)
    assert np.array_equal(ref.gelu_tanh(big), big)
    assert np.all(ref.gelu_tanh(-big) == 0.0)
    assert ref.gelu_tanh([0.0])[0] == 0.0


def test_top1_oracle_equals_argmax_on_finite_values():
    """The reference's two-stage top-1 (quad candidates, then a merge that
    prefers lower indices on ties) picks numpy's argmax (first maximum) for
    finite inputs, ties included."""
    rng = np.random.default_rng(7)
    for n in (4, 8, 12, 64, 1000, 4096):
        v = rng.standard_normal(n).astype(np.float32)
        assert ref.top1(v) == int(np.argmax(v))
        w = np.round(v * 2).astype(np.float32)  # many ties
        assert ref.top1(w) == int(np.argmax(w))
    v = np.zeros(16, np.float32)
    assert ref.top1(v) == 0
    v[[6, 9, 13]] = 3.0
    assert ref.top1(v) == 6


def test_top1_oracle_nan_and_infinity_rules():
    """Hand-derived from the kernels' comparisons: a NaN in a quad's first row
    makes the quad's candidate NaN, which never wins the merge; a NaN later in
    a quad is skipped; with every candidate -inf the merge keeps its start
    value (-inf, row 0)."""
    nan, inf = float("nan"), float("inf")
    assert ref.top1([nan, 9, 9, 9, 1, 2, 3, 0]) == 6     # quad 0 dropped
    assert ref.top1([1, nan, 5, 2, 0, 0, 0, 0]) == 2     # NaN skipped inside the quad
    assert ref.top1([nan] * 8) == 0
    assert ref.top1([-inf] * 8) == 0
    assert ref.top1([-inf, -inf, -inf, -inf, -inf, -5.0, -inf, -inf]) == 5
    assert ref.top1([0, 0, 0, 0, inf, 0, 0, inf]) == 4


def test_rmsnorm_oracle():
    """cpuRMSNorm (FusedKernelTests.swift:53-57): with w = 1 the output has
    unit RMS (eps small), scaling x does not change it, and a constant
    vector c maps to c / sqrt(c^2 + eps) * w exactly as fp32 evaluates it."""
    x = synth.normal_f32(11, 4096) * 3.0
    ones = np.ones(4096, np.float32)
    n = ref.rmsnorm(x, ones, 1e-6)
    assert abs(float(np.sqrt(np.mean(n.astype(np.float64) ** 2))) - 1.0) < 1e-5
    assert np.allclose(ref.rmsnorm(x * 8.0, ones, 0.0), ref.rmsnorm(x, ones, 0.0), rtol=1e-5, atol=1e-6)
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    c = np.full(64, 0.25, np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(0.0625) + np.float32(1e-5))
    assert np.array_equal(ref.rmsnorm(c, w, 1e-5), (c * scale * w).astype(np.float32))


def test_silu_oracle():
    """silu (FusedKernelTests.swift:85-87): odd-part identity, zero, limits."""
    xs = np.linspace(-20, 20, 401).astype(np.float32)
    s, sm = ref.silu(xs), ref.silu(-xs)
    assert np.allclose(s - sm, xs, atol=1e-5)
    assert ref.silu([0.0])[0] == 0.0
    assert abs(ref.silu([30.0])[0] - 30.0) < 1e-5 and abs(ref.silu([-30.0])[0]) < 1e-10
