"""CU-resident GEMV family (K % 256 == 0; Q4_K rows up to 16384 weights, Q8_0
and Q6_K rows up to 4096, longer rows of those fall back to the lane-group
family; Q6_K rows of 4096 < K <= 16384 run here on the default dispatch, whose
K-sliced CU-resident kernels take them):
the GEMV parity bar of the other kernels (relative L2 <= 1e-3 against the CPU
oracle, the reference test's absolute 1e-4 on its case, exact one-hot
columns, batched equal to per-token) with the family forced on for every
shape it covers, through a context created with ER_HIP_GEMV_CU=1.  The
shapes reach every configuration (16/32/64 lanes per row, one or two slots
per lane), workgroups with no rows (M below the CU count) and partial last
steps."""
import os

import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import Context, GEMVKernel
from oracle import ref
from oracle import restate_np as rn
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-3
DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01},
          "q6_k": {"dscale": 0.005}}
EXEC = {"q8_0": "executeQ8_0Weights", "q4_k": "executeQ4KWeights", "q6_k": "executeQ6KWeights"}
EXEC_B = {"q8_0": "executeBatchedQ8_0Weights", "q4_k": "executeBatchedQ4KWeights",
          "q6_k": "executeBatchedQ6KWeights"}
FMTS = ["q4_k", "q8_0", "q6_k"]


def _context(mode: str) -> Context:
    old = os.environ.get("ER_HIP_GEMV_CU")
    os.environ["ER_HIP_GEMV_CU"] = mode
    try:
        return Context(int(os.environ.get("ER_DEVICE", "0")))
    finally:
        if old is None:
            os.environ.pop("ER_HIP_GEMV_CU", None)
        else:
            os.environ["ER_HIP_GEMV_CU"] = old


@pytest.fixture(scope="module")
def cu_gemv():
    c = _context("1")
    yield GEMVKernel(c)
    c.close()


# K -> configuration picked (lanes per row x slots per lane): 256 -> 16x1,
# 1024 -> 16x1, 2048 -> 32x1, 3072 -> 64x1, 4096 -> 64x1, 1536 -> 32x1
# (24 slots); Q4_K 5120 -> 64x2, 8192 -> 64x2, 12288 -> 64x3, 14336 -> 32x7,
# 16384 -> 64x4 (one or two row steps per CU)
SHAPES = [(1, 256), (7, 1024), (100, 2048), (333, 3072), (1000, 4096), (64, 5120), (250, 1536),
          (513, 8192), (14336, 4096), (64, 12288), (100, 14336), (4096, 14336), (2048, 16384)]
# more than 8 row steps per CU (rolled kernel): 28672 x 4096 (14 steps),
# 151936 x 1024 (19 steps of 32 rows), 140000 x 256 (capped at 64 steps, more
# workgroups than CUs)
ROLLED = [(28672, 4096), (151936, 1024), (140000, 256)]


def _family(cu_gemv, gemv, fmt, K):
    """The forced whole-row family, or for Q6_K rows beyond 4096 weights (which
    it does not cover) the default dispatch's K-sliced kernels."""
    return gemv if fmt == "q6_k" and K > 4096 else cu_gemv


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,K", SHAPES)
def test_cu_family_matches_oracle(cu_gemv, gemv, fmt, M, K):
    W = synth.weights(fmt, synth.seed(80, M % 97), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(80, 200 + K % 89), K)
    y = getattr(_family(cu_gemv, gemv, fmt, K), EXEC[fmt])(W, x, M, K)
    exp = ref.gemv(fmt, W, x, M, K, threads=ref.max_threads())
    assert rel_l2(y, exp) < TOL


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,K", ROLLED)
def test_cu_family_rolled_matches_oracle(cu_gemv, fmt, M, K):
    W = synth.weights(fmt, synth.seed(85, M % 97), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(85, 200 + K % 89), K)
    y = getattr(cu_gemv, EXEC[fmt])(W, x, M, K)
    exp = ref.gemv(fmt, W, x, M, K, threads=ref.max_threads())
    assert rel_l2(y, exp) < TOL


def test_cu_family_reference_q4k_case(cu_gemv):
    """GEMVTests.swift's Q4_K case (M 9, K 512) to its absolute bound 1e-4."""
    M, K = 9, 512
    W = ref.make_q4k_weights(M, K)
    x = (((np.arange(K) % 17) - 8) / 19.0).astype(np.float32)
    y = cu_gemv.executeQ4KWeights(W, x, M, K)
    exp = ref.gemv("q4_k", W, x, M, K)
    assert np.max(np.abs(y - exp)) < 1e-4 and rel_l2(y, exp) < TOL


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("K", [1024, 4096, 8192])
def test_cu_family_one_hot_columns(cu_gemv, gemv, fmt, K):
    cu_gemv = _family(cu_gemv, gemv, fmt, K)
    M = 40
    W = synth.weights(fmt, synth.seed(81, 0), M, K, **DSCALE[fmt])
    cols = rn.weights_f32(fmt, W, M, K)
    for j in (0, 1, 31, 32, 255, 256, K // 2 + 3, K - 1):
        x = np.zeros(K, np.float32)
        x[j] = 1.0
        y = getattr(cu_gemv, EXEC[fmt])(W, x, M, K)
        assert np.array_equal(y, cols[:, j]), j


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,K,T", [(300, 1024, 5), (1000, 4096, 3), (77, 8192, 2)])
def test_cu_family_batched_equals_per_token(cu_gemv, gemv, fmt, M, K, T):
    cu_gemv = _family(cu_gemv, gemv, fmt, K)
    W = synth.weights(fmt, synth.seed(82, 0), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(82, 1), T * K)
    yb = getattr(cu_gemv, EXEC_B[fmt])(W, x, T, M, K).reshape(T, M)
    for t in range(T):
        single = getattr(cu_gemv, EXEC[fmt])(W, x[t * K:(t + 1) * K], M, K)
        assert np.array_equal(yb[t], single)


@pytest.mark.parametrize("fmt", FMTS)
def test_cu_family_equals_lane_matched_family1(cu_gemv, fmt):
    """At 64 lanes x 1 slot both families form each row's sum the same way
    (slot dot, then the 64-lane reduction), so they agree bit for bit."""
    M, K = 4096, 4096
    W = synth.weights(fmt, synth.seed(83, 0), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(83, 1), K)
    c0 = _context("0")
    try:
        y0 = getattr(GEMVKernel(c0), EXEC[fmt])(W, x, M, K)
    finally:
        c0.close()
    y1 = getattr(cu_gemv, EXEC[fmt])(W, x, M, K)
    assert np.array_equal(y0, y1)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,K,T", [(12288, 2048, 3), (24576, 1024, 2), (6144, 4096, 4)])
def test_default_dispatch_batched_equals_per_token(gemv, fmt, M, K, T):
    """Default dispatch on shapes the CU-resident family takes: the family is
    chosen from M and K alone, so batched and per-token calls agree bit for
    bit although the batch changes the row partition."""
    W = synth.weights(fmt, synth.seed(84, 0), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(84, 1), T * K)
    yb = getattr(gemv, EXEC_B[fmt])(W, x, T, M, K).reshape(T, M)
    for t in range(T):
        single = getattr(gemv, EXEC[fmt])(W, x[t * K:(t + 1) * K], M, K)
        assert np.array_equal(yb[t], single)
    exp = ref.gemv(fmt, W, x[:K], M, K, threads=ref.max_threads())
    assert rel_l2(yb[0], exp) < TOL


# Q6_K top-1 through the CU-resident kernels: the index equals the selection
# rule applied to the same context's plain GEMV output (the same per-row
# arithmetic), on shapes with 1..8 unrolled steps and rolled ones.
@pytest.mark.parametrize("M,K", [(400, 256), (4096, 1024), (20000, 3072), (14336, 4096), (151936, 1024),
                                 (128256, 4096)])
def test_cu_top1_matches_rule(cu_gemv, M, K):
    W = synth.weights("q6_k", synth.seed(86, M % 97), M, K, dscale=0.005)
    x = synth.normal_f32(synth.seed(86, 200 + K % 89), K)
    y = cu_gemv.executeQ6KWeights(W, x, M, K)
    assert cu_gemv.executeQ6KWeightsTop1(W, x, M, K) == ref.top1(y)


def test_cu_top1_ties_and_nan(cu_gemv):
    """A copy of the winning row at a lower index wins the tie, at a higher one
    loses it; identical rows give row 0, and all-NaN logits keep row 0."""
    M, K = 8192, 1024
    W = synth.weights("q6_k", synth.seed(87, 0), M, K, dscale=0.005).reshape(M, -1).copy()
    x = synth.normal_f32(synth.seed(87, 1), K)
    a = cu_gemv.executeQ6KWeightsTop1(W.reshape(-1), x, M, K)
    for b in (0, 5, a // 2 if a > 0 else 3, a - 1 if a > 0 else 7):
        if b >= a:
            continue
        Wt = W.copy()
        Wt[b] = W[a]
        assert cu_gemv.executeQ6KWeightsTop1(Wt.reshape(-1), x, M, K) == b
    hi = min(M - 1, a + 1000)
    Wt = W.copy()
    Wt[hi] = W[a]
    assert cu_gemv.executeQ6KWeightsTop1(Wt.reshape(-1), x, M, K) == min(a, hi)
    Wsame = np.tile(W[a], (M, 1))
    assert cu_gemv.executeQ6KWeightsTop1(Wsame.reshape(-1), x, M, K) == 0
    xn = np.full(K, np.nan, np.float32)
    assert cu_gemv.executeQ6KWeightsTop1(W.reshape(-1), xn, M, K) == 0


def test_default_dispatch_q6k_head_top1_consistent(gemv):
    """Default dispatch on the 128256 x 4096 head (rolled CU-resident kernels
    for both the plain GEMV and the top-1)."""
    M, K = 128256, 4096
    W = synth.weights("q6_k", synth.seed(88, 0), M, K, dscale=0.005)
    x = synth.normal_f32(synth.seed(88, 1), K)
    y = gemv.executeQ6KWeights(W, x, M, K)
    assert gemv.executeQ6KWeightsTop1(W, x, M, K) == ref.top1(y)
    exp = ref.gemv("q6_k", W, x, M, K, threads=ref.max_threads())
    assert rel_l2(y, exp) < TOL


@pytest.fixture(scope="module")
def lane_group_gemv():
    c = _context("0")
    yield GEMVKernel(c)
    c.close()


# Every unrolled step count is its own compiled kernel.  (fmt, K, lanes per
# row, step counts): K picks the configuration (the planner's choice at that
# row length), M = CUs x rows per step x steps picks the kernel.
STEP_SWEEP = [("q4_k", 1024, 16, (1, 2, 3, 5, 8)), ("q4_k", 2048, 32, (1, 2, 4, 7, 8)),
              ("q4_k", 4096, 64, (1, 2, 3, 5, 6, 8)), ("q4_k", 8192, 64, (1, 2, 4, 8)),
              ("q4_k", 12288, 64, (1, 2)), ("q4_k", 14336, 32, (1,)), ("q4_k", 16384, 64, (1, 2)),
              ("q8_0", 1024, 16, (1, 3, 8)), ("q8_0", 2048, 32, (2, 5, 8)), ("q8_0", 4096, 64, (1, 4, 7)),
              ("q6_k", 1024, 16, (2, 6, 8)), ("q6_k", 2048, 32, (1, 3, 8)), ("q6_k", 4096, 64, (1, 5, 8))]


@pytest.mark.parametrize("fmt,K,lpr,steps", STEP_SWEEP)
def test_cu_family_every_step_count(cu_gemv, lane_group_gemv, fmt, K, lpr, steps):
    """Each unrolled step count of each configuration: 61 rows spread over
    the matrix (first and last included) against the CPU oracle at the parity
    bar, and every row against the lane-group family, which forms the same
    22-bit x products and fp32 sums in another order."""
    cus = cu_gemv.ctx.compute_units
    step_rows = 8 * (64 // lpr)
    x = synth.normal_f32(synth.seed(86, K % 89), K)
    for j in steps:
        M = cus * step_rows * j
        W = synth.weights(fmt, synth.seed(86, 10 * j + K % 7), M, K, **DSCALE[fmt])
        y = getattr(cu_gemv, EXEC[fmt])(W, x, M, K)
        assert np.all(np.isfinite(y)), (fmt, K, j)
        rows = np.unique(np.linspace(0, M - 1, 61).astype(np.int64))
        Wr = W.reshape(M, -1)[rows].reshape(-1)
        exp = ref.gemv(fmt, Wr, x, len(rows), K)
        assert rel_l2(y[rows], exp) < TOL, (fmt, K, j)
        lg = getattr(lane_group_gemv, EXEC[fmt])(W, x, M, K)
        assert rel_l2(y, lg) < 1e-5, (fmt, K, j, rel_l2(y, lg))


@pytest.mark.parametrize("K,lpr,steps", [(1024, 16, (1, 2, 3, 5, 8)), (2048, 32, (1, 4, 7, 8)),
                                         (4096, 64, (1, 2, 6, 8))])
def test_cu_top1_every_step_count(cu_gemv, K, lpr, steps):
    """Each unrolled step count of the top-1 kernels: the index equals the
    selection rule applied to the same context's GEMV logits (the same
    arithmetic), including a winner planted in the last row."""
    cus = cu_gemv.ctx.compute_units
    step_rows = 8 * (64 // lpr)
    x = synth.normal_f32(synth.seed(88, K % 89), K)
    for j in steps:
        M = cus * step_rows * j
        W = synth.weights("q6_k", synth.seed(88, 10 * j + K % 7), M, K, dscale=0.005)
        y = cu_gemv.executeQ6KWeights(W, x, M, K)
        assert cu_gemv.executeQ6KWeightsTop1(W, x, M, K) == ref.top1(y), (K, j)
        Wl = W.reshape(M, -1).copy()
        Wl[M - 1] = Wl[ref.top1(y)]
        Wl = Wl.reshape(-1)
        yl = cu_gemv.executeQ6KWeights(Wl, x, M, K)
        assert cu_gemv.executeQ6KWeightsTop1(Wl, x, M, K) == ref.top1(yl), (K, j)
