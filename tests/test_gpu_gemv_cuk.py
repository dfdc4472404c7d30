"""K-sliced CU-resident GEMV kernels (Q4_K, Q8_0 and Q6_K rows of up to 16384
weights, the Llama FFN down projection 4096 x 14336 among them): each wave of
a workgroup owns a slice of K, so a row's value is the sum of 8 wave partials.
Against the CPU oracle at the GEMV parity bar (relative L2 <= 1e-3) on 61
rows spread over each matrix, and every row against the whole-row kernels
(ER_HIP_GEMV_CUK=0) at 1e-5; every unrolled step count 1..16; slices that end
mid-wave and a wave with no slice (K = 8448: 20 slots per wave, 132 slots);
exact one-hot columns at the slice boundaries; the same row bit for bit
whatever the row partition or the batch; non-finite and heavy-tailed x; the
Q6_K top-1 on the same kernels equal to the selection rule over the plain
call's logits; the Q4_K dual / triple over the same kernels equal to the
single-matrix calls."""
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
DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01}, "q6_k": {"dscale": 0.005}}
EXEC = {"q8_0": "executeQ8_0Weights", "q4_k": "executeQ4KWeights", "q6_k": "executeQ6KWeights"}
EXEC_B = {"q8_0": "executeBatchedQ8_0Weights", "q4_k": "executeBatchedQ4KWeights",
          "q6_k": "executeBatchedQ6KWeights"}
FMTS = ["q4_k", "q8_0", "q6_k"]  # long rows: all three formats
FMTS_SHORT = ["q4_k", "q8_0"]     # ER_HIP_GEMV_CUK=2 short rows: Q6_K keeps its whole-row kernels


def _ctx(**env):
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return Context(int(os.environ.get("ER_DEVICE", "0")))
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.fixture(scope="module")
def whole_rows():
    c = _ctx(ER_HIP_GEMV_CUK="0")
    yield GEMVKernel(c)
    c.close()


@pytest.fixture(scope="module")
def cuk_everywhere():
    c = _ctx(ER_HIP_GEMV_CUK="2")
    yield GEMVKernel(c)
    c.close()


def sample_rows(M):
    return np.unique(np.linspace(0, M - 1, 61).astype(np.int64))


def oracle_rows(fmt, W, x, M, K, rows):
    Wr = W.reshape(M, -1)[rows].reshape(-1)
    return ref.gemv(fmt, Wr, x, len(rows), K)


# K: 132 slots (17 per wave; for Q6_K 20, the last wave empty), 172 (22 per
# wave; Q6_K 24, 4 in the last), 192, 224 (28 per wave, half of the last
# conversion pass), 256
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("K", [8448, 11008, 12288, 14336, 16384])
def test_every_step_count(gemv, whole_rows, fmt, K):
    cus = gemv.ctx.compute_units
    x = synth.normal_f32(synth.seed(110, K % 97), K)
    for j in range(1, 17):
        M = cus * 2 * j
        W = synth.weights(fmt, synth.seed(110, 10 * j + K % 7), M, K, **DSCALE[fmt])
        y = getattr(gemv, EXEC[fmt])(W, x, M, K)
        assert np.all(np.isfinite(y)), (fmt, K, j)
        rows = sample_rows(M)
        assert rel_l2(y[rows], oracle_rows(fmt, W, x, M, K, rows)) < TOL, (fmt, K, j)
        other = getattr(whole_rows, EXEC[fmt])(W, x, M, K)
        assert rel_l2(y, other) < 1e-5, (fmt, K, j, rel_l2(y, other))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,K", [(1, 14336), (37, 12288), (4095, 14336), (14336, 14336), (5000, 16384),
                                 (5120, 13824)])
def test_partial_and_many_workgroups(gemv, fmt, M, K):
    """A single row, a partial last workgroup, 10 row steps (5000 / 5120
    rows), and more workgroups than CUs (14336 rows: 448 workgroups of 32)."""
    W = synth.weights(fmt, synth.seed(111, M % 89), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(111, 1), K)
    y = getattr(gemv, EXEC[fmt])(W, x, M, K)
    rows = sample_rows(M)
    assert rel_l2(y[rows], oracle_rows(fmt, W, x, M, K, rows)) < TOL


@pytest.mark.parametrize("fmt", FMTS)
def test_one_hot_columns_at_slice_edges(gemv, fmt):
    """K = 14336: 28 slots (1792 weights) per wave.  A one-hot x reads one
    weight column exactly, at each end of a wave's slice and mid-slice."""
    M, K = 600, 14336
    W = synth.weights(fmt, synth.seed(112, 0), M, K, **DSCALE[fmt])
    cols = rn.weights_f32(fmt, W, M, K)
    for j in (0, 63, 64, 1791, 1792, 1793, 5 * 1792 + 700, 7 * 1792, K - 1):
        x = np.zeros(K, np.float32)
        x[j] = 1.0
        y = getattr(gemv, EXEC[fmt])(W, x, M, K)
        assert np.array_equal(y, cols[:, j]), j


@pytest.mark.parametrize("fmt", FMTS)
def test_row_value_independent_of_partition(gemv, fmt):
    """A row's sum is the same bits whether its workgroup holds 2 rows
    (M = 512: one step) or 16 (M = 4096: eight steps), and batched calls
    equal per-token ones."""
    K = 14336
    W = synth.weights(fmt, synth.seed(113, 0), 4096, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(113, 1), 3 * K)
    full = getattr(gemv, EXEC[fmt])(W, x[:K], 4096, K)
    head = getattr(gemv, EXEC[fmt])(W.reshape(4096, -1)[:512].reshape(-1), x[:K], 512, K)
    assert np.array_equal(full[:512].view(np.uint32), head.view(np.uint32))
    yb = getattr(gemv, EXEC_B[fmt])(W, x, 3, 4096, K).reshape(3, 4096)
    for t in range(3):
        single = getattr(gemv, EXEC[fmt])(W, x[t * K:(t + 1) * K], 4096, K)
        assert np.array_equal(yb[t].view(np.uint32), single.view(np.uint32)), t


def _poison(x, kind):
    x = x.copy()
    K = x.size
    if kind == "nan":
        x[K // 3] = np.nan
    elif kind == "pinf":
        x[5000] = np.inf
    elif kind == "pm_inf":
        x[100] = np.inf
        x[K - 7] = -np.inf
    elif kind == "inf_group":
        x[1792 * 3:1792 * 3 + 64] = np.inf
    return x


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("kind", ["nan", "pinf", "pm_inf", "inf_group"])
def test_nonfinite(gemv, fmt, kind):
    M, K = 512, 14336
    W = synth.weights(fmt, synth.seed(114, 0), M, K, **DSCALE[fmt])
    x = _poison(synth.normal_f32(synth.seed(114, 1), K), kind)
    y = getattr(gemv, EXEC[fmt])(W, x, M, K)
    exp = ref.gemv(fmt, W, x, M, K, threads=ref.max_threads())
    assert np.array_equal(np.isnan(y), np.isnan(exp)), kind
    inf = np.isinf(exp)
    assert np.array_equal(y[inf], exp[inf]), kind
    fin = np.isfinite(exp)
    assert np.all(np.isfinite(y[fin])) and (not fin.any() or rel_l2(y[fin], exp[fin]) < TOL), kind


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("amp", [1e3, 1e4, 1e5])
def test_heavy_tailed_x(gemv, fmt, amp):
    """N(0, 1) activations with one channel at amp in six 64-groups spread
    over the wave slices, and every even row's weight zero at those channels
    (those rows sum only the ordinary values)."""
    from test_gpu_heavy_tail import heavy_case, check
    M, K = 1024, 14336
    W, x = heavy_case(fmt, M, K, amp, 3)
    y = getattr(gemv, EXEC[fmt])(W, x, M, K)
    check(y, ref.gemv(fmt, W, x, M, K, threads=ref.max_threads()))


# ER_HIP_GEMV_CUK=2 takes the K-sliced kernels for every K <= 16384: 8 rows per
# step for rows of up to 64 slots (K <= 4096), 4 for up to 128.  K = 256 and
# 512 leave waves with no slice.
@pytest.mark.parametrize("fmt", FMTS_SHORT)
@pytest.mark.parametrize("K", [256, 512, 1024, 3072, 4096, 6144, 8192])
def test_short_rows_every_step_count(cuk_everywhere, whole_rows, fmt, K):
    cus = cuk_everywhere.ctx.compute_units
    par = 8 if K <= 4096 else 4
    x = synth.normal_f32(synth.seed(115, K % 97), K)
    for j in range(1, 17, 3 if par == 4 else 1):  # 8 rows per step: every step count 1..16
        M = cus * par * j
        W = synth.weights(fmt, synth.seed(115, 10 * j + K % 7), M, K, **DSCALE[fmt])
        y = getattr(cuk_everywhere, EXEC[fmt])(W, x, M, K)
        assert np.all(np.isfinite(y)), (fmt, K, j)
        rows = sample_rows(M)
        assert rel_l2(y[rows], oracle_rows(fmt, W, x, M, K, rows)) < TOL, (fmt, K, j)
        other = getattr(whole_rows, EXEC[fmt])(W, x, M, K)
        assert rel_l2(y, other) < 1e-5, (fmt, K, j, rel_l2(y, other))


@pytest.mark.parametrize("fmt", FMTS_SHORT)
@pytest.mark.parametrize("kind", ["nan", "pm_inf"])
def test_short_rows_nonfinite_and_one_hot(cuk_everywhere, fmt, kind):
    M, K = 777, 4096
    W = synth.weights(fmt, synth.seed(116, 0), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(116, 1), K).copy()
    if kind == "nan":
        x[1000] = np.nan
    else:
        x[3] = np.inf
        x[4000] = -np.inf
    y = getattr(cuk_everywhere, EXEC[fmt])(W, x, M, K)
    exp = ref.gemv(fmt, W, x, M, K, threads=ref.max_threads())
    assert np.array_equal(np.isnan(y), np.isnan(exp))
    inf = np.isinf(exp)
    assert np.array_equal(y[inf], exp[inf])
    cols = rn.weights_f32(fmt, W, M, K)
    for j in (0, 511, 512, K - 1):
        xo = np.zeros(K, np.float32)
        xo[j] = 1.0
        assert np.array_equal(getattr(cuk_everywhere, EXEC[fmt])(W, xo, M, K), cols[:, j]), j


# Q6_K top-1 over the K-sliced kernels: the index equals the selection rule
# applied to the same context's plain GEMV output.  Shapes: 2 rows per step
# at 8 and 16 steps, 2 rows at 1 step (the top-1 form rounds to 2), 4 rows
# per step at 2 and 16 steps.
@pytest.mark.parametrize("M,K", [(4096, 14336), (8192, 16384), (400, 10240), (1000, 12288), (2048, 8192),
                                 (16384, 6144)])
def test_q6k_top1_matches_rule(gemv, M, K):
    W = synth.weights("q6_k", synth.seed(117, M % 97), M, K, dscale=0.005)
    x = synth.normal_f32(synth.seed(117, 200 + K % 89), K)
    y = gemv.executeQ6KWeights(W, x, M, K)
    assert gemv.executeQ6KWeightsTop1(W, x, M, K) == ref.top1(y)
    rows = sample_rows(M)
    assert rel_l2(y[rows], oracle_rows("q6_k", W, x, M, K, rows)) < TOL


def test_q6k_top1_ties_and_nan(gemv):
    """A copy of the winning row at a lower index wins the tie, at a higher one
    loses it; all-NaN logits keep row 0."""
    M, K = 4096, 14336
    W = synth.weights("q6_k", synth.seed(118, 0), M, K, dscale=0.005).reshape(M, -1).copy()
    x = synth.normal_f32(synth.seed(118, 1), K)
    a = gemv.executeQ6KWeightsTop1(W.reshape(-1), x, M, K)
    for b in (0, 5, a // 2 if a > 0 else 3):
        if b >= a:
            continue
        Wt = W.copy()
        Wt[b] = W[a]
        assert gemv.executeQ6KWeightsTop1(Wt.reshape(-1), x, M, K) == b
    hi = min(M - 1, a + 1000)
    Wt = W.copy()
    Wt[hi] = W[a]
    assert gemv.executeQ6KWeightsTop1(Wt.reshape(-1), x, M, K) == min(a, hi)
    xn = np.full(K, np.nan, np.float32)
    assert gemv.executeQ6KWeightsTop1(W.reshape(-1), xn, M, K) == 0


# (rows of each matrix -- the dual's two are of one height --, K, whether the
# default plan takes the K-sliced kernels for the total rows: from 12 rows per
# CU at K = 4096 and 8 beyond, with slices filling 7/8 of their lanes): steps
# that straddle two
# matrices (3201 with 8 rows per step, 700 + 130 and 5001 with 4, 9 with 2),
# every PAR, K = 16384
@pytest.mark.parametrize("rows,K,default_cuk", [((4096, 1024, 1024), 4096, True), ((3201, 3201), 4096, True),
                                                ((5001, 1000, 1000), 7680, True), ((3100, 3100), 8192, True),
                                                ((5001, 1000, 1000), 5120, False),
                                                ((700, 130, 130), 5120, False), ((300, 300), 8192, False),
                                                ((9, 9), 16384, False), ((40, 17, 5), 1024, False)])
def test_q4k_multi_over_k_sliced(gemv, cuk_everywhere, rows, K, default_cuk):
    """Q4_K dual / triple where the total rows take the K-sliced kernels (one
    launch over the concatenated rows): every row equal bit for bit to a
    K-sliced call of its own matrix (a row's value depends on K alone) and
    within the parity bar of the oracle.  With ER_HIP_GEMV_CUK=2 the smaller
    totals, the half-filled slices and the short rows take them too."""
    Ws = [synth.q4_k(synth.seed(52, i), m, K) for i, m in enumerate(rows)]
    x = synth.normal_f32(synth.seed(52, 9), K)
    singles = [cuk_everywhere.executeQ4KWeights(W, x, m, K) for W, m in zip(Ws, rows)]
    for kern in ((gemv, cuk_everywhere) if default_cuk else (cuk_everywhere,)):
        ys = kern.executeQ4KWeightsMulti(Ws, x, list(rows), K)
        for W, m, y, s in zip(Ws, rows, ys, singles):
            assert np.array_equal(y, s)
            assert rel_l2(y, ref.gemv("q4_k", W, x, m, K)) < TOL
