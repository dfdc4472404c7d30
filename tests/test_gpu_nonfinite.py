"""Non-finite activations: NaN and +-inf in x, carried as the reference's CPU
loops carry them (GEMVTests.swift:61-134, FusedKernelTests.swift:60-83, and
the NaN/inf logit checks that rely on it, LlamaLanguageModel.swift:849-850).

Bar, against the CPU oracle on the same inputs: the set of NaN outputs is
the oracle's, every infinite output equals the oracle's (sign included), and
the finite outputs are within 1e-3 relative L2.  Every GEMV kernel family
runs: the lane-group integer kernels (ER_HIP_GEMV_CU=0), the CU-resident
kernels (ER_HIP_GEMV_CU=1, unrolled and rolled), the fp32 family
(ER_HIP_GEMV_FP32=1, and rows longer than 16384 weights), the odd-block Q8_0
kernel, batched calls with one poisoned token, the fused Q4_K and Q8_0
projections (with and without the RMSNorm prologue) and the Q6_K top-1."""
import os

import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import Context, FusedQ8Kernel, GEMVKernel
from oracle import ref
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-3
EPS = 1e-5
FMTS = ["q4_k", "q8_0", "q6_k"]
EXEC = {"q8_0": "executeQ8_0Weights", "q4_k": "executeQ4KWeights", "q6_k": "executeQ6KWeights"}
EXEC_B = {"q8_0": "executeBatchedQ8_0Weights", "q4_k": "executeBatchedQ4KWeights",
          "q6_k": "executeBatchedQ6KWeights"}
DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01},
          "q6_k": {"dscale": 0.005}}
KINDS = ["nan", "pinf", "ninf", "pinf_group", "nan_group", "pm_inf"]


def poison(x: np.ndarray, kind: str) -> np.ndarray:
    """x with non-finite values planted: one NaN / +inf / -inf in the middle,
    a whole 64-group of +inf or NaN, or +inf and -inf in different groups."""
    x = x.copy()
    K = x.size
    p = K // 3 + 5
    g = (K // 64) // 2
    if kind == "nan":
        x[p] = np.nan
    elif kind == "pinf":
        x[p] = np.inf
    elif kind == "ninf":
        x[p] = -np.inf
    elif kind == "pinf_group":
        x[64 * g:64 * g + 64] = np.inf
    elif kind == "nan_group":
        x[64 * g:64 * g + 64] = np.nan
    elif kind == "pm_inf":
        x[p] = np.inf
        x[(p + K // 2) % K] = -np.inf
    else:
        raise ValueError(kind)
    return x


def assert_matches(got, exp, what=""):
    got = np.asarray(got, dtype=np.float32).ravel()
    exp = np.asarray(exp, dtype=np.float32).ravel()
    gn, en = np.isnan(got), np.isnan(exp)
    assert np.array_equal(gn, en), f"{what}: NaN mask differs at {np.flatnonzero(gn != en)[:8]}"
    gi, ei = np.isinf(got), np.isinf(exp)
    assert np.array_equal(gi, ei), f"{what}: inf mask differs at {np.flatnonzero(gi != ei)[:8]}"
    assert np.array_equal(got[gi], exp[ei]), f"{what}: inf signs differ"
    fin = ~(en | ei)
    if fin.any():
        assert rel_l2(got[fin], exp[fin]) < TOL, what


def _context(**env) -> Context:
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
def families():
    ctxs = {"lane": _context(ER_HIP_GEMV_CU="0"), "cu": _context(ER_HIP_GEMV_CU="1"),
            "fp32": _context(ER_HIP_GEMV_FP32="1")}
    yield {k: GEMVKernel(c) for k, c in ctxs.items()}
    for c in ctxs.values():
        c.close()


def weights(fmt, M, K, t):
    return synth.weights(fmt, synth.seed(90, t), M, K, **DSCALE[fmt])


def oracle(fmt, W, x, M, K, tokens=1):
    return ref.gemv(fmt, W, x, M, K, tokens=tokens, threads=ref.max_threads())


# (family, M, K): lane-group and fp32 kernels on a partial last workgroup,
# CU-resident unrolled (1000 x 4096, 14336 x 4096) and rolled (28672 x 1024).
SHAPES = [("lane", 203, 1024), ("lane", 96, 4096), ("cu", 1000, 4096), ("cu", 14336, 4096),
          ("cu", 28672, 1024), ("fp32", 203, 1024)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("family,M,K", SHAPES)
@pytest.mark.parametrize("kind", KINDS)
def test_gemv_nonfinite(families, fmt, family, M, K, kind):
    W = weights(fmt, M, K, 1)
    x = poison(synth.normal_f32(synth.seed(90, 2), K), kind)
    got = getattr(families[family], EXEC[fmt])(W, x, M, K)
    assert_matches(got, oracle(fmt, W, x, M, K), f"{fmt} {family} {M}x{K} {kind}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("kind", ["nan", "pinf", "pinf_group", "pm_inf"])
def test_long_rows_nonfinite(gemv, fmt, kind):
    """Rows longer than the integer kernels take (fp32 family by default)."""
    M, K = 64, 16640
    W = weights(fmt, M, K, 3)
    x = poison(synth.normal_f32(synth.seed(90, 4), K), kind)
    assert_matches(getattr(gemv, EXEC[fmt])(W, x, M, K), oracle(fmt, W, x, M, K), f"{fmt} {kind}")


@pytest.mark.parametrize("kind", KINDS)
def test_q8_0_odd_blocks_nonfinite(gemv, kind):
    """K / 32 odd: the fp32 any-shape Q8_0 kernel."""
    M, K = 77, 1056
    W = weights("q8_0", M, K, 5)
    x = poison(synth.normal_f32(synth.seed(90, 6), K), kind)
    assert_matches(gemv.executeQ8_0Weights(W, x, M, K), oracle("q8_0", W, x, M, K), kind)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("family,M,K", [("lane", 203, 1024), ("cu", 14336, 4096)])
@pytest.mark.parametrize("kind", ["nan", "pinf", "nan_group"])
def test_batched_one_token_poisoned(families, fmt, family, M, K, kind):
    T = 3
    W = weights(fmt, M, K, 7)
    xs = [synth.normal_f32(synth.seed(90, 8 + t), K) for t in range(T)]
    xs[1] = poison(xs[1], kind)
    x = np.concatenate(xs)
    g = families[family]
    got = getattr(g, EXEC_B[fmt])(W, x, T, M, K).reshape(T, M)
    exp = oracle(fmt, W, x, M, K, tokens=T).reshape(T, M)
    for t in range(T):
        assert_matches(got[t], exp[t], f"token {t}")
        single = getattr(g, EXEC[fmt])(W, xs[t], M, K)
        assert np.array_equal(got[t].view(np.uint32), single.view(np.uint32))
    assert np.all(np.isfinite(got[0])) and np.all(np.isfinite(got[2]))


@pytest.mark.parametrize("kind", ["nan", "pinf", "ninf", "pinf_group", "pm_inf"])
@pytest.mark.parametrize("mode", ["dual", "triple", "geglu"])
@pytest.mark.parametrize("K", [1024, 4096])
def test_q4k_multi_nonfinite(gemv, kind, mode, K):
    """Dual / triple Q4_K projections sharing x, and the GeGLU pair (K = 4096:
    on the K-sliced kernels)."""
    geglu = mode == "geglu"
    rows = [2048, 1024, 1024] if mode == "triple" else [3072, 3072]
    Ws = [weights("q4_k", r, K, 10 + i) for i, r in enumerate(rows)]
    x = poison(synth.normal_f32(synth.seed(90, 13), K), kind)
    got = gemv.executeQ4KWeightsMulti(Ws, x, rows, K, geglu=geglu)
    exps = [oracle("q4_k", W, x, r, K) for W, r in zip(Ws, rows)]
    if geglu:
        assert_matches(got, ref.gelu_tanh(exps[0]) * exps[1], kind)
    else:
        for g, e in zip(got, exps):
            assert_matches(g, e, kind)


def norm_weight(K):
    return (0.5 + np.arange(K, dtype=np.float32) % 7 / 7.0).astype(np.float32)


@pytest.mark.parametrize("kind", ["nan", "pinf", "ninf", "pm_inf"])
@pytest.mark.parametrize("dim,qd,kvd", [(1024, 1024, 256), (4096, 4096, 1024)])
def test_q8_0_fused_nonfinite(ctx, kind, dim, qd, kvd):
    """RMSNorm-fused QKV / gate-up-SiLU / final-norm GEMV (a non-finite x makes
    every normalised value NaN in the reference's cpuRMSNorm, so every output
    is NaN), and the unnormalised f16-out / residual-add GEMVs (dim 4096: on
    the K-sliced kernels)."""
    fk = FusedQ8Kernel(ctx)
    inter, T = 3072, 2
    Wq, Wk, Wv = weights("q8_0", qd, dim, 20), weights("q8_0", kvd, dim, 21), weights("q8_0", kvd, dim, 22)
    Wg, Wu = weights("q8_0", inter, dim, 23), weights("q8_0", inter, dim, 24)
    xs = [synth.normal_f32(synth.seed(90, 25), dim), poison(synth.normal_f32(synth.seed(90, 26), dim), kind)]
    x = np.concatenate(xs)
    nw = norm_weight(dim)
    res = synth.normal_f32(synth.seed(90, 27), qd)
    bufs = {k: ctx.upload(v) for k, v in dict(Wq=Wq, Wk=Wk, Wv=Wv, Wg=Wg, Wu=Wu, x=x, nw=nw, res=res).items()}
    out = {k: ctx.alloc(n) for k, n in dict(q=4 * T * qd, k=4 * T * kvd, v=2 * T * kvd, a=4 * T * inter,
                                            f=4 * qd, h=2 * qd, r=4 * qd).items()}
    xp = bufs["x"].view(4 * dim, 4 * dim)  # the poisoned token alone
    try:
        fk.encodeFusedQKV(None, bufs["Wq"], bufs["Wk"], bufs["Wv"], bufs["x"], out["q"], out["k"], out["v"],
                          bufs["nw"], qd, kvd, dim, T, EPS)
        fk.encodeFusedGateUpSilu(None, bufs["Wg"], bufs["Wu"], bufs["x"], out["a"], bufs["nw"], inter, dim, T, EPS)
        fk.encodeFusedFinalNormGEMV(None, bufs["Wq"], xp, out["f"], bufs["nw"], qd, dim, EPS)
        fk.encodeGEMVF16Out(None, bufs["Wq"], xp, out["h"], qd, dim)
        fk.encodeGEMVAdd(None, bufs["Wq"], xp, bufs["res"], out["r"], qd, dim)
        ctx.synchronize()
        q = out["q"].download(np.float32).reshape(T, qd)
        k = out["k"].download(np.float32).reshape(T, kvd)
        v = out["v"].download(np.float16).reshape(T, kvd).astype(np.float32)
        a = out["a"].download(np.float32).reshape(T, inter)
        f = out["f"].download(np.float32)
        h = out["h"].download(np.float16).astype(np.float32)
        r = out["r"].download(np.float32)
    finally:
        for b in list(bufs.values()) + list(out.values()):
            b.free()
    for t in range(T):
        n = ref.rmsnorm(xs[t], nw, EPS)
        assert_matches(q[t], oracle("q8_0", Wq, n, qd, dim), f"q token {t}")
        assert_matches(k[t], oracle("q8_0", Wk, n, kvd, dim), f"k token {t}")
        ev = oracle("q8_0", Wv, n, kvd, dim).astype(np.float16).astype(np.float32)
        assert_matches(v[t], ev, f"v token {t}")
        g, u = oracle("q8_0", Wg, n, inter, dim), oracle("q8_0", Wu, n, inter, dim)
        assert_matches(a[t], ref.silu(g) * u, f"silu token {t}")
    assert np.all(np.isnan(q[1])) and np.all(np.isnan(a[1]))
    assert_matches(f, oracle("q8_0", Wq, ref.rmsnorm(xs[1], nw, EPS), qd, dim), "final norm")
    plain = oracle("q8_0", Wq, xs[1], qd, dim)
    assert_matches(h, plain.astype(np.float16).astype(np.float32), "f16 out")
    assert_matches(r, plain + res, "gemv add")


@pytest.mark.parametrize("M,K", [(2048, 1024), (151936, 1024)])
@pytest.mark.parametrize("kind", ["nan", "pinf", "ninf", "pm_inf"])
def test_q6k_top1_nonfinite(gemv, M, K, kind):
    """The top-1 index over non-finite logits follows the selection rule
    (NaN quad heads, lowest index among equal infinities) on the oracle's
    logits, whose NaN / inf pattern the kernels reproduce exactly."""
    W = weights("q6_k", M, K, 30)
    x = poison(synth.normal_f32(synth.seed(90, 31), K), kind)
    logits = oracle("q6_k", W, x, M, K)
    assert_matches(gemv.executeQ6KWeights(W, x, M, K), logits, kind)
    assert gemv.executeQ6KWeightsTop1(W, x, M, K) == ref.top1(logits)
