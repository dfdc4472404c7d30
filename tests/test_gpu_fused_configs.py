"""Every multi-matrix (int8-limb) kernel configuration, forced through
ER_HIP_GEMV_MULTI_CONFIG=lpr:ns:r in a context of its own, on a row length
that makes some lanes use all NS slots: the Q4_K triple projection and dual
GeGLU, and the Q8_0 RMSNorm + gate/up + SiLU, against the CPU oracle at the
parity bar (relative L2 <= 1e-3); and every one-row form (r = 1) of the
unpaired kernels: the Q4_K triple and the Q8_0 RMSNorm + QKV."""
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
MAX_K = 16384
NS_R = [(1, 4), (1, 2), (2, 4), (2, 2), (3, 2), (4, 2)]


def row_length(lpr: int, ns: int):
    """Smallest multiple of 256 with more than lpr * (ns - 1) 64-weight slots,
    or None when no such row fits the family."""
    slots = -(-(lpr * (ns - 1) + 1) // 4) * 4
    K = 64 * slots
    return K if K <= MAX_K and slots <= lpr * ns else None


CONFIGS = [(l, n, r) for l in (64, 32, 16, 4) for n, r in NS_R if row_length(l, n) is not None]


@pytest.mark.parametrize("lpr,ns,r", CONFIGS)
def test_forced_multi_config(lpr, ns, r):
    K = row_length(lpr, ns)
    old = os.environ.get("ER_HIP_GEMV_MULTI_CONFIG")
    os.environ["ER_HIP_GEMV_MULTI_CONFIG"] = f"{lpr}:{ns}:{r}"
    try:
        ctx = Context(int(os.environ.get("ER_DEVICE", "0")))
    finally:
        if old is None:
            os.environ.pop("ER_HIP_GEMV_MULTI_CONFIG", None)
        else:
            os.environ["ER_HIP_GEMV_MULTI_CONFIG"] = old
    try:
        gemv, fk = GEMVKernel(ctx), FusedQ8Kernel(ctx)
        tag = lpr * 100 + ns * 10 + r
        x = synth.normal_f32(synth.seed(92, tag), K)
        rows = [203, 77, 130]
        Ws = [synth.q4_k(synth.seed(93, 3 * tag + i), m, K) for i, m in enumerate(rows)]
        ys = gemv.executeQ4KWeightsMulti(Ws, x, rows, K)
        exps = [ref.gemv("q4_k", W, x, m, K, threads=ref.max_threads()) for W, m in zip(Ws, rows)]
        for y, e in zip(ys, exps):
            assert rel_l2(y, e) < TOL, ("triple", lpr, ns, r, K)
        y = gemv.executeQ4KWeightsMulti(Ws[:1] * 2, x, [rows[0]] * 2, K, geglu=True)
        assert rel_l2(y, ref.gelu_tanh(exps[0]) * exps[0]) < TOL, ("geglu", lpr, ns, r, K)

        inter, T = 203, 2
        Wg, Wu = synth.q8_0(synth.seed(94, tag), inter, K), synth.q8_0(synth.seed(95, tag), inter, K)
        xt = synth.normal_f32(synth.seed(96, tag), T * K)
        nw = (0.5 + synth.normal_f32(synth.seed(97, tag), K) ** 2 / 4).astype(np.float32)
        bufs = [ctx.upload(a) for a in (Wg, Wu, xt, nw)]
        out = ctx.alloc(4 * T * inter)
        try:
            fk.encodeFusedGateUpSilu(None, bufs[0], bufs[1], bufs[2], out, bufs[3], inter, K, T, EPS)
            ctx.synchronize()
            got = out.download(np.float32).reshape(T, inter)
        finally:
            for b in bufs + [out]:
                b.free()
        for t in range(T):
            n = ref.rmsnorm(xt[t * K:(t + 1) * K], nw, EPS)
            g = ref.gemv("q8_0", Wg, n, inter, K, threads=ref.max_threads())
            u = ref.gemv("q8_0", Wu, n, inter, K, threads=ref.max_threads())
            assert rel_l2(got[t], ref.silu(g) * u) < TOL, ("q8 gate-up-silu", lpr, ns, r, K, t)
    finally:
        ctx.close()


# One-row forms of the unpaired multi-matrix kernels (the Q4_K dual / triple
# and the fused Q8_0 QKV), forced the same way with r = 1.
CONFIGS1 = [(l, n) for l in (64, 32, 16, 4) for n in (1, 2, 3, 4) if row_length(l, n) is not None]


@pytest.mark.parametrize("lpr,ns", CONFIGS1)
def test_forced_one_row_multi_config(lpr, ns):
    K = row_length(lpr, ns)
    old = os.environ.get("ER_HIP_GEMV_MULTI_CONFIG")
    os.environ["ER_HIP_GEMV_MULTI_CONFIG"] = f"{lpr}:{ns}:1"
    try:
        ctx = Context(int(os.environ.get("ER_DEVICE", "0")))
    finally:
        if old is None:
            os.environ.pop("ER_HIP_GEMV_MULTI_CONFIG", None)
        else:
            os.environ["ER_HIP_GEMV_MULTI_CONFIG"] = old
    try:
        gemv, fk = GEMVKernel(ctx), FusedQ8Kernel(ctx)
        tag = lpr * 100 + ns * 10 + 1
        x = synth.normal_f32(synth.seed(92, tag), K)
        rows = [203, 77, 130]
        Ws = [synth.q4_k(synth.seed(93, 3 * tag + i), m, K) for i, m in enumerate(rows)]
        ys = gemv.executeQ4KWeightsMulti(Ws, x, rows, K)
        for W, m, y in zip(Ws, rows, ys):
            assert rel_l2(y, ref.gemv("q4_k", W, x, m, K, threads=ref.max_threads())) < TOL, ("triple", lpr, ns, K)

        qd, kvd = 203, 77
        Wq, Wk, Wv = (synth.q8_0(synth.seed(98, 3 * tag + i), m, K) for i, m in enumerate((qd, kvd, kvd)))
        nw = (0.5 + synth.normal_f32(synth.seed(97, tag), K) ** 2 / 4).astype(np.float32)
        bufs = [ctx.upload(a) for a in (Wq, Wk, Wv, x, nw)]
        oq, ok, ov = ctx.alloc(4 * qd), ctx.alloc(4 * kvd), ctx.alloc(2 * kvd)
        try:
            fk.encodeFusedQKV(None, bufs[0], bufs[1], bufs[2], bufs[3], oq, ok, ov, bufs[4], qd, kvd, K, 1, EPS)
            ctx.synchronize()
            q, k = oq.download(np.float32), ok.download(np.float32)
            v = ov.download(np.float16).astype(np.float32)
        finally:
            for b in bufs + [oq, ok, ov]:
                b.free()
        n = ref.rmsnorm(x, nw, EPS)
        for got, W, m, half in ((q, Wq, qd, False), (k, Wk, kvd, False), (v, Wv, kvd, True)):
            e = ref.gemv("q8_0", W, n, m, K, threads=ref.max_threads())
            if half:
                e = e.astype(np.float16).astype(np.float32)
            assert rel_l2(got, e) < TOL, ("q8 qkv", lpr, ns, K, m)
    finally:
        ctx.close()
