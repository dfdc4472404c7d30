"""Fused Q8_0 projections (dequant_q8_0_fused_qkv / _fused_gate_up_silu /
_fused_final_norm_gemv / _gemv_f16out / _gemv_add) against the CPU oracle:
RMSNorm restated from FusedKernelTests.cpuRMSNorm, the Q8_0 GEMV oracle,
silu from FusedKernelTests.silu.  Bar: relative L2 <= 1e-3 per output
(fp16 outputs compared with the fp16 rounding of the oracle), on the
reference tests' shapes (dim 128, q 64, kv 32, inter 96, 1 and 3 tokens) and
on Llama-sized ones (those of 6144 rows or more on the K-sliced kernels);
batched calls equal per-token calls exactly; every entry forced onto the
K-sliced kernels at odd shapes."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import EncodingFailed, FusedQ8Kernel, GEMVKernel, InvalidMatrixShape, InvalidVectorShape
from oracle import ref
from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3
EPS = 1e-5


@pytest.fixture(scope="module")
def fk(ctx):
    return FusedQ8Kernel(ctx)


def q8(M, K, t):
    return synth.q8_0(synth.seed(70, t), M, K)


def norm_weight(K, t):
    """U[0.5, 1.5) as the reference tests' normW (24-bit uniforms from the seeded generator)."""
    u = (synth.rng_outputs(synth.seed(70, 50 + t), K) >> np.uint64(40)).astype(np.float32) / np.float32(2 ** 24)
    return (np.float32(0.5) + u).astype(np.float32)


def oracle_proj(W, x_t, nw, M, K):
    n = ref.rmsnorm(x_t, nw, EPS) if nw is not None else x_t
    return ref.gemv("q8_0", W, n, M, K, threads=ref.max_threads())


@pytest.mark.parametrize("dim,qd,kvd,T", [(128, 64, 32, 1), (128, 64, 32, 3), (4096, 4096, 1024, 1),
                                          (4096, 4096, 1024, 4), (2048, 2048, 512, 2),
                                          # odd block count and rows beyond 16384 weights: the fp32
                                          # kernels (the reference takes any blocksPerRow,
                                          # Dequant_Q8_0.metal:214-483)
                                          (96, 64, 32, 2), (16416, 256, 128, 2), (160, 96, 40, 3)])
def test_fused_qkv(ctx, fk, dim, qd, kvd, T):
    Wq, Wk, Wv = q8(qd, dim, 1), q8(kvd, dim, 2), q8(kvd, dim, 3)
    x = synth.normal_f32(synth.seed(70, 10 + T), T * dim)
    nw = norm_weight(dim, 0)
    bufs = [ctx.upload(a) for a in (Wq, Wk, Wv, x, nw)]
    oq, ok, ov = ctx.alloc(4 * T * qd), ctx.alloc(4 * T * kvd), ctx.alloc(2 * T * kvd)
    try:
        fk.encodeFusedQKV(None, bufs[0], bufs[1], bufs[2], bufs[3], oq, ok, ov, bufs[4], qd, kvd, dim, T, EPS)
        ctx.synchronize()
        q = oq.download(np.float32).reshape(T, qd)
        k = ok.download(np.float32).reshape(T, kvd)
        v = ov.download(np.float16).reshape(T, kvd)
    finally:
        for b in bufs + [oq, ok, ov]:
            b.free()
    for t in range(T):
        xt = x[t * dim:(t + 1) * dim]
        assert rel_l2(q[t], oracle_proj(Wq, xt, nw, qd, dim)) < TOL
        assert rel_l2(k[t], oracle_proj(Wk, xt, nw, kvd, dim)) < TOL
        ev = oracle_proj(Wv, xt, nw, kvd, dim).astype(np.float16).astype(np.float32)
        assert rel_l2(v[t].astype(np.float32), ev) < TOL


@pytest.mark.parametrize("dim,inter,T", [(128, 96, 3), (128, 96, 1), (4096, 14336, 2), (1024, 3072, 5),
                                         (96, 96, 3), (16416, 512, 2), (20480, 70, 1)])
def test_fused_gate_up_silu(ctx, fk, dim, inter, T):
    Wg, Wu = q8(inter, dim, 4), q8(inter, dim, 5)
    x = synth.normal_f32(synth.seed(70, 20 + T), T * dim)
    nw = norm_weight(dim, 1)
    bufs = [ctx.upload(a) for a in (Wg, Wu, x, nw)]
    out = ctx.alloc(4 * T * inter)
    try:
        fk.encodeFusedGateUpSilu(None, bufs[0], bufs[1], bufs[2], out, bufs[3], inter, dim, T, EPS)
        ctx.synchronize()
        got = out.download(np.float32).reshape(T, inter)
    finally:
        for b in bufs + [out]:
            b.free()
    for t in range(T):
        xt = x[t * dim:(t + 1) * dim]
        g = oracle_proj(Wg, xt, nw, inter, dim)
        u = oracle_proj(Wu, xt, nw, inter, dim)
        assert rel_l2(got[t], ref.silu(g) * u) < TOL


@pytest.mark.parametrize("rows,dim", [(256, 128), (32000, 4096), (151936, 1024), (256, 96), (1000, 16416)])
def test_fused_final_norm_gemv(ctx, fk, rows, dim):
    W = q8(rows, dim, 6)
    x = synth.normal_f32(synth.seed(70, 30), dim)
    nw = norm_weight(dim, 2)
    bufs = [ctx.upload(a) for a in (W, x, nw)]
    out = ctx.alloc(4 * rows)
    try:
        fk.encodeFusedFinalNormGEMV(None, bufs[0], bufs[1], out, bufs[2], rows, dim, EPS)
        ctx.synchronize()
        got = out.download(np.float32)
    finally:
        for b in bufs + [out]:
            b.free()
    assert rel_l2(got, oracle_proj(W, x, nw, rows, dim)) < TOL


@pytest.mark.parametrize("rows,dim", [(96, 128), (1024, 4096), (4096, 14336), (96, 96), (501, 16416),
                                      (6144, 4096)])
def test_gemv_f16out_and_add(ctx, fk, rows, dim):
    W = q8(rows, dim, 7)
    x = synth.normal_f32(synth.seed(70, 31), dim)
    res = synth.normal_f32(synth.seed(70, 32), rows)
    wb, xb, rb = ctx.upload(W), ctx.upload(x), ctx.upload(res)
    yh, ya = ctx.alloc(2 * rows), ctx.alloc(4 * rows)
    try:
        fk.encodeGEMVF16Out(None, wb, xb, yh, rows, dim)
        fk.encodeGEMVAdd(None, wb, xb, rb, ya, rows, dim)
        ctx.synchronize()
        h = yh.download(np.float16).astype(np.float32)
        a = ya.download(np.float32)
    finally:
        for b in (wb, xb, rb, yh, ya):
            b.free()
    exp = oracle_proj(W, x, None, rows, dim)
    assert rel_l2(h, exp.astype(np.float16).astype(np.float32)) < TOL
    assert rel_l2(a, exp + res) < TOL
    plain = GEMVKernel(ctx).executeQ8_0Weights(W, x, rows, dim)
    assert np.allclose(a, plain + res, rtol=1e-5, atol=1e-5 * float(np.max(np.abs(plain))))


def test_fused_qkv_turbo_keeps_v_fp32(ctx, fk):
    """dequant_q8_0_fused_qkv_turbo: q and k equal the fp16-V kernel's exactly;
    v is the fp32 value whose fp16 rounding the other kernel stores."""
    dim, qd, kvd, T = 2048, 2048, 512, 3
    Wq, Wk, Wv = q8(qd, dim, 21), q8(kvd, dim, 22), q8(kvd, dim, 23)
    x = synth.normal_f32(synth.seed(70, 41), T * dim)
    nw = norm_weight(dim, 4)
    bufs = [ctx.upload(a) for a in (Wq, Wk, Wv, x, nw)]
    a = [ctx.alloc(4 * T * qd), ctx.alloc(4 * T * kvd), ctx.alloc(2 * T * kvd)]
    b = [ctx.alloc(4 * T * qd), ctx.alloc(4 * T * kvd), ctx.alloc(4 * T * kvd)]
    try:
        fk.encodeFusedQKV(None, *bufs[:4], *a, bufs[4], qd, kvd, dim, T, EPS)
        fk.encodeFusedQKVTurbo(None, *bufs[:4], *b, bufs[4], qd, kvd, dim, T, EPS)
        ctx.synchronize()
        assert np.array_equal(a[0].download(np.float32), b[0].download(np.float32))
        assert np.array_equal(a[1].download(np.float32), b[1].download(np.float32))
        v32 = b[2].download(np.float32)
        assert np.array_equal(a[2].download(np.float16), v32.astype(np.float16))
        for t in range(T):
            ev = oracle_proj(Wv, x[t * dim:(t + 1) * dim], nw, kvd, dim)
            assert rel_l2(v32[t * kvd:(t + 1) * kvd], ev) < TOL
    finally:
        for buf in bufs + a + b:
            buf.free()


# the second shape's 6144 rows take the K-sliced kernels
@pytest.mark.parametrize("dim,qd,kvd,T", [(1024, 1024, 256, 4), (4096, 4096, 1024, 2)])
def test_batched_equals_per_token(ctx, fk, dim, qd, kvd, T):
    Wq, Wk, Wv = q8(qd, dim, 11), q8(kvd, dim, 12), q8(kvd, dim, 13)
    x = synth.normal_f32(synth.seed(70, 40), T * dim)
    nw = norm_weight(dim, 3)
    bufs = [ctx.upload(a) for a in (Wq, Wk, Wv, x, nw)]
    outs = [ctx.alloc(4 * T * qd), ctx.alloc(4 * T * kvd), ctx.alloc(2 * T * kvd)]
    one = [ctx.alloc(4 * qd), ctx.alloc(4 * kvd), ctx.alloc(2 * kvd)]
    try:
        fk.encodeFusedQKV(None, *bufs[:4], *outs, bufs[4], qd, kvd, dim, T, EPS)
        ctx.synchronize()
        batched = [o.download(np.uint8) for o in outs]
        for t in range(T):
            xt = bufs[3].view(4 * t * dim, 4 * dim)
            fk.encodeFusedQKV(None, *bufs[:3], xt, *one, bufs[4], qd, kvd, dim, 1, EPS)
            ctx.synchronize()
            for o, b, w in zip(one, batched, (4 * qd, 4 * kvd, 2 * kvd)):
                assert np.array_equal(o.download(np.uint8), b[t * w:(t + 1) * w])
    finally:
        for b in bufs + outs + one:
            b.free()


@pytest.fixture(scope="module")
def fk_cuk2():
    """A context whose fused Q8_0 calls take the K-sliced kernels wherever K %
    256 == 0 (ER_HIP_GEMV_CUK=2, read at creation)."""
    import os
    from edgerunner_amd import Context
    old = os.environ.get("ER_HIP_GEMV_CUK")
    os.environ["ER_HIP_GEMV_CUK"] = "2"
    try:
        c = Context(0)
    finally:
        if old is None:
            os.environ.pop("ER_HIP_GEMV_CUK", None)
        else:
            os.environ["ER_HIP_GEMV_CUK"] = old
    yield c, FusedQ8Kernel(c)
    c.close()


# (dim, rows: q / kv for the QKV and final-norm projections, gate/up for the
# SiLU, T): 8, 4 and 2 rows per step (K = 512, 8192, 14336), steps that
# straddle q | k | v and gate/up pairs, a wave with a partial slice (14336:
# 28 of 32 lanes)
@pytest.mark.parametrize("dim,qd,kvd,T", [(512, 130, 42, 2), (8192, 300, 77, 1), (14336, 70, 21, 2)])
def test_k_sliced_fused_forms(fk_cuk2, dim, qd, kvd, T):
    """Every fused Q8_0 entry on the K-sliced kernels (the RMSNorm factor from
    the waves' sums of x^2, fp16 V, the residual, gate/up pairs): within the
    parity bar of the oracle."""
    c, f = fk_cuk2
    Wq, Wk, Wv = q8(qd, dim, 31), q8(kvd, dim, 32), q8(kvd, dim, 33)
    x = synth.normal_f32(synth.seed(70, 60 + T), T * dim)
    nw = norm_weight(dim, 5)
    res = synth.normal_f32(synth.seed(70, 61), qd)
    bufs = [c.upload(a) for a in (Wq, Wk, Wv, x, nw, res)]
    oq, ok, ov = c.alloc(4 * T * qd), c.alloc(4 * T * kvd), c.alloc(2 * T * kvd)
    os_, on, oh, oa = c.alloc(4 * T * kvd), c.alloc(4 * qd), c.alloc(2 * qd), c.alloc(4 * qd)
    try:
        f.encodeFusedQKV(None, bufs[0], bufs[1], bufs[2], bufs[3], oq, ok, ov, bufs[4], qd, kvd, dim, T, EPS)
        f.encodeFusedGateUpSilu(None, bufs[1], bufs[2], bufs[3], os_, bufs[4], kvd, dim, T, EPS)
        f.encodeFusedFinalNormGEMV(None, bufs[0], bufs[3], on, bufs[4], qd, dim, EPS)
        f.encodeGEMVF16Out(None, bufs[0], bufs[3], oh, qd, dim)
        f.encodeGEMVAdd(None, bufs[0], bufs[3], bufs[5], oa, qd, dim)
        c.synchronize()
        q = oq.download(np.float32).reshape(T, qd)
        k = ok.download(np.float32).reshape(T, kvd)
        v = ov.download(np.float16).reshape(T, kvd).astype(np.float32)
        sl = os_.download(np.float32).reshape(T, kvd)
        n, h, a = on.download(np.float32), oh.download(np.float16).astype(np.float32), oa.download(np.float32)
    finally:
        for b in bufs + [oq, ok, ov, os_, on, oh, oa]:
            b.free()
    for t in range(T):
        xt = x[t * dim:(t + 1) * dim]
        eq, ek, ev = (oracle_proj(W, xt, nw, m, dim) for W, m in ((Wq, qd), (Wk, kvd), (Wv, kvd)))
        assert rel_l2(q[t], eq) < TOL and rel_l2(k[t], ek) < TOL
        assert rel_l2(v[t], ev.astype(np.float16).astype(np.float32)) < TOL
        assert rel_l2(sl[t], ref.silu(ek) * ev) < TOL
    x0 = x[:dim]
    assert rel_l2(n, oracle_proj(Wq, x0, nw, qd, dim)) < TOL
    plain = oracle_proj(Wq, x0, None, qd, dim)
    assert rel_l2(h, plain.astype(np.float16).astype(np.float32)) < TOL
    assert rel_l2(a, plain + res) < TOL


def test_validation(ctx, fk):
    W = q8(64, 128, 1)
    wb, xb, nb = ctx.upload(W), ctx.alloc(4 * 128), ctx.alloc(4 * 128)
    y, small = ctx.alloc(4 * 64), ctx.alloc(4 * 10)
    try:
        with pytest.raises(InvalidVectorShape):   # K % 32 != 0
            fk.encodeFusedFinalNormGEMV(None, wb, xb, y, nb, 64, 80, EPS)
        with pytest.raises(InvalidMatrixShape):   # a long row the weight buffer does not hold
            fk.encodeGEMVF16Out(None, wb, xb, y, 1, 16384 + 64)
        with pytest.raises(EncodingFailed):       # output too small
            fk.encodeGEMVAdd(None, wb, xb, y, small, 64, 128)
        with pytest.raises(EncodingFailed):       # norm weight too small
            fk.encodeFusedFinalNormGEMV(None, wb, xb, y, small, 64, 128, EPS)
    finally:
        for b in (wb, xb, nb, y, small):
            b.free()
