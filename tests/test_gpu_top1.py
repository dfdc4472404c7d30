"""Greedy top-1 over a Q6_K head (encodeQ6KWeightsPackedTop1): the index must
equal the reference's selection rule applied to the logits.  Exact equality
on three inputs: the oracle's logits where their top two are clearly apart,
this library's own Q6_K GEMV logits (the same kernel arithmetic, so the rule
must reproduce its choice bit for bit), and constructed ties."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import EncodingFailed, InvalidMatrixShape, InvalidVectorShape
from oracle import ref

pytestmark = pytest.mark.gpu


def q6(M, K, seed):
    return synth.weights("q6_k", synth.seed(40, seed), M, K, dscale=0.005)


def test_reference_top1_case(gemv):
    """packedQ6KTop1MatchesCPUReference (GEMVTests.swift:624-660)."""
    M, K = 12, 768
    W = ref.make_q6k_weights(M, K)
    x = (((np.arange(K) % 23) - 11) / 29.0).astype(np.float32)
    expected = ref.gemv("q6_k", W, x, M, K)
    assert gemv.executeQ6KWeightsTop1(W, x, M, K) == ref.argmax(expected) == ref.top1(expected)


@pytest.mark.parametrize("M,K", [(4, 256), (8, 512), (100, 1024), (1000, 3072), (4096, 4096),
                                 (65536, 1024), (1024, 16384), (12, 2304),
                                 # rows longer than the integer-dot kernels take: the fp32
                                 # family with the top-1 epilogue (the reference takes any
                                 # K % 256 == 0, GEMVKernel.swift:1205-1265)
                                 (64, 16640), (1000, 20480), (8, 33024)])
def test_top1_matches_rule_on_gemv_logits(gemv, M, K):
    W = q6(M, K, M % 13)
    x = synth.normal_f32(synth.seed(40, 100 + K % 97), K)
    y = gemv.executeQ6KWeights(W, x, M, K)
    idx = gemv.executeQ6KWeightsTop1(W, x, M, K)
    assert idx == ref.top1(y)
    exp = ref.gemv("q6_k", W, x, M, K, threads=ref.max_threads())
    near_oracle_max(idx, y, exp)
    top2 = np.sort(exp)[-2:]
    if top2[1] - top2[0] > 1e-3 * max(1.0, abs(top2[1])):
        assert idx == ref.argmax(exp)


def near_oracle_max(idx, y, exp):
    """Every case, whatever the oracle's top-2 gap: the chosen row is the
    first maximum of the library's logits y, and y is within e = max|y - exp|
    of the oracle's logits, so exp[idx] >= y[idx] - e >= y[j] - e >= exp[j] - 2e
    for every row j: the chosen row's oracle logit is within 2e of the oracle's
    maximum."""
    e = float(np.max(np.abs(y.astype(np.float64) - exp)))
    assert exp[idx] >= np.max(exp) - 2.0 * e - 1e-6 * abs(float(np.max(exp))), (idx, e)


def test_top1_head_shape(gemv):
    """BASELINE config 3 head (151936 x 1024)."""
    M, K = 151936, 1024
    W = synth.weights("q6_k", synth.seed(3, 0), M, K, dscale=0.005)
    x = synth.normal_f32(synth.seed(3, 1), K)
    y = gemv.executeQ6KWeights(W, x, M, K)
    idx = gemv.executeQ6KWeightsTop1(W, x, M, K)
    assert idx == ref.top1(y)
    exp = ref.gemv("q6_k", W, x, M, K, threads=ref.max_threads())
    near_oracle_max(idx, y, exp)
    top2 = np.sort(exp)[-2:]
    print(f"head top-1 row {idx}, oracle top-2 gap {top2[1] - top2[0]:.3e}")
    if top2[1] - top2[0] > 1e-3 * max(1.0, abs(top2[1])):
        assert idx == ref.argmax(exp)


def test_top1_ties_pick_lowest_row(gemv):
    M, K = 2048, 1024
    W = q6(M, K, 3).reshape(M, -1).copy()
    x = synth.normal_f32(synth.seed(40, 7), K)
    a = gemv.executeQ6KWeightsTop1(W.reshape(-1), x, M, K)
    # a copy of the winning row at a lower index wins the tie; at a higher one it loses
    for b in (0, 1, 5, a // 2 if a > 0 else 3):
        if b >= a:
            continue
        Wt = W.copy()
        Wt[b] = W[a]
        assert gemv.executeQ6KWeightsTop1(Wt.reshape(-1), x, M, K) == b
    hi = min(M - 1, a + 4 + 3)
    Wt = W.copy()
    Wt[hi] = W[a]
    assert gemv.executeQ6KWeightsTop1(Wt.reshape(-1), x, M, K) == min(a, hi)
    # every row identical: row 0
    Wsame = np.tile(W[a], (M, 1))
    assert gemv.executeQ6KWeightsTop1(Wsame.reshape(-1), x, M, K) == 0


def test_top1_nan_input_returns_row_zero(gemv):
    """All logits NaN: no quad candidate can win the merge, which keeps row 0."""
    M, K = 64, 256
    W = q6(M, K, 9)
    x = np.full(K, np.nan, np.float32)
    assert gemv.executeQ6KWeightsTop1(W, x, M, K) == 0


def test_top1_validation(ctx, gemv):
    M, K = 16, 256
    W = q6(M, K, 1)
    x = synth.normal_f32(1, K)
    wb, xb = ctx.upload(W), ctx.upload(x)
    pv, pi, ob = ctx.alloc(4 * 4), ctx.alloc(4 * 4), ctx.alloc(4)
    small = ctx.alloc(4 * 3)
    try:
        with pytest.raises(InvalidMatrixShape):   # M % 4 != 0
            gemv.encodeQ6KWeightsPackedTop1(None, wb, xb, pv, pi, ob, 14, K)
        with pytest.raises(InvalidVectorShape):   # K % 256 != 0
            gemv.encodeQ6KWeightsPackedTop1(None, wb, xb, pv, pi, ob, M, 128)
        with pytest.raises(EncodingFailed):       # partials below M/4
            gemv.encodeQ6KWeightsPackedTop1(None, wb, xb, small, pi, ob, M, K)
        with pytest.raises(EncodingFailed):
            gemv.encodeQ6KWeightsPackedTop1(None, wb, xb, pv, small, ob, M, K)
        gemv.encodeQ6KWeightsPackedTop1(None, wb, xb, pv, pi, ob, M, K)
        ctx.synchronize()
        y = gemv.executeQ6KWeights(W, x, M, K)
        assert int(ob.download(np.uint32, 1)[0]) == ref.top1(y)
    finally:
        for b in (wb, xb, pv, pi, ob, small):
            b.free()


def test_top1_graph_replays(ctx, gemv):
    """Recorded once, replayed three times with new x written between replays."""
    from edgerunner_amd import Capture
    M, K = 8192, 1024
    W = q6(M, K, 4)
    s = ctx.stream()
    wb = ctx.upload(W, s)
    n = gemv.q6KTop1PartialCount(M)
    xb, pv, pi, ob = ctx.alloc(4 * K), ctx.alloc(4 * n), ctx.alloc(4 * n), ctx.alloc(4)
    with Capture(ctx, s) as cap:
        gemv.encodeQ6KWeightsPackedTop1(s, wb, xb, pv, pi, ob, M, K)
    try:
        for t in range(3):
            x = synth.normal_f32(synth.seed(40, 200 + t), K)
            xb.upload(x, stream=s)
            cap.graph.launch(s)
            s.synchronize()
            y = gemv.executeQ6KWeights(W, x, M, K)
            assert int(ob.download(np.uint32, 1, stream=s)[0]) == ref.top1(y)
    finally:
        cap.graph.destroy()
        for b in (wb, xb, pv, pi, ob):
            b.free()
        s.destroy()


def _top1_setup(ctx, gemv, M, K, seed, stream):
    W = q6(M, K, seed)
    x = synth.normal_f32(synth.seed(41, seed), K)
    n = gemv.q6KTop1PartialCount(M)
    bufs = (ctx.upload(W, stream), ctx.upload(x, stream), ctx.alloc(4 * n), ctx.alloc(4 * n), ctx.alloc(4))
    return W, x, bufs


def test_top1_concurrent_streams(ctx, gemv):
    """Top-1 launches in flight on two streams at once, CU-resident and
    lane-group kernels mixed: every index matches its own logits."""
    shapes = [(151936, 1024), (8192, 1024), (20000, 3072), (4096, 4096)]
    streams = [ctx.stream(), ctx.stream()]
    cases = []
    try:
        for i, (M, K) in enumerate(shapes):
            cases.append((M, K) + _top1_setup(ctx, gemv, M, K, i, streams[i % 2]))
        for s in streams:
            s.synchronize()
        for rep in range(3):
            for i, (M, K, W, x, (wb, xb, pv, pi, ob)) in enumerate(cases):
                gemv.encodeQ6KWeightsPackedTop1(streams[i % 2], wb, xb, pv, pi, ob, M, K)
        for s in streams:
            s.synchronize()
        for i, (M, K, W, x, (wb, xb, pv, pi, ob)) in enumerate(cases):
            y = gemv.executeQ6KWeights(W, x, M, K)
            assert int(ob.download(np.uint32, 1)[0]) == ref.top1(y), (M, K)
    finally:
        for c in cases:
            for b in c[4]:
                b.free()
        for s in streams:
            s.destroy()


def test_top1_many_launches_share_partials(ctx, gemv):
    """1100 top-1 launches back to back on one stream, all over the same
    partial buffers and four index buffers: each launch's partials are
    complete before the next launch overwrites them."""
    M, K = 4096, 1024
    s = ctx.stream()
    W, x, (wb, xb, pv, pi, ob) = _top1_setup(ctx, gemv, M, K, 9, s)
    outs = [ctx.alloc(4) for _ in range(4)]
    try:
        for i in range(1100):
            gemv.encodeQ6KWeightsPackedTop1(s, wb, xb, pv, pi, outs[i % 4], M, K)
        s.synchronize()
        exp = ref.top1(gemv.executeQ6KWeights(W, x, M, K))
        for o in outs:
            assert int(o.download(np.uint32, 1, stream=s)[0]) == exp
    finally:
        for b in (wb, xb, pv, pi, ob, *outs):
            b.free()
        s.destroy()
