"""The reference's alternative GEMVKernel encoders (GEMVKernel.swift:724,
745, 767, 789, 840, 1045, 1184) and the synchronous execute* conveniences
(:545, 575, 605, 627, 1146) through the C ABI: every alias gives bytes
identical to its canonical entry point on the same buffers, and the execute
forms equal the encode path (and the CPU oracle at the GEMV bar)."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import _ffi
from oracle import ref
from conftest import rel_l2

pytestmark = pytest.mark.gpu

SINGLE = [("er_hip_encode_q4k_weights_packed", "er_hip_encode_q4k_weights", "q4_k"),
          ("er_hip_encode_q4k_weights_packed_four_rows", "er_hip_encode_q4k_weights", "q4_k"),
          ("er_hip_encode_q4k_weights_llama_style", "er_hip_encode_q4k_weights", "q4_k"),
          ("er_hip_encode_q4k_weights_two_rows", "er_hip_encode_q4k_weights", "q4_k"),
          ("er_hip_encode_q6k_weights_packed", "er_hip_encode_q6k_weights", "q6_k")]


def _w(fmt, M, K, t):
    kw = {"dscale": 0.01, "dminscale": 0.01} if fmt == "q4_k" else {"dscale": 0.005}
    return synth.weights(fmt, synth.seed(96, t), M, K, **kw)


@pytest.mark.parametrize("alias,canon,fmt", SINGLE)
@pytest.mark.parametrize("M,K", [(203, 1024), (14336, 4096)])
def test_single_alias_bit_identical(ctx, alias, canon, fmt, M, K):
    lib = _ffi.load()
    W, x = _w(fmt, M, K, 1), synth.normal_f32(synth.seed(96, 2), K)
    wb, xb, ya, yc = ctx.upload(W), ctx.upload(x), ctx.alloc(4 * M), ctx.alloc(4 * M)
    try:
        assert getattr(lib, alias)(ctx.handle, None, wb.raw, xb.raw, ya.raw, M, K) == 0, _ffi.last_error()
        assert getattr(lib, canon)(ctx.handle, None, wb.raw, xb.raw, yc.raw, M, K) == 0, _ffi.last_error()
        ctx.synchronize()
        a, c = ya.download(np.uint32), yc.download(np.uint32)
    finally:
        for b in (wb, xb, ya, yc):
            b.free()
    assert np.array_equal(a, c)


def test_multi_aliases_bit_identical(ctx):
    lib = _ffi.load()
    K = 1024
    rows = [2048, 1024, 1024]
    Ws = [_w("q4_k", r, K, 10 + i) for i, r in enumerate(rows)]
    x = synth.normal_f32(synth.seed(96, 20), K)
    wbs, xb = [ctx.upload(W) for W in Ws], ctx.upload(x)
    outs = [ctx.alloc(4 * r) for r in rows + rows]
    dual = [ctx.alloc(4 * rows[1]) for _ in range(4)]
    try:
        args = [w.raw for w in wbs] + [xb.raw]
        assert lib.er_hip_encode_q4k_weights_triple_packed(ctx.handle, None, *args, *[o.raw for o in outs[:3]],
                                                           *rows, K) == 0
        assert lib.er_hip_encode_q4k_weights_triple(ctx.handle, None, *args, *[o.raw for o in outs[3:]], *rows,
                                                    K) == 0
        d = (wbs[1].raw, wbs[2].raw, xb.raw)
        assert lib.er_hip_encode_q4k_weights_llama_style_dual(ctx.handle, None, *d, dual[0].raw, dual[1].raw,
                                                              rows[1], K) == 0
        assert lib.er_hip_encode_q4k_weights_dual(ctx.handle, None, *d, dual[2].raw, dual[3].raw, rows[1], K) == 0
        ctx.synchronize()
        for i in range(3):
            assert np.array_equal(outs[i].download(np.uint32), outs[3 + i].download(np.uint32))
        assert np.array_equal(dual[0].download(np.uint32), dual[2].download(np.uint32))
        assert np.array_equal(dual[1].download(np.uint32), dual[3].download(np.uint32))
    finally:
        for b in wbs + [xb] + outs + dual:
            b.free()


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k"])
def test_execute_conveniences(ctx, gemv, fmt):
    lib = _ffi.load()
    M, K, T = 96, 1024, 3
    W = _w(fmt, M, K, 30)
    x = synth.normal_f32(synth.seed(96, 31), T * K)
    x0 = np.ascontiguousarray(x[:K])
    enc = gemv.executeQ4KWeights(W, x0, M, K) if fmt == "q4_k" else gemv.executeQ6KWeights(W, x0, M, K)
    y = np.empty(M, np.float32)
    entry = lib.er_hip_execute_q4k_weights if fmt == "q4_k" else lib.er_hip_execute_q6k_weights
    assert entry(ctx.handle, W.ctypes.data, W.size, x0.ctypes.data, K, y.ctypes.data, M, M, K) == 0, _ffi.last_error()
    assert np.array_equal(y.view(np.uint32), enc.view(np.uint32))
    wb = ctx.upload(W)
    try:
        wy = (gemv.executeQ4KWeightsWithWeightBuffer if fmt == "q4_k" else gemv.executeQ6KWeightsWithWeightBuffer)(
            wb, x0, M, K)
    finally:
        wb.free()
    assert np.array_equal(wy.view(np.uint32), enc.view(np.uint32))
    assert rel_l2(y, ref.gemv(fmt, W, x0, M, K)) < 1e-3
    if fmt == "q4_k":
        yb = np.empty(T * M, np.float32)
        assert lib.er_hip_execute_batched_q4k_weights(ctx.handle, W.ctypes.data, W.size, x.ctypes.data, T * K,
                                                      yb.ctypes.data, T * M, T, M, K) == 0, _ffi.last_error()
        assert np.array_equal(yb.view(np.uint32), gemv.executeBatchedQ4KWeights(W, x, T, M, K).view(np.uint32))
