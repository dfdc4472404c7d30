"""Output bounds of every kernel family.  Each launch writes into a view of a
larger device buffer whose bytes before and after the view hold a sentinel
pattern (0xA5); after the launch the sentinel bytes must be unchanged, so no
kernel writes outside its output -- including partial row and token tiles,
split-K atomics and its zero fill, the top-1 partial buffers and the
quantizer's destination rows.  Inside the view every element must have been
written (none keeps the sentinel pattern) and be finite."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import (DequantQ4KMKernel, DequantQ6KKernel, DequantQ8_0Kernel, GEMVKernel,
                            QuantGEMMKernel, QuantizeQ8RowsKernel, _ffi)

pytestmark = pytest.mark.gpu

PAD = 4096  # sentinel bytes on each side; keeps every view 16-byte aligned
SENT = 0xA5
SENT_WORD = 0xA5A5A5A5
DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01}, "q6_k": {"dscale": 0.005}}


def guarded(ctx, nbytes):
    """(whole buffer, view of nbytes at PAD) with every byte set to SENT."""
    buf = ctx.alloc(nbytes + 2 * PAD)
    buf.upload(np.full(nbytes + 2 * PAD, SENT, np.uint8))
    return buf, buf.view(PAD, nbytes)


def inside(buf, nbytes, dtype=np.float32):
    """Checks the sentinel bytes around the view and returns the view's contents."""
    ctx = buf.ctx
    ctx.synchronize()
    b = buf.download(np.uint8)
    head, tail = b[:PAD], b[PAD + nbytes:]
    assert np.all(head == SENT), f"bytes written before the output: {np.flatnonzero(head != SENT)[:8]}"
    assert np.all(tail == SENT), f"bytes written past the output: {np.flatnonzero(tail != SENT)[:8]}"
    return b[PAD:PAD + nbytes].view(dtype)


def written_finite(v):
    assert not np.any(v.view(np.uint32) == SENT_WORD), "output elements left unwritten"
    assert np.all(np.isfinite(v))


def _weights(ctx, fmt, M, K, seed):
    return ctx.upload(synth.weights(fmt, synth.seed(seed, 0), M, K, **DSCALE[fmt]))


ENC = {"q8_0": "encodeQ8_0Weights", "q4_k": "encodeQ4KWeights", "q6_k": "encodeQ6KWeights"}
BATCHED = {"q8_0": "encodeBatchedQ8_0Weights", "q4_k": "encodeBatchedQ4KWeights", "q6_k": "encodeBatchedQ6KWeights"}


# shapes that reach the CU-resident family (4096 x 14336, 151936 x 1024), the
# lane-group integer-dot family and partial last steps (777, 1000 rows)
@pytest.mark.parametrize("fmt,M,K", [("q4_k", 4096, 14336), ("q4_k", 777, 2048), ("q8_0", 3072, 1024),
                                     ("q8_0", 1000, 4096), ("q6_k", 151936, 1024), ("q6_k", 777, 1024)])
def test_gemv_writes_only_y(ctx, fmt, M, K):
    gemv = GEMVKernel(ctx)
    wb = _weights(ctx, fmt, M, K, 61)
    xb = ctx.upload(synth.normal_f32(synth.seed(61, 1), K))
    buf, y = guarded(ctx, 4 * M)
    try:
        getattr(gemv, ENC[fmt])(None, wb, xb, y, M, K)
        written_finite(inside(buf, 4 * M))
    finally:
        for b in (wb, xb, buf):
            b.free()


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0", "q6_k"])
def test_batched_gemv_writes_only_y(ctx, fmt):
    gemv = GEMVKernel(ctx)
    B, M, K = 3, 1000, 2048
    wb = _weights(ctx, fmt, M, K, 62)
    xb = ctx.upload(synth.normal_f32(synth.seed(62, 1), B * K))
    buf, y = guarded(ctx, 4 * B * M)
    try:
        getattr(gemv, BATCHED[fmt])(None, wb, xb, y, B, M, K)
        written_finite(inside(buf, 4 * B * M))
    finally:
        for b in (wb, xb, buf):
            b.free()


def test_fused_projections_write_only_their_outputs(ctx):
    gemv = GEMVKernel(ctx)
    K = 1024
    rows = (2048, 1024, 1000)
    ws = [_weights(ctx, "q4_k", M, K, 63 + i) for i, M in enumerate(rows)]
    xb = ctx.upload(synth.normal_f32(synth.seed(63, 9), K))
    outs = [guarded(ctx, 4 * M) for M in rows]
    try:
        gemv.encodeQ4KWeightsTriple(None, *ws, xb, *(o[1] for o in outs), *rows, K)
        for (buf, _), M in zip(outs, rows):
            written_finite(inside(buf, 4 * M))
        dual = [guarded(ctx, 4 * 2048) for _ in range(2)]
        gemv.encodeQ4KWeightsDual(None, ws[0], ws[0], xb, dual[0][1], dual[1][1], 2048, K)
        for buf, _ in dual:
            written_finite(inside(buf, 4 * 2048))
        geglu = guarded(ctx, 4 * 2048)
        gemv.encodeQ4KWeightsDualGeGLU(None, ws[0], ws[0], xb, geglu[1], 2048, K)
        written_finite(inside(geglu[0], 4 * 2048))
        for buf, _ in dual + [geglu]:
            buf.free()
    finally:
        for b in ws + [xb] + [o[0] for o in outs]:
            b.free()


# 512 x 14336 x 256: the loader-specialised kernel (224 tiles); 256 x 1024 x
# 4096: 16 tiles split 8 ways with fp32 atomics into a zero-filled Y;
# 33 x 520 x 2048: 64-token tiles, partial in both dimensions; 200 x 300 x 4096:
# the warp-specialised kernel with partial tiles
@pytest.mark.parametrize("fmt", ["q4_k", "q8_0"])
@pytest.mark.parametrize("T,N,K", [(512, 14336, 256), (256, 1024, 4096), (33, 520, 2048), (200, 300, 4096)])
def test_gemm_writes_only_y(ctx, fmt, T, N, K):
    gemm = QuantGEMMKernel(ctx)
    wb = _weights(ctx, fmt, N, K, 64)
    xb = ctx.upload(synth.normal_bf16(synth.seed(64, 1), T * K))
    buf, y = guarded(ctx, 4 * T * N)
    try:
        (gemm.encodeQ4K if fmt == "q4_k" else gemm.encodeQ8_0)(None, wb, xb, y, T, N, K)
        written_finite(inside(buf, 4 * T * N))
    finally:
        for b in (wb, xb, buf):
            b.free()


@pytest.mark.parametrize("M,K", [(151936, 1024), (1000, 3072)])
def test_top1_writes_only_its_buffers(ctx, M, K):
    gemv = GEMVKernel(ctx)
    n = GEMVKernel.q6KTop1PartialCount(M)
    wb = _weights(ctx, "q6_k", M, K, 65)
    xb = ctx.upload(synth.normal_f32(synth.seed(65, 1), K))
    pv, pi, ob = guarded(ctx, 4 * n), guarded(ctx, 4 * n), guarded(ctx, 4)
    ob2 = guarded(ctx, 4)
    try:
        gemv.encodeQ6KWeightsPackedTop1(None, wb, xb, pv[1], pi[1], ob[1], M, K)
        idx = int(inside(ob[0], 4, np.uint32)[0])
        assert 0 <= idx < M
        inside(pv[0], 4 * n)
        inside(pi[0], 4 * n, np.uint32)
        lib = _ffi.load()
        st = lib.er_hip_encode_q6k_weights_packed_top1_noalloc(ctx.handle, None, wb.raw, xb.raw, ob2[1].raw, M, K)
        assert st == 0, _ffi.last_error()
        assert int(inside(ob2[0], 4, np.uint32)[0]) == idx
    finally:
        for b in (wb, xb, pv[0], pi[0], ob[0], ob2[0]):
            b.free()


def test_quantizer_writes_only_its_rows(ctx):
    q = QuantizeQ8RowsKernel(ctx)
    rows, bpr, base = 5, 8, 3
    src = ctx.upload(synth.normal_f32(synth.seed(66, 1), rows * bpr * 32))
    nbytes = (base + rows) * bpr * 34
    buf, dst = guarded(ctx, nbytes)
    try:
        q.encode(None, src, dst, rows, bpr * 32, base, bpr)
        got = inside(buf, nbytes, np.uint8)
        # rows before the destination row base are not touched either
        assert np.all(got[:base * bpr * 34] == SENT)
        assert not np.all(got[base * bpr * 34:] == SENT)
    finally:
        src.free()
        buf.free()


@pytest.mark.parametrize("kern,fmt", [(DequantQ8_0Kernel, "q8_0"), (DequantQ4KMKernel, "q4_k"),
                                      (DequantQ6KKernel, "q6_k")])
def test_dequant_writes_only_its_values(ctx, kern, fmt):
    k = kern(ctx)
    count = 37
    blocks = synth.weights(fmt, synth.seed(67, 0), 1, count * k.weights_per_block, **DSCALE[fmt])
    ib = ctx.upload(blocks)
    nbytes = 4 * count * k.weights_per_block
    buf, out = guarded(ctx, nbytes)
    try:
        k.encode(None, ib, count, out)
        written_finite(inside(buf, nbytes))
    finally:
        ib.free()
        buf.free()
