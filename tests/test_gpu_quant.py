"""Q8_0 row quantizer (quantize_q8_0_rows): byte-exact against the CPU oracle
(integer output: every d and q byte must match), on random rows, padded
source strides, a destination row base with the surrounding rows kept,
unaligned sources (scalar-load kernel), closed-form edge rows, and the
prefill activation size; plus the round-trip bound at full size."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import EncodingFailed, QuantizeQ8RowsKernel
from oracle import ref
from oracle import restate_np as rn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def quant(ctx):
    return QuantizeQ8RowsKernel(ctx)


@pytest.mark.parametrize("rows,bpr,pad", [(1, 1, 0), (3, 4, 0), (17, 4, 8), (64, 32, 0),
                                          (5, 3, 1), (1000, 2, 0), (33, 128, 32)])
def test_random_rows_byte_exact(quant, rows, bpr, pad):
    stride = bpr * 32 + pad
    src = (synth.normal_f32(synth.seed(50, rows % 16), rows * stride) * 3.0).astype(np.float32)
    got = quant.execute(src, rows, stride, 0, bpr)
    exp = ref.quantize_q8_0_rows(src, rows, stride, 0, bpr)
    assert np.array_equal(got, exp)


def test_destination_row_base_keeps_other_rows(quant):
    rows, bpr, base = 4, 4, 3
    src = synth.normal_f32(synth.seed(50, 20), rows * bpr * 32)
    total = base + rows + 2
    before = synth.q8_0(synth.seed(50, 21), total, bpr * 32)
    got = quant.execute(src, rows, bpr * 32, base, bpr,
                        destination=before[: (base + rows) * bpr * 34])
    exp = ref.quantize_q8_0_rows(src, rows, bpr * 32, base, bpr,
                                 dst=before[: (base + rows) * bpr * 34].copy())
    assert np.array_equal(got, exp)
    assert np.array_equal(got[: base * bpr * 34], before[: base * bpr * 34])


@pytest.mark.parametrize("offset,base,rows,bpr", [(0, 0, 37, 24), (2, 0, 37, 24), (16, 0, 37, 24),
                                                  (0, 2, 37, 4), (0, 1, 37, 4), (34, 1, 40, 8),
                                                  (0, 0, 3, 3), (16, 2, 130, 32)])
def test_destination_alignments(ctx, quant, offset, base, rows, bpr):
    """Destinations whose first written block is 16-byte aligned or not (a
    byte offset into the buffer, a destination row base), with block counts
    that are not multiples of a wave's 8 blocks or a workgroup's 64: every
    written byte matches the oracle, every other byte is kept."""
    src = synth.normal_f32(synth.seed(50, 30 + offset + base), rows * bpr * 32)
    n = offset + (base + rows) * bpr * 34 + 40
    before = synth.q8_0(synth.seed(50, 31), (n + 33) // 34, 32)[:n].copy()
    sb, db = ctx.upload(src), ctx.upload(before)
    try:
        quant.encode(None, sb, db.view(offset), rows, bpr * 32, base, bpr)
        ctx.synchronize()
        got = db.download(np.uint8)
    finally:
        sb.free()
        db.free()
    exp = before.copy()
    region = exp[offset:offset + (base + rows) * bpr * 34]
    exp[offset:offset + (base + rows) * bpr * 34] = ref.quantize_q8_0_rows(src, rows, bpr * 32, base, bpr,
                                                                            dst=region.copy())
    assert np.array_equal(got, exp)


def test_unaligned_source_uses_scalar_kernel(ctx, quant):
    rows, bpr = 9, 4
    src = synth.normal_f32(synth.seed(50, 22), rows * bpr * 32 + 1)
    sb = ctx.upload(src)
    db = ctx.alloc(rows * bpr * 34)
    try:
        quant.encode(None, sb.view(4), db, rows, bpr * 32, 0, bpr)   # 4-byte aligned source
        ctx.synchronize()
        got = db.download(np.uint8)
    finally:
        sb.free()
        db.free()
    assert np.array_equal(got, ref.quantize_q8_0_rows(src[1:], rows, bpr * 32, 0, bpr))


def test_edge_rows_byte_exact(quant):
    """Zero block, rint ties, fp16-subnormal and fp16-overflowing scales,
    signed zeros, a single nonzero value, values just below the maximum."""
    blocks = []
    blocks.append(np.zeros(32, np.float32))
    b = np.zeros(32, np.float32)
    b[:4] = [127.0, 0.5, 1.5, -2.5]
    blocks.append(b)
    blocks.append((synth.normal_f32(1, 32) * 1e-6).astype(np.float32))      # scale ~ 1e-8: fp16 subnormal
    blocks.append((synth.normal_f32(2, 32) * 1e-9).astype(np.float32))      # scale rounds to fp16 zero
    blocks.append((synth.normal_f32(3, 32) * 3e7).astype(np.float32))       # scale above fp16 max
    blocks.append(np.array([-0.0] * 31 + [0.0], np.float32))
    b = np.zeros(32, np.float32)
    b[17] = -3.25
    blocks.append(b)
    blocks.append(np.linspace(-1.0, 1.0 - 2 ** -20, 32).astype(np.float32))
    src = np.concatenate(blocks)
    n = len(blocks)
    got = quant.execute(src, n, 32, 0, 1)
    exp = ref.quantize_q8_0_rows(src, n, 32, 0, 1)
    assert np.array_equal(got, exp)


def test_prefill_activation_size_and_round_trip(quant):
    """512 x 4096 activations (BASELINE config 4 X): byte-exact, and the
    dequantised values lie within half a quantisation step (plus the fp16
    rounding of d) of the source."""
    T, K = 512, 4096
    src = synth.normal_f32(synth.seed(4, 9), T * K)
    got = quant.execute(src, T, K, 0, K // 32)
    assert np.array_equal(got, ref.quantize_q8_0_rows(src, T, K, 0, K // 32))
    back = rn.dequant_q8_0(got)
    v = src.reshape(-1, 32)
    amax = np.max(np.abs(v), axis=1, keepdims=True)
    step = amax / 127.0
    err = np.abs(back.reshape(-1, 32) - v)
    assert np.all(err <= 0.5 * step * (1 + 2e-3) + amax * 1e-3)


def test_bounds_are_checked(ctx, quant):
    sb, db = ctx.alloc(4 * 64), ctx.alloc(34)
    try:
        with pytest.raises(EncodingFailed):          # destination holds one block, two needed
            quant.encode(None, sb, db, 2, 32, 0, 1)
        with pytest.raises(EncodingFailed):          # source holds 64 floats, 96 needed
            quant.encode(None, sb, db, 1, 32, 0, 3)
        quant.encode(None, sb, db, 0, 32, 0, 1)      # nothing to do
    finally:
        sb.free()
        db.free()
