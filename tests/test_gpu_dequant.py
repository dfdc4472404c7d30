"""Dequantisation on the GPU is bit-identical to the CPU oracle
(DequantQ*Tests.swift cases + seeded synthetic blocks + special values)."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import (DequantQ4KMKernel, DequantQ6KKernel, DequantQ8_0Kernel,
                            InvalidBlockDataCount)
from oracle import ref

pytestmark = pytest.mark.gpu

KERNELS = {"q8_0": DequantQ8_0Kernel, "q4_k": DequantQ4KMKernel, "q6_k": DequantQ6KKernel}
PER = {"q8_0": 32, "q4_k": 256, "q6_k": 256}


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k"])
def test_reference_patterns(ctx, fmt):
    k = KERNELS[fmt](ctx)
    n = PER[fmt]
    pats = [np.arange(n) * (0.1 if fmt == "q8_0" else 0.01) - (1.6 if fmt == "q8_0" else 1.28)]
    if fmt == "q8_0":
        pats += [((b * 31 + np.arange(32)) % 19 - 9) * 0.22 for b in range(32)]
    else:
        pats += [((b * 17 + np.arange(256)) % 29 - 14) * 0.14 for b in range(8)]
    blocks = np.concatenate([ref.pack_block(fmt, np.asarray(p, np.float32)) for p in pats])
    got = k.dequantise(blocks, len(pats))
    assert same_bits(got, ref.dequant(fmt, blocks))
    zero = ref.pack_block(fmt, np.zeros(n, np.float32))
    assert np.all(k.dequantise(zero, 1) == 0)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("nblocks", [1, 3, 257, 40001])
def test_synthetic_blocks(ctx, fmt, nblocks):
    per = PER[fmt]
    K = per
    W = synth.weights(fmt, synth.seed(20, nblocks % 16), nblocks, K)
    got = KERNELS[fmt](ctx).dequantise(W, nblocks)
    assert same_bits(got, ref.dequant(fmt, W))


@pytest.mark.parametrize("fmt", ["q8_0", "q4_k", "q6_k"])
def test_random_bytes_and_special_scales(ctx, fmt):
    """Arbitrary bytes: every fp16 scale pattern incl. subnormals, zeros,
    negative scales, infinities and NaNs."""
    bb = {"q8_0": 34, "q4_k": 144, "q6_k": 210}[fmt]
    rng = np.random.default_rng(99)
    n = 4096
    blocks = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    dpos = {"q8_0": [0], "q4_k": [0, 2], "q6_k": [208]}[fmt]
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x8001, 0x0400, 0x7BFF, 0x7C00, 0xFC00,
                         0x7E00, 0x3C00, 0xBC00], dtype=np.uint16)
    for i, s in enumerate(specials):
        for p in dpos:
            blocks[i, p] = s & 0xFF
            blocks[i, p + 1] = s >> 8
    got = KERNELS[fmt](ctx).dequantise(blocks, n)
    exp = ref.dequant(fmt, blocks)
    fin = np.isfinite(exp)
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    assert same_bits(got[fin], exp[fin])
    assert np.array_equal(got[np.isinf(exp)], exp[np.isinf(exp)])


def test_full_size_q4k_bit_exact(ctx):
    """BASELINE config 2 weight tensor (14336 x 4096 Q4_K), every value."""
    M, K = 14336, 4096
    W = synth.q4_k(synth.seed(2, 0), M, K)
    got = DequantQ4KMKernel(ctx).dequantise(W, M * K // 256)
    assert same_bits(got, ref.dequant("q4_k", W))


def test_block_count_mismatch_raises(ctx):
    with pytest.raises(InvalidBlockDataCount) as e:
        DequantQ4KMKernel(ctx).dequantise(np.zeros(144 * 2 + 1, np.uint8), 2)
    assert e.value.expected == 288 and e.value.actual == 289
