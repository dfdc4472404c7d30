"""Fused Q4_K projections (one launch, one x read): dual, triple and the
gate/up GeGLU.  Reference cases of GEMVTests.swift:735-1105 restated (the
second and third matrices are the formula filler with qs bytes XOR 0x11 /
0x22), with the reference's tolerances (1e-4 absolute; 5e-3 for GeGLU,
GEMVTests.swift:851), plus the decode-chain shapes against the oracle (1e-3
relative L2) and bit-equality with the single-matrix launches."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from oracle import ref
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def xor_qs(W, v):
    W = W.copy().reshape(-1, 144)
    W[:, 16:] ^= v
    return W.reshape(-1)


def test_reference_dual(gemv):
    rows, K = 7, 512
    A = ref.make_q4k_weights(rows, K)
    B = xor_qs(ref.make_q4k_weights(rows, K), 0x11)
    x = (((np.arange(K) % 23) - 11) / 29.0).astype(np.float32)
    ya, yb = gemv.executeQ4KWeightsMulti([A, B], x, [rows, rows], K)
    assert np.max(np.abs(ya - ref.gemv("q4_k", A, x, rows, K))) < 1e-4
    assert np.max(np.abs(yb - ref.gemv("q4_k", B, x, rows, K))) < 1e-4


def test_reference_triple(gemv):
    K = 512
    A = ref.make_q4k_weights(6, K)
    B = xor_qs(ref.make_q4k_weights(3, K), 0x11)
    Cw = xor_qs(ref.make_q4k_weights(4, K), 0x22)
    x = (((np.arange(K) % 31) - 15) / 41.0).astype(np.float32)
    ys = gemv.executeQ4KWeightsMulti([A, B, Cw], x, [6, 3, 4], K)
    for y, W, m in zip(ys, (A, B, Cw), (6, 3, 4)):
        assert np.max(np.abs(y - ref.gemv("q4_k", W, x, m, K))) < 1e-4


def test_reference_geglu(gemv):
    rows, K = 7, 512
    G = ref.make_q4k_weights(rows, K)
    U = xor_qs(ref.make_q4k_weights(rows, K), 0x11)
    x = (((np.arange(K) % 23) - 11) / 29.0).astype(np.float32)
    y = gemv.executeQ4KWeightsMulti([G, U], x, [rows, rows], K, geglu=True)
    exp = ref.gelu_tanh(ref.gemv("q4_k", G, x, rows, K)) * ref.gemv("q4_k", U, x, rows, K)
    assert np.max(np.abs(y - exp)) < 5e-3


@pytest.mark.parametrize("rows,K", [((2048, 1024, 1024), 1024), ((3000, 17, 130), 2048),
                                    ((5, 9, 1), 256)])
def test_triple_shapes_match_oracle_and_single(gemv, rows, K):
    Ws = [synth.q4_k(synth.seed(50, i), m, K) for i, m in enumerate(rows)]
    x = synth.normal_f32(synth.seed(50, 9), K)
    ys = gemv.executeQ4KWeightsMulti(Ws, x, list(rows), K)
    for W, m, y in zip(Ws, rows, ys):
        assert rel_l2(y, ref.gemv("q4_k", W, x, m, K)) < 1e-3
        assert np.array_equal(y, gemv.executeQ4KWeights(W, x, m, K))


@pytest.mark.parametrize("M,K", [(3072, 1024), (10240, 2560), (33, 768),
                                 # 2M rows on the K-sliced kernels: 8, 4 and 2 rows per step
                                 (3000, 4096), (2560, 4096), (1100, 8192), (1100, 14336),
                                 # beyond the integer-dot kernels' 16384 weights: the fp32
                                 # pair kernel (encodeQ4KWeightsDualGeGLU takes any K % 256 == 0,
                                 # GEMVKernel.swift:930-976)
                                 (512, 16640), (37, 32768)])
def test_dual_and_geglu_shapes(gemv, M, K):
    G = synth.q4_k(synth.seed(51, 0), M, K)
    U = synth.q4_k(synth.seed(51, 1), M, K)
    x = synth.normal_f32(synth.seed(51, 2), K)
    yg, yu = gemv.executeQ4KWeightsMulti([G, U], x, [M, M], K)
    eg, eu = ref.gemv("q4_k", G, x, M, K), ref.gemv("q4_k", U, x, M, K)
    assert rel_l2(yg, eg) < 1e-3 and rel_l2(yu, eu) < 1e-3
    y = gemv.executeQ4KWeightsMulti([G, U], x, [M, M], K, geglu=True)
    assert rel_l2(y, ref.gelu_tanh(eg) * eu) < 1e-3
