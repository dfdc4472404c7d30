"""Golden fixtures (tests/golden/reference_cases.npz): the reference tests'
own inputs with recorded oracle outputs.  CPU: the oracle and the independent
numpy statement reproduce them exactly.  GPU: the HIP kernels match them to the
reference tests' tolerances (absolute 1e-4 for K-quant GEMV, GEMVTests.swift
:475-477; relative 2% per row for Q8_0, FusedKernelTests.swift:122-125) and to
1e-3 relative L2; dequantisation bit-exact."""
import numpy as np
import pytest

from golden_cases import load
from oracle import ref
from oracle import restate_np as rn
from conftest import rel_l2

GEMV, DEQ = load()


@pytest.mark.parametrize("name", sorted(GEMV))
def test_oracle_reproduces_gemv_fixture(name):
    c = GEMV[name]
    M, K, T = (int(v) for v in c["shape"])
    y = ref.gemv(c["fmt"], c["W"], c["x"], M, K, tokens=T)
    assert np.array_equal(y.view(np.uint32), c["y"].view(np.uint32))


@pytest.mark.parametrize("name", sorted(GEMV))
def test_fixture_against_float64(name):
    c = GEMV[name]
    M, K, T = (int(v) for v in c["shape"])
    tol = 2e-4 if T > 1 else 1e-4  # the reference's batched bound, GEMVTests.swift:510
    for t in range(T):
        y64 = rn.gemv_f64(c["fmt"], c["W"], c["x"][t * K:(t + 1) * K], M, K).ravel()
        assert np.max(np.abs(c["y"][t * M:(t + 1) * M] - y64)) < tol


@pytest.mark.parametrize("name", sorted(DEQ))
def test_dequant_fixture_bit_exact(name):
    c = DEQ[name]
    got = ref.dequant(c["fmt"], c["blocks"])
    assert np.array_equal(got.view(np.uint32), c["values"].view(np.uint32))
    npv = {"q8_0": rn.dequant_q8_0, "q4_k": rn.dequant_q4_k, "q6_k": rn.dequant_q6_k}[c["fmt"]]
    assert np.array_equal(np.asarray(npv(c["blocks"]), np.float32).view(np.uint32),
                          c["values"].view(np.uint32))


EXEC = {"q8_0": "executeQ8_0Weights", "q4_k": "executeQ4KWeights", "q6_k": "executeQ6KWeights"}
EXEC_B = {"q8_0": "executeBatchedQ8_0Weights", "q4_k": "executeBatchedQ4KWeights",
          "q6_k": "executeBatchedQ6KWeights"}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(GEMV))
def test_gpu_gemv_matches_fixture(gemv, name):
    c = GEMV[name]
    M, K, T = (int(v) for v in c["shape"])
    if T == 1:
        y = getattr(gemv, EXEC[c["fmt"]])(c["W"], c["x"], M, K)
    else:
        y = getattr(gemv, EXEC_B[c["fmt"]])(c["W"], c["x"], T, M, K)
    exp = c["y"]
    assert rel_l2(y, exp) < 1e-3
    if c["fmt"] == "q8_0":
        assert np.all(np.abs(y - exp) / np.maximum(np.abs(exp), 1e-6) < 0.02)
    else:
        assert np.max(np.abs(y - exp)) < (2e-4 if T > 1 else 1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(DEQ))
def test_gpu_dequant_matches_fixture(ctx, name):
    from edgerunner_amd import DequantQ4KMKernel, DequantQ6KKernel, DequantQ8_0Kernel
    c = DEQ[name]
    k = {"q8_0": DequantQ8_0Kernel, "q4_k": DequantQ4KMKernel, "q6_k": DequantQ6KKernel}[c["fmt"]](ctx)
    bb = {"q8_0": 34, "q4_k": 144, "q6_k": 210}[c["fmt"]]
    got = k.dequantise(c["blocks"], c["blocks"].size // bb)
    assert np.array_equal(got.view(np.uint32), c["values"].view(np.uint32))
