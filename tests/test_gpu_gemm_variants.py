"""Every prefill GEMM kernel through contexts that force it: the
warp-specialised kernel at each K split (ER_HIP_GEMM_TILE=128:sk, 1 to 8 ways,
split-K summing with fp32 atomics into a zero-filled Y), the loader-specialised
kernel with 256- and 128-row tiles on shapes whose tiles alone would not select
it (ER_HIP_GEMM_VARIANT=4 / 5: partial token and weight-row tiles, one token
tile of 33 rows, K = 768, an odd count of Q4_K super-blocks cycling the
kernel's header slots, and K = 256, fewer weight chunks than the kernel's
copy-ahead depth), and the
earlier kernels kept for comparison (=1 single-stage, =2 pipelined, =3
warp-specialised).  Same bars as test_gpu_gemm.py: <= 1e-5 relative L2
against the float64 product with the bf16-rounded dequantised weights (the
kernels' own arithmetic) and <= 1e-2 against the CPU oracle."""
import os

import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import Context, QuantGEMMKernel
from oracle import ref
from oracle import restate_np as rn
from conftest import rel_l2
from test_gpu_gemm import DSCALE, bf16_round, bf16_to_f32

pytestmark = pytest.mark.gpu


def _gemm(**env):
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        c = Context(int(os.environ.get("ER_DEVICE", "0")))
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    return c, QuantGEMMKernel(c)


CONFIGS = [{"ER_HIP_GEMM_TILE": f"128:{sk}"} for sk in (1, 2, 3, 4, 8)] + \
          [{"ER_HIP_GEMM_VARIANT": v} for v in ("1", "2", "3", "4", "5")]


@pytest.mark.parametrize("env", CONFIGS, ids=lambda e: ",".join(f"{k}={v}" for k, v in e.items()))
@pytest.mark.parametrize("fmt", ["q4_k", "q8_0"])
@pytest.mark.parametrize("T,N,K", [(200, 300, 4096), (384, 8192, 1024), (33, 520, 2048), (130, 700, 768),
                                   (130, 700, 256)])
def test_forced_kernel(env, fmt, T, N, K):
    c, gemm = _gemm(**env)
    try:
        W = synth.weights(fmt, synth.seed(47, 0), N, K, **DSCALE[fmt])
        X = synth.normal_bf16(synth.seed(47, 1), T * K)
        Y = gemm.execute(fmt, W, X, T, N, K)
    finally:
        c.close()
    Wd = rn.weights_f32(fmt, W, N, K)
    Xf = bf16_to_f32(X).reshape(T, K)
    exact = Xf.astype(np.float64) @ bf16_round(Wd).astype(np.float64).T
    assert rel_l2(Y, exact) < 1e-5
    rows = [0, T // 2, T - 1]
    oracle = np.stack([ref.gemv(fmt, W, Xf[t], N, K) for t in rows])
    assert rel_l2(Y[rows], oracle) < 1e-2
