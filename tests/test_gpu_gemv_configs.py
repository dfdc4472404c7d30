"""Every lane-group (int8-limb) GEMV configuration, forced through
ER_HIP_GEMV_CONFIG=lpr:ns:r in a context of its own.  The row length makes
some lanes use all NS slots; the row count (203) leaves a partial last
workgroup.  Q4_K, Q6_K and Q8_0 against the CPU oracle at the parity bar
(relative L2 <= 1e-3), and the Q6_K top-1 index against the selection rule
on the same context's logits.  The host's own picker reaches only some of
these kernels at the benchmark shapes; this covers the rest."""
import os

import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import Context, GEMVKernel
from oracle import ref
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-3
EXEC = {"q8_0": "executeQ8_0Weights", "q4_k": "executeQ4KWeights", "q6_k": "executeQ6KWeights"}
DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01},
          "q6_k": {"dscale": 0.005}}
MAX_K = 16384  # longest row the lane-group family takes

# (slots per lane, row computations per lane group), per lanes-per-row value
NS_R = [(1, 4), (1, 2), (1, 1), (2, 4), (2, 2), (2, 1), (3, 2), (3, 1), (4, 2), (4, 1), (5, 1), (6, 1),
        (7, 1), (8, 1)]


def row_length(lpr: int, ns: int):
    """Smallest multiple of 256 with more than lpr * (ns - 1) 64-weight slots,
    or None when no such row fits the family."""
    slots = -(-(lpr * (ns - 1) + 1) // 4) * 4
    K = 64 * slots
    return K if K <= MAX_K and slots <= lpr * ns else None


CONFIGS = [(l, n, r) for l in (64, 32, 16, 4) for n, r in NS_R if row_length(l, n) is not None]


@pytest.mark.parametrize("lpr,ns,r", CONFIGS)
def test_forced_lane_group_config(lpr, ns, r):
    K, M = row_length(lpr, ns), 203
    old = os.environ.get("ER_HIP_GEMV_CONFIG")
    os.environ["ER_HIP_GEMV_CONFIG"] = f"{lpr}:{ns}:{r}"
    try:
        ctx = Context(int(os.environ.get("ER_DEVICE", "0")))
    finally:
        if old is None:
            os.environ.pop("ER_HIP_GEMV_CONFIG", None)
        else:
            os.environ["ER_HIP_GEMV_CONFIG"] = old
    try:
        gemv = GEMVKernel(ctx)
        x = synth.normal_f32(synth.seed(90, K % 97), K)
        for fmt in ("q4_k", "q6_k", "q8_0"):
            W = synth.weights(fmt, synth.seed(90, lpr * 100 + ns * 10 + r), M, K, **DSCALE[fmt])
            y = getattr(gemv, EXEC[fmt])(W, x, M, K)
            exp = ref.gemv(fmt, W, x, M, K, threads=ref.max_threads())
            assert rel_l2(y, exp) < TOL, (fmt, lpr, ns, r, K)
        M4 = 204  # top-1 needs M % 4 == 0
        W = synth.weights("q6_k", synth.seed(91, lpr * 100 + ns * 10 + r), M4, K, dscale=0.005)
        y = gemv.executeQ6KWeights(W, x, M4, K)
        assert gemv.executeQ6KWeightsTop1(W, x, M4, K) == ref.top1(y), (lpr, ns, r, K)
    finally:
        ctx.close()
