"""The allocation-free Q6_K top-1 (er_hip_encode_q6k_weights_packed_top1_noalloc,
partials in the library's own device scratch array) called through the C
ABI, against the caller-scratch entry point er_hip_encode_q6k_weights_packed_top1
on the same inputs: the row index must be identical (integer result, exact).
Two calls in a row on one context, the second over a smaller head (fewer
partials, a different kernel family), so the second reads none of the first
call's scratch contents, then a third in the fp32 family.  The rejection of
heads past the array's size needs no device and is tested on the CPU
(tests/test_abi.py)."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import _ffi
from oracle import ref

pytestmark = pytest.mark.gpu

MAX_ROWS = 262144


def _top1_both(ctx, M, K, seed):
    lib = _ffi.load()
    W = synth.q6_k(synth.seed(95, seed), M, K, dscale=0.005)
    x = synth.normal_f32(synth.seed(95, seed + 1), K)
    wb, xb = ctx.upload(W), ctx.upload(x)
    n = max(1, M // 4)
    pv, pi = ctx.alloc(4 * n), ctx.alloc(4 * n)
    out_a, out_b = ctx.alloc(4), ctx.alloc(4)
    try:
        st = lib.er_hip_encode_q6k_weights_packed_top1(ctx.handle, None, wb.raw, xb.raw, pv.raw, pi.raw,
                                                       out_a.raw, M, K)
        assert st == 0, _ffi.last_error()
        st = lib.er_hip_encode_q6k_weights_packed_top1_noalloc(ctx.handle, None, wb.raw, xb.raw, out_b.raw, M, K)
        assert st == 0, _ffi.last_error()
        assert lib.er_hip_synchronize(ctx.handle, None) == 0
        a = int(out_a.download(np.uint32, 1)[0])
        b = int(out_b.download(np.uint32, 1)[0])
    finally:
        for buf in (wb, xb, pv, pi, out_a, out_b):
            buf.free()
    return a, b, W, x


def test_noalloc_top1_matches_caller_scratch_twice(ctx):
    # 151936 x 1024: the CU-resident kernel; 2048 x 1024: the lane-group kernel;
    # 1024 x 16640: the fp32 family (rows beyond the integer-dot kernels)
    for M, K, seed in ((151936, 1024, 1), (2048, 1024, 3), (1024, 16640, 5)):
        print(f"[no-alloc] top-1 M={M} K={K}", flush=True)
        a, b, W, x = _top1_both(ctx, M, K, seed)
        assert a == b, (M, K, a, b)
        if M <= 4096:
            assert b == ref.top1(ref.gemv("q6_k", W, x, M, K))
