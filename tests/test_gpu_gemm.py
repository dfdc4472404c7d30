"""Prefill GEMM parity: Y = X (bf16) . W^T over raw Q4_K / Q8_0 weights on the
matrix cores.  Shapes cover both kernels: the warp-specialised one (128-token
tiles whose K splits hold a multiple of 4 chunks: 256x256x2048, 200x300x4096,
384x8192x1024 and the BASELINE shapes) and the 256-thread pipelined one (the
rest), with partial token and weight-row tiles.  Bars: relative L2 <= 1e-2 against the CPU oracle (per-token GEMV
on bf16-widened X; the north-star bound for bf16-MFMA GEMM), and <= 1e-5
against a float64 product of X and the bf16-rounded dequantised weights --
the kernel's own arithmetic, which pins the MFMA operand and accumulator
layouts exactly."""
import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import EncodingFailed, InvalidMatrixShape, InvalidVectorShape, QuantGEMMKernel
from oracle import ref
from oracle import restate_np as rn
from conftest import rel_l2

pytestmark = pytest.mark.gpu

DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01}}


def bf16_round(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def bf16_to_f32(x):
    return (np.asarray(x, np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.fixture(scope="module")
def gemm(ctx):
    return QuantGEMMKernel(ctx)


def case(fmt, T, N, K, seed):
    W = synth.weights(fmt, synth.seed(40 + seed, 0), N, K, **DSCALE[fmt])
    X = synth.normal_bf16(synth.seed(40 + seed, 1), T * K)
    return W, X


def check(gemm, fmt, T, N, K, seed=0, rows=None):
    W, X = case(fmt, T, N, K, seed)
    Y = gemm.execute(fmt, W, X, T, N, K)
    Wd = rn.weights_f32(fmt, W, N, K)
    Xf = bf16_to_f32(X).reshape(T, K)
    sel = np.arange(T) if rows is None else np.asarray(rows)
    exact = Xf[sel].astype(np.float64) @ bf16_round(Wd).astype(np.float64).T
    assert rel_l2(Y[sel], exact) < 1e-5, "kernel arithmetic (bf16 W, fp32 sums)"
    oracle = np.stack([ref.gemv(fmt, W, Xf[t], N, K) for t in sel])
    err = rel_l2(Y[sel], oracle)
    print(f"{fmt} T={T} N={N} K={K}: rel_l2 vs oracle {err:.2e}")
    assert err < 1e-2
    return Y


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0"])
@pytest.mark.parametrize("T,N,K", [(128, 128, 256), (1, 128, 512), (37, 100, 1024), (200, 300, 768),
                                   (256, 256, 2048), (300, 130, 1280), (200, 300, 4096), (384, 8192, 1024)])
def test_shapes(gemm, fmt, T, N, K):
    if fmt == "q4_k" and K % 256:
        pytest.skip("Q4_K needs K % 256 == 0")
    check(gemm, fmt, T, N, K)


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0"])
def test_q8_0_small_k(gemm, fmt):
    if fmt == "q8_0":
        check(gemm, fmt, 64, 96, 64)


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0"])
@pytest.mark.parametrize("N", [4096, 14336])
def test_baseline_shapes_sampled(gemm, fmt, N):
    """T = 512 tokens, K = 4096; every column of a sample of
    token rows (first, last, tile edges, seeded random) against the oracle."""
    T, K = 512, 4096
    rng = np.random.default_rng(N)
    rows = sorted(set([0, 1, 127, 128, 255, 256, 511]) | set(rng.integers(0, T, 9).tolist()))
    check(gemm, fmt, T, N, K, seed=1, rows=rows)


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0"])
@pytest.mark.parametrize("N", [4096, 14336])
def test_baseline_shapes_every_row(gemm, fmt, N):
    """BASELINE config 4 at full size, every one of the 512 token rows: against
    the float64 product of X and the bf16-rounded dequantised weights (the
    kernel's own arithmetic, <= 1e-5 relative L2 over all of Y and per row
    <= 1e-4) and against the oracle's per-token GEMV (<= 1e-2 relative L2)."""
    T, K = 512, 4096
    W, X = case(fmt, T, N, K, 2)
    Y = gemm.execute(fmt, W, X, T, N, K)
    Xf = bf16_to_f32(X).reshape(T, K)
    exact = Xf.astype(np.float64) @ bf16_round(rn.weights_f32(fmt, W, N, K)).astype(np.float64).T
    assert rel_l2(Y, exact) < 1e-5
    per_row = np.linalg.norm(Y - exact, axis=1) / np.maximum(np.linalg.norm(exact, axis=1), 1e-30)
    assert per_row.max() < 1e-4, int(per_row.argmax())
    oracle = ref.gemm(fmt, W, X, T, N, K, threads=ref.max_threads()).reshape(T, N)
    err = rel_l2(Y, oracle)
    print(f"{fmt} 512x{N}x4096 all rows: rel_l2 vs oracle {err:.2e}")
    assert err < 1e-2


@pytest.mark.parametrize("fmt", ["q4_k", "q8_0"])
def test_unsplit_gemm_is_deterministic(gemm, fmt):
    """Shapes that run without a K split (no fp32 atomics) give bit-identical Y
    on every call; split-K shapes add their partial tiles with atomics in an
    order that varies, so only those may differ in the last bits."""
    T, N, K = 512, 14336, 1024
    W, X = case(fmt, T, N, K, 3)
    first = gemm.execute(fmt, W, X, T, N, K)
    for _ in range(3):
        assert np.array_equal(gemm.execute(fmt, W, X, T, N, K).view(np.uint32), first.view(np.uint32))


def test_one_hot_tokens_extract_weight_rows(gemm):
    """X = identity rows: Y[t] is column t of the dequantised (bf16-rounded) W."""
    T, N, K = 256, 64, 256
    W = synth.q4_k(synth.seed(45, 0), N, K)
    eye = np.zeros((T, K), np.float32)
    eye[np.arange(T), np.arange(T)] = 1.0
    X = (eye.view(np.uint32) >> 16).astype(np.uint16)
    Y = gemm.execute("q4_k", W, X, T, N, K)
    Wd = bf16_round(rn.weights_f32("q4_k", W, N, K))
    assert np.array_equal(Y, Wd.T)


def test_validation(ctx, gemm):
    N, K, T = 8, 512, 4
    W = synth.q4_k(1, N, K)
    X = synth.normal_bf16(2, T * K)
    with pytest.raises(InvalidVectorShape):
        gemm.execute("q4_k", W, synth.normal_bf16(2, T * 384), T, N, 384)
    with pytest.raises(InvalidMatrixShape):
        gemm.execute("q4_k", W[:-1], X, T, N, K)
    wb, xb, yb = ctx.upload(W), ctx.upload(X), ctx.alloc(T * N * 4 - 4)
    with pytest.raises(EncodingFailed):
        gemm.encodeQ4K(None, wb, xb, yb, T, N, K)
    with pytest.raises(InvalidVectorShape):
        gemm.encodeQ8_0(None, wb, xb, ctx.alloc(T * N * 4), T, N, 96)


@pytest.mark.parametrize("fmt,T,N,items", [("q4_k", 512, 4096, 128), ("q8_0", 512, 14336, 224)])
def test_clock_probe(ctx, gemm, fmt, T, N, items):
    """er_hip_probe_gemm_clock (the measurement library) runs a stamped copy
    of the product kernel: Y is bit-identical to the product library's call,
    one stamp set per work item (128-row tiles at N = 4096, 256-row tiles at
    14336), each with both counters advancing and a clock between 100 MHz and
    3.5 GHz.  Buffers of the product context pass to the measurement
    library's context (plain device memory)."""
    import ctypes as C
    from edgerunner_amd import Context
    K = 1024
    W, X = case(fmt, T, N, K, 5)
    want = gemm.execute(fmt, W, X, T, N, K)
    pctx = Context(ctx.info.device, probes=True)
    lib = pctx.lib
    typ = 12 if fmt == "q4_k" else 8
    wb, xb, yb = ctx.upload(W), ctx.upload(X), ctx.alloc(4 * T * N)
    stamps = ctx.alloc(32 * items)
    n = C.c_uint32(0)
    try:
        assert lib.er_hip_probe_gemm_clock(pctx.handle, None, typ, wb.raw, xb.raw, yb.raw, T, N, K, stamps.raw,
                                           C.byref(n)) == 0
        ctx.synchronize()
        assert n.value == items
        assert np.array_equal(yb.download(np.float32).view(np.uint32), want.reshape(-1).view(np.uint32))
        s = stamps.download(np.uint64).reshape(-1, 4)
        assert np.all(s[:, 1] > s[:, 0]) and np.all(s[:, 3] > s[:, 2])
        mhz = (s[:, 3] - s[:, 2]).astype(np.float64) / (s[:, 1] - s[:, 0]).astype(np.float64) * 100.0
        print(f"{fmt} {T}x{N}x{K}: workgroups at {np.median(mhz):.0f} MHz (min {mhz.min():.0f})")
        assert np.all((mhz > 100.0) & (mhz < 3500.0))
        # too few stamps, a shape the kernel does not take, a format without it
        small = ctx.alloc(32 * items - 8)
        try:
            assert lib.er_hip_probe_gemm_clock(pctx.handle, None, typ, wb.raw, xb.raw, yb.raw, T, N, K, small.raw,
                                               C.byref(n)) != 0
        finally:
            small.free()
        assert lib.er_hip_probe_gemm_clock(pctx.handle, None, typ, wb.raw, xb.raw, yb.raw, 33, 64, K, stamps.raw,
                                           C.byref(n)) != 0
        assert lib.er_hip_probe_gemm_clock(pctx.handle, None, 14, wb.raw, xb.raw, yb.raw, T, N, K, stamps.raw,
                                           C.byref(n)) != 0
    finally:
        for b in (wb, xb, yb, stamps):
            b.free()
        pctx.close()
