#!/usr/bin/env python3
"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline (BASELINE.json `metric`, configs[1]): Q4_K decode GEMV at
14336x4096, reported as achieved HBM GB/s = algorithmic bytes per call
(W + x + y, the reference's formula, GEMVTests.swift:1438-1440) / average
launch duration.  One step = one GEMV call over one of >= 768 MB of distinct
weight copies, with x and y resident in HBM.  The `--steps` launches are
recorded into a HIP graph and replayed; HIP events on the launch stream
bracket the replay (after `--warmup` untimed launches and UNTIMED_REPLAYS
untimed replays, which let the clocks and the graph's first-launch work
settle; the timed replay is queued behind one more untimed graph, so the
start event is not stamped while the host is still submitting the graph to
an idle GPU).  With fewer steps than copies, the calls over the remaining copies
run untimed before each replay (rotation_time_us), so at any --steps every
timed call reads weights that >= 768 MB of other reads have pushed out of the
256 MB Infinity Cache; each result reports its copies, timed launches and the
distinct bytes one such cycle reads.

Also reported in `results`: the other BASELINE GEMV shapes (Q8_0 3072x1024 and
14336x4096, Q4_K 4096x14336, Q6_K 151936x1024 and 128256x4096), the Q6_K
top-1 heads, the Q8_0 row quantizer, the dequantisation of the 14336x4096
matrix in each format, the fused projections at Llama-3-8B shapes (Q4_K
triple / dual / dual GeGLU, Q8_0 RMSNorm + QKV and RMSNorm + gate-up-SiLU),
the prefill GEMMs, the GGUF upload, the decode chain and the ceilings.

The cpu_baseline leg times the CPU oracle (a C restatement of the reference's
Swift CPU dequant+dot loop, oracle/er_oracle.c) on a bounded sample of the
same workload on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "quant GEMV achieved HBM GB/s (% of 8 TB/s) at 14336x4096; prefill GEMM TFLOP/s"
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 768 << 20
UNTIMED_REPLAYS = 3  # graph replays before the timed one

BLOCK = {"q8_0": (34, 32), "q4_k": (144, 256), "q6_k": (210, 256)}
ENCODE = {"q8_0": "encodeQ8_0Weights", "q4_k": "encodeQ4KWeights", "q6_k": "encodeQ6KWeights"}
KERNEL_PREFIX = {"q8_0": "er_gemv_q8_0", "q4_k": "er_gemv_q4k", "q6_k": "er_gemv_q6k"}
DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01},
          "q6_k": {"dscale": 0.005}}

# (name, fmt, M, K, BASELINE config index)
GEMV_WORKLOADS = [
    ("q4_k_gemv_14336x4096", "q4_k", 14336, 4096, 2),
    ("q4_k_gemv_4096x14336", "q4_k", 4096, 14336, 2),
    ("q8_0_gemv_14336x4096", "q8_0", 14336, 4096, 1),
    ("q8_0_gemv_3072x1024", "q8_0", 3072, 1024, 1),
    ("q6_k_gemv_151936x1024", "q6_k", 151936, 1024, 3),
    ("q6_k_gemv_128256x4096", "q6_k", 128256, 4096, 3),
]


# Greedy top-1 heads: (name, M, K, BASELINE config index)
TOP1_WORKLOADS = [
    ("q6_k_top1_151936x1024", 151936, 1024, 3),
    ("q6_k_top1_128256x4096", 128256, 4096, 3),
]

# Q8_0 row quantizer: (name, rows, row length, BASELINE config index)
QUANT_WORKLOADS = [
    ("q8_0_quantize_512x4096", 512, 4096, 4),
    ("q8_0_quantize_8192x4096", 8192, 4096, 4),
]

# Dequantisation to fp32 of the headline matrix in each format: (name, fmt,
# M, K, BASELINE config index of the format's synthetic weights)
DEQUANT_WORKLOADS = [
    ("q8_0_dequant_14336x4096", "q8_0", 14336, 4096, 1),
    ("q4_k_dequant_14336x4096", "q4_k", 14336, 4096, 2),
    ("q6_k_dequant_14336x4096", "q6_k", 14336, 4096, 3),
]

# Fused projections at Llama-3-8B shapes (hidden 4096, q 4096, kv 1024, FFN
# 14336; the BASELINE GEMV shapes): (name, kind, fmt, rows of each matrix, K,
# BASELINE config index of the format's synthetic weights).  Kinds: the Q4_K
# triple / dual / dual GeGLU entries, and the Q8_0 RMSNorm + QKV (fp16 V) and
# RMSNorm + gate-up-SiLU pipelines, one token each.
FUSED_WORKLOADS = [
    ("q4_k_triple_4096+1024+1024x4096", "triple", "q4_k", (4096, 1024, 1024), 4096, 2),
    ("q4_k_dual_2x14336x4096", "dual", "q4_k", (14336, 14336), 4096, 2),
    ("q4_k_dual_geglu_2x14336x4096", "geglu", "q4_k", (14336, 14336), 4096, 2),
    ("q8_0_fused_qkv_4096+1024+1024x4096", "qkv", "q8_0", (4096, 1024, 1024), 4096, 1),
    ("q8_0_fused_gate_up_silu_2x14336x4096", "silu", "q8_0", (14336, 14336), 4096, 1),
]

# (name, fmt, T tokens, N, K, BASELINE config index)
GEMM_WORKLOADS = [
    ("q4_k_gemm_512x4096x4096", "q4_k", 512, 4096, 4096, 4),
    ("q4_k_gemm_512x14336x4096", "q4_k", 512, 14336, 4096, 4),
    ("q8_0_gemm_512x4096x4096", "q8_0", 512, 4096, 4096, 4),
    ("q8_0_gemm_512x14336x4096", "q8_0", 512, 14336, 4096, 4),
]
MFMA_BF16_PEAK_TFLOPS = 2500.0
PEAK_SCLK_MHZ = 2400.0  # the engine clock the MFMA peak is quoted at
CLOCK_LAUNCHES = 5      # back-to-back stamped GEMM launches per workload; the last one is read


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def weight_bytes(fmt: str, M: int, K: int) -> int:
    bb, bw = BLOCK[fmt]
    return M * (K // bw) * bb


def algorithmic_bytes(fmt: str, M: int, K: int) -> int:
    return weight_bytes(fmt, M, K) + 4 * K + 4 * M


def gemm_min_bytes(fmt: str, T: int, N: int, K: int) -> int:
    """Least HBM traffic of one prefill GEMM: W once, X (bf16) once, Y (fp32) written once."""
    return weight_bytes(fmt, N, K) + 2 * T * K + 4 * T * N


def bench_gemv(ctx, fmt: str, M: int, K: int, cfg: int, steps: int, warmup: int) -> dict:
    """Times `steps` GEMV launches over rotating weight copies.  The launches
    are recorded once into a HIP graph and replayed, so the events bracket
    GPU work only (no Python launch overhead); the eager, Python-launched
    rate is reported alongside."""
    import edgerunner_amd.synth as synth
    from edgerunner_amd import GEMVKernel

    gemv = GEMVKernel(ctx)
    W = synth.weights(fmt, synth.seed(cfg, 0), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(cfg, 1), K)
    copies = max(2, -(-ROTATE_BYTES // W.nbytes))
    stream = ctx.stream()
    wbufs = [ctx.upload(W, stream) for _ in range(copies)]
    xb = ctx.upload(x, stream)
    yb = ctx.alloc(4 * M)
    enc = getattr(gemv, ENCODE[fmt])
    for i in range(warmup):
        enc(stream, wbufs[i % copies], xb, yb, M, K)
    stream.synchronize()
    avg_us = rotation_time_us(ctx, stream, lambda i: enc(stream, wbufs[i % copies], xb, yb, M, K), steps, copies)
    ms = avg_us * steps / 1000.0
    # eager: Python-launched back-to-back (includes host launch cost), from
    # the cold cache state rotation_time_us leaves
    e0, e1 = ctx.event(), ctx.event()
    e0.record(stream)
    for i in range(steps):
        enc(stream, wbufs[i % copies], xb, yb, M, K)
    e1.record(stream)
    stream.synchronize()
    eager_us = e0.elapsed_ms(e1) * 1000.0 / steps
    nbytes = algorithmic_bytes(fmt, M, K)
    y = yb.download(np.float32, stream=stream)
    for b in wbufs:
        b.free()
    xb.free()
    yb.free()
    e0.destroy()
    e1.destroy()
    stream.destroy()
    return {
        "fmt": fmt, "M": M, "K": K, **rotation_fields(copies, W.nbytes, steps), "bytes_per_call": nbytes,
        "us_per_call": avg_us, "GBps": nbytes / (avg_us * 1e-6) / 1e9,
        "frac_of_hbm_peak": nbytes / (avg_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        "us_per_call_eager": eager_us,
        "ms_total": ms, "y_finite": bool(np.all(np.isfinite(y))),
    }


def bench_top1(ctx, M: int, K: int, cfg: int, steps: int, warmup: int) -> dict:
    """Q6_K head with fused greedy top-1 (GEMV + partial epilogue, then the
    one-workgroup reduce): `steps` calls over rotating weight copies in a HIP
    graph, as bench_gemv.  Bytes per call: W + x + the 4-byte index."""
    import edgerunner_amd.synth as synth
    from edgerunner_amd import GEMVKernel

    gemv = GEMVKernel(ctx)
    W = synth.weights("q6_k", synth.seed(cfg, 0), M, K, **DSCALE["q6_k"])
    x = synth.normal_f32(synth.seed(cfg, 1), K)
    copies = max(2, -(-ROTATE_BYTES // W.nbytes))
    stream = ctx.stream()
    wbufs = [ctx.upload(W, stream) for _ in range(copies)]
    xb = ctx.upload(x, stream)
    n = gemv.q6KTop1PartialCount(M)
    pv, pi, ob = ctx.alloc(4 * n), ctx.alloc(4 * n), ctx.alloc(4)

    def enc(i):
        gemv.encodeQ6KWeightsPackedTop1(stream, wbufs[i % copies], xb, pv, pi, ob, M, K)

    for i in range(warmup):
        enc(i)
    stream.synchronize()
    avg_us = rotation_time_us(ctx, stream, enc, steps, copies)
    nbytes = weight_bytes("q6_k", M, K) + 4 * K + 4
    idx = int(ob.download(np.uint32, 1, stream=stream)[0])
    for b in wbufs + [xb, pv, pi, ob]:
        b.free()
    stream.destroy()
    return {"M": M, "K": K, **rotation_fields(copies, W.nbytes, steps), "bytes_per_call": nbytes,
            "us_per_call": avg_us,
            "GBps": nbytes / (avg_us * 1e-6) / 1e9,
            "frac_of_hbm_peak": nbytes / (avg_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "launches_per_call": 2, "index": idx}


def bench_quant(ctx, rows: int, K: int, cfg: int, steps: int, warmup: int) -> dict:
    """Q8_0 row quantizer over `rows` fp32 rows of K values, rotating source
    copies, in a HIP graph.  Bytes per call: 4 per value read + 34 per block
    written."""
    import edgerunner_amd.synth as synth
    from edgerunner_amd import QuantizeQ8RowsKernel

    qk = QuantizeQ8RowsKernel(ctx)
    src = synth.normal_f32(synth.seed(cfg, 9), rows * K)
    copies = max(2, -(-ROTATE_BYTES // src.nbytes))
    stream = ctx.stream()
    sbufs = [ctx.upload(src, stream) for _ in range(copies)]
    db = ctx.alloc(rows * (K // 32) * 34)
    for i in range(warmup):
        qk.encode(stream, sbufs[i % copies], db, rows, K, 0, K // 32)
    stream.synchronize()
    avg_us = rotation_time_us(ctx, stream, lambda i: qk.encode(stream, sbufs[i % copies], db, rows, K, 0, K // 32),
                              steps, copies)
    nbytes = rows * K * 4 + rows * (K // 32) * 34
    for b in sbufs + [db]:
        b.free()
    stream.destroy()
    return {"rows": rows, "K": K, **rotation_fields(copies, src.nbytes, steps), "bytes_per_call": nbytes,
            "us_per_call": avg_us,
            "GBps": nbytes / (avg_us * 1e-6) / 1e9,
            "frac_of_hbm_peak": nbytes / (avg_us * 1e-6) / 1e9 / HBM_PEAK_GBS}


DEQUANT_KERNELS = {"q8_0": "DequantQ8_0Kernel", "q4_k": "DequantQ4KMKernel", "q6_k": "DequantQ6KKernel"}


def dequant_bytes(fmt: str, M: int, K: int) -> int:
    """Least HBM traffic of one dequantisation: the blocks read once, fp32 written once."""
    return weight_bytes(fmt, M, K) + 4 * M * K


def bench_dequant(ctx, fmt: str, M: int, K: int, cfg: int, steps: int, warmup: int) -> dict:
    """Dequantisation of an M x K matrix to fp32 (er_hip_dequant_*), rotating
    block copies (>= 768 MB, so every call reads HBM), in a HIP graph.  Bytes
    per call: the blocks read + 4 per weight written."""
    import edgerunner_amd
    import edgerunner_amd.synth as synth

    kern = getattr(edgerunner_amd, DEQUANT_KERNELS[fmt])(ctx)
    W = synth.weights(fmt, synth.seed(cfg, 0), M, K, **DSCALE[fmt])
    count = M * K // BLOCK[fmt][1]
    copies = max(2, -(-ROTATE_BYTES // W.nbytes))
    stream = ctx.stream()
    wbufs = [ctx.upload(W, stream) for _ in range(copies)]
    out = ctx.alloc(4 * M * K)
    for i in range(warmup):
        kern.encode(stream, wbufs[i % copies], count, out)
    stream.synchronize()
    avg_us = rotation_time_us(ctx, stream, lambda i: kern.encode(stream, wbufs[i % copies], count, out), steps, copies)
    nbytes = dequant_bytes(fmt, M, K)
    for b in wbufs + [out]:
        b.free()
    stream.destroy()
    return {"fmt": fmt, "M": M, "K": K, **rotation_fields(copies, W.nbytes, steps), "bytes_per_call": nbytes,
            "us_per_call": avg_us, "GBps": nbytes / (avg_us * 1e-6) / 1e9,
            "frac_of_hbm_peak": nbytes / (avg_us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def fused_bytes(kind: str, fmt: str, rows, K: int) -> int:
    """Least HBM traffic of one fused call: every matrix once, x once (and
    the RMSNorm weight), the outputs once (fp16 V for the Q8_0 QKV; one
    activated vector for GeGLU / SiLU)."""
    w = sum(weight_bytes(fmt, M, K) for M in rows)
    if kind in ("triple", "dual"):
        out = 4 * sum(rows)
    elif kind in ("geglu", "silu"):
        out = 4 * rows[0]
    else:  # qkv
        out = 4 * (rows[0] + rows[1]) + 2 * rows[2]
    return w + 4 * K + out + (4 * K if fmt == "q8_0" else 0)


def fused_calls(ctx, stream, kind: str, fmt: str, rows, K: int, cfg: int):
    """Device buffers of one fused workload: rotating sets of its matrices
    (>= 768 MB), x, the RMSNorm weight and the outputs.  Returns (enc, copies,
    set_bytes, buffers): enc(i) encodes the call reading set i % copies."""
    import edgerunner_amd.synth as synth
    from edgerunner_amd import FusedQ8Kernel, GEMVKernel

    gemv, fq = GEMVKernel(ctx), FusedQ8Kernel(ctx)
    Ws = [synth.weights(fmt, synth.seed(cfg, 10 + i), M, K, **DSCALE[fmt]) for i, M in enumerate(rows)]
    set_bytes = sum(W.nbytes for W in Ws)
    copies = max(2, -(-ROTATE_BYTES // set_bytes))
    sets = [[ctx.upload(W, stream) for W in Ws] for _ in range(copies)]
    xb = ctx.upload(synth.normal_f32(synth.seed(cfg, 1), K), stream)
    norm = ctx.upload((1.0 + 0.1 * synth.normal_f32(synth.seed(cfg, 2), K)).astype(np.float32), stream)
    ys = [ctx.alloc(4 * M) for M in rows]
    eps = 1e-5

    def enc(i):
        w = sets[i % copies]
        if kind == "triple":
            gemv.encodeQ4KWeightsTriple(stream, *w, xb, *ys, *rows, K)
        elif kind == "dual":
            gemv.encodeQ4KWeightsDual(stream, *w, xb, *ys, rows[0], K)
        elif kind == "geglu":
            gemv.encodeQ4KWeightsDualGeGLU(stream, *w, xb, ys[0], rows[0], K)
        elif kind == "qkv":
            fq.encodeFusedQKV(stream, *w, xb, *ys, norm, rows[0], rows[1], K, 1, eps)
        else:  # silu
            fq.encodeFusedGateUpSilu(stream, *w, xb, ys[0], norm, rows[0], K, 1, eps)

    return enc, copies, set_bytes, [b for w in sets for b in w] + [xb, norm] + ys


def bench_fused(ctx, kind: str, fmt: str, rows, K: int, cfg: int, steps: int, warmup: int) -> dict:
    """One fused projection call (one x read for all its matrices) over
    rotating sets of its matrices (>= 768 MB), in a HIP graph."""
    stream = ctx.stream()
    enc, copies, set_bytes, bufs = fused_calls(ctx, stream, kind, fmt, rows, K, cfg)
    for i in range(warmup):
        enc(i)
    stream.synchronize()
    avg_us = rotation_time_us(ctx, stream, enc, steps, copies)
    finite = bool(np.all(np.isfinite(bufs[-len(rows)].download(np.float32, stream=stream))))
    nbytes = fused_bytes(kind, fmt, rows, K)
    for b in bufs:
        b.free()
    stream.destroy()
    return {"kind": kind, "fmt": fmt, "rows": list(rows), "K": K, **rotation_fields(copies, set_bytes, steps),
            "bytes_per_call": nbytes, "us_per_call": avg_us, "GBps": nbytes / (avg_us * 1e-6) / 1e9,
            "frac_of_hbm_peak": nbytes / (avg_us * 1e-6) / 1e9 / HBM_PEAK_GBS, "y_finite": finite}


def bench_gguf_upload(ctx, gib: float, reps: int = 3) -> dict:
    """GGUF file -> HBM: writes a synthetic GGUF of `gib` GiB (random Q4_K
    bytes) to a temporary file, opens it (map + parse + checks) and times
    er_hip_gguf_upload of its data section.  Host-to-device over PCIe:
    page-cache reads, pinned staging, DMA."""
    import tempfile
    from edgerunner_amd.gguf import GGUFLoader, GGUFMetadataValueType as VT, GGUFTensorType as TT
    from edgerunner_amd.gguf import write_gguf

    rows = int(gib * (1 << 30)) // (16 * 144)  # 4096-column Q4_K rows
    payload = np.random.default_rng(7).integers(0, 256, size=rows * 16 * 144, dtype=np.uint8)
    with tempfile.TemporaryDirectory() as d:
        path = write_gguf(Path(d) / "synthetic.gguf", [("general.architecture", VT.string, "llama")],
                          [("blk.0.ffn_up.weight", [4096, rows], TT.q4_K, payload.tobytes())])
        del payload
        t0 = time.perf_counter()
        loader = GGUFLoader(path)
        open_s = time.perf_counter() - t0
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            w = loader.load(ctx)
            times.append(time.perf_counter() - t0)
            loader.deviceData.free()
            del w
        off, n = loader.dataSection()
        loader.close()
    best = min(times)
    return {"bytes": n, "open_ms": open_s * 1e3, "upload_ms": best * 1e3,
            "GBps": n / best / 1e9, "reps": reps}


def bench_gemm(ctx, fmt: str, T: int, N: int, K: int, cfg: int, steps: int, warmup: int) -> dict:
    """Prefill GEMM: `steps` launches over rotating weight copies, recorded
    into a HIP graph and replayed between HIP events (as bench_gemv)."""
    import edgerunner_amd.synth as synth
    from edgerunner_amd import QuantGEMMKernel

    gemm = QuantGEMMKernel(ctx)
    W = synth.weights(fmt, synth.seed(cfg, 0), N, K, **DSCALE[fmt])
    X = synth.normal_bf16(synth.seed(cfg, 1), T * K)
    copies = max(2, -(-ROTATE_BYTES // W.nbytes))
    stream = ctx.stream()
    wbufs = [ctx.upload(W, stream) for _ in range(copies)]
    xb = ctx.upload(X, stream)
    yb = ctx.alloc(4 * T * N)
    enc = gemm.encodeQ4K if fmt == "q4_k" else gemm.encodeQ8_0
    for i in range(warmup):
        enc(stream, wbufs[i % copies], xb, yb, T, N, K)
    stream.synchronize()
    us = rotation_time_us(ctx, stream, lambda i: enc(stream, wbufs[i % copies], xb, yb, T, N, K), steps, copies)
    y = yb.download(np.float32, count=min(T * N, 1 << 20), stream=stream)
    clock = gemm_clock(ctx, stream, fmt, wbufs, xb, yb, T, N, K)
    for b in wbufs:
        b.free()
    xb.free()
    yb.free()
    stream.destroy()
    flops = 2.0 * T * N * K
    tflops = flops / (us * 1e-6) / 1e12
    out = {"fmt": fmt, "T": T, "N": N, "K": K, **rotation_fields(copies, W.nbytes, steps),
           "us_per_call": us, "TFLOPs": tflops,
           "frac_of_mfma_bf16_peak": tflops / MFMA_BF16_PEAK_TFLOPS,
           "min_bytes": gemm_min_bytes(fmt, T, N, K), "y_finite": bool(np.all(np.isfinite(y)))}
    if clock:
        out.update(clock)
        out["frac_of_mfma_bf16_peak_at_clock"] = tflops / (MFMA_BF16_PEAK_TFLOPS * clock["sclk_mhz"] / PEAK_SCLK_MHZ)
    return out


def gemm_clock(ctx, stream, fmt: str, wbufs, xb, yb, T: int, N: int, K: int) -> dict:
    """The shader clock the GEMM's workgroups run at: CLOCK_LAUNCHES
    back-to-back launches through er_hip_probe_gemm_clock (the same kernel
    and result as the product call, plus per-workgroup stamps of the 100 MHz
    real-time and the shader-clock counters); the last launch's workgroups
    give d(shader clock) / d(real time).  Empty where the loader-specialised
    kernel does not take the shape."""
    import ctypes as C
    pctx = probe_context(ctx)
    lib = pctx.lib
    nT = -(-T // 128)
    stamps = ctx.alloc(32 * nT * -(-N // 128))  # enough for either tile height
    items = C.c_uint32(0)
    typ = 12 if fmt == "q4_k" else 8  # ER_TYPE_Q4_K / ER_TYPE_Q8_0
    try:
        for i in range(CLOCK_LAUNCHES):
            st = lib.er_hip_probe_gemm_clock(pctx.handle, stream.handle, typ, wbufs[i % len(wbufs)].raw, xb.raw, yb.raw,
                                             T, N, K, stamps.raw, C.byref(items))
            if st != 0:
                return {}
        stream.synchronize()
        s = stamps.download(np.uint64, count=4 * items.value, stream=stream).reshape(-1, 4).astype(np.float64)
    finally:
        stamps.free()
    mhz = (s[:, 3] - s[:, 2]) / (s[:, 1] - s[:, 0]) * 100.0
    return {"sclk_mhz": float(np.median(mhz)), "sclk_mhz_min": float(mhz.min()), "sclk_mhz_max": float(mhz.max()),
            "workgroup_us_median": float(np.median(s[:, 1] - s[:, 0]) / 100.0), "clock_workgroups": int(items.value)}


_PROBE_CTX = {}


def probe_context(ctx):
    """A context of the measurement library (libedgerunner_probe.so) on ctx's
    device, created once: the probes and the clock-stamped GEMM copy live
    there, not in the product library.  Device buffers and streams of ctx
    pass to it."""
    from edgerunner_amd import Context
    dev = int(ctx.info.device)
    if dev not in _PROBE_CTX:
        _PROBE_CTX[dev] = Context(dev, probes=True)
    return _PROBE_CTX[dev]


def bench_chain(ctx, steps: int, warmup: int) -> dict:
    """one decode step's projections (28 Qwen3-0.6B layers,
    Q4_K_M mix, 151936-row Q6_K head), recorded into a HIP graph; `steps`
    replays timed between HIP events, per-projection and fused forms."""
    from edgerunner_amd.chain import ChainSpec, DecodeChain, make_inputs, make_weights

    spec = ChainSpec()
    stream = ctx.stream()
    ch = DecodeChain(ctx, spec, make_weights(spec), make_inputs(spec), stream)
    stream.synchronize()
    out = {"weight_bytes_per_step": spec.weight_bytes()}
    e0, e1 = ctx.event(), ctx.event()
    for fused in (False, True):
        for _ in range(warmup):
            ch.encode(stream, fused)
        g = ch.capture(stream, fused)
        g.launch(stream)
        stream.synchronize()
        g.launch(stream)  # untimed: the timed replays queue behind it (rotation_time_us)
        e0.record(stream)
        for _ in range(steps):
            g.launch(stream)
        e1.record(stream)
        stream.synchronize()
        us = e0.elapsed_ms(e1) * 1000.0 / steps
        e0.record(stream)
        for _ in range(max(1, steps // 10)):
            ch.encode(stream, fused)
        e1.record(stream)
        stream.synchronize()
        eager = e0.elapsed_ms(e1) * 1000.0 / max(1, steps // 10)
        g.destroy()
        tag = "fused" if fused else "per_projection"
        out[tag] = {"launches": spec.launches(fused), "us_per_step": us,
                    "GBps": spec.weight_bytes() / (us * 1e-6) / 1e9,
                    "frac_of_hbm_peak": spec.weight_bytes() / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                    "us_per_step_eager": eager}
    e0.destroy()
    e1.destroy()
    ch.free()
    stream.destroy()
    return out


def rotation_time_us(ctx, stream, enc, steps: int, copies: int) -> float:
    """Average GPU time per call of calls enc(0..steps-1), where call i reads
    weight copy i % copies and `copies` copies hold >= ROTATE_BYTES.  The
    `steps` calls are recorded into one HIP graph, replayed between HIP events
    (after UNTIMED_REPLAYS untimed replays).  When steps < copies, an untimed
    graph of calls steps..copies-1 runs before every replay of the timed one
    (and is left as the last work before return, so an eager loop that follows
    starts cold too): between two reads of any copy every other copy is read,
    >= ROTATE_BYTES - one copy, so no timed call finds its weights in the
    256 MB Infinity Cache, whatever `steps` is."""
    from edgerunner_amd import Capture
    with Capture(ctx, stream) as cap:
        for i in range(steps):
            enc(i)
    timed = cap.graph
    flush = None
    if steps < copies:
        with Capture(ctx, stream) as cap:
            for i in range(steps, copies):
                enc(i)
        flush = cap.graph
    for _ in range(UNTIMED_REPLAYS):
        if flush:
            flush.launch(stream)
        timed.launch(stream)
    stream.synchronize()
    # The timed replay is queued behind untimed work (the flush graph, or one
    # more replay of the timed graph, which leaves the cache as cold as the
    # replays above), so the start event is stamped when the GPU reaches it and
    # not while the host is still submitting the graph to an idle GPU.
    e0, e1 = ctx.event(), ctx.event()
    (flush or timed).launch(stream)
    e0.record(stream)
    timed.launch(stream)
    e1.record(stream)
    stream.synchronize()
    us = e0.elapsed_ms(e1) * 1000.0 / steps
    if flush:
        flush.launch(stream)
        stream.synchronize()
        flush.destroy()
    timed.destroy()
    e0.destroy()
    e1.destroy()
    return us


def rotation_fields(copies: int, per_call_bytes: int, steps: int) -> dict:
    """What every rotated workload reports about its cache state: the copies,
    the distinct bytes one cycle (timed calls + flush calls) reads, and the
    timed calls."""
    return {"copies": copies, "timed_launches": steps,
            "distinct_bytes_per_cycle": max(steps, copies) * per_call_bytes}


def _graph_time_us(ctx, stream, enc, steps: int) -> float:
    """Average GPU time per call of `steps` calls of enc(i) recorded into one
    HIP graph (after untimed replays), bracketed by HIP events."""
    from edgerunner_amd import Capture
    with Capture(ctx, stream) as cap:
        for i in range(steps):
            enc(i)
    g = cap.graph
    for _ in range(UNTIMED_REPLAYS):
        g.launch(stream)
    stream.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    g.launch(stream)  # untimed: the timed replay queues behind it (rotation_time_us)
    e0.record(stream)
    g.launch(stream)
    e1.record(stream)
    stream.synchronize()
    us = e0.elapsed_ms(e1) * 1000.0 / steps
    g.destroy()
    e0.destroy()
    e1.destroy()
    return us


# (name, bytes): the weight bytes of the two headline GEMV matrices
STREAM_WORKLOADS = [("stream_read_33MB", 33030144), ("stream_read_62MB", 62390272)]
BARRIER_GRIDS = (64, 128, 256)


def bench_ceilings(ctx, steps: int) -> dict:
    """The ceilings the GEMV and chain designs are measured against:
      - a plain non-temporal 16-byte-per-lane read of each headline matrix's
        weight bytes, over rotating copies (>= 768 MB, so every launch misses
        the Infinity Cache), graph-timed like the GEMVs, best of 3 grid sizes;
      - an empty kernel: GPU time per node of a graph of `steps` launches;
      - a grid-wide barrier (one agent-scope counter, bounded waits) across
        64 / 128 / 256 resident workgroups: (time of 200 rounds - time of 0
        rounds) / 200, each one launch bracketed by events;
      - per-CU rates behind the prefill GEMM: LDS reads (A-fragment layout)
        with 4 / 8 / 16 waves per CU, bf16 MFMA / fp32 FMA overlap within
        one wave and across two waves of a SIMD, and int8 MFMAs alone and with
        a Q8_0 per-block rescale each (best of 3 launches each)."""
    pctx = probe_context(ctx)
    lib = pctx.lib
    _check = pctx.check
    stream = ctx.stream()
    out = {}
    for name, nbytes in STREAM_WORKLOADS:
        copies = max(2, -(-ROTATE_BYTES // nbytes))
        bufs = [ctx.alloc(nbytes) for _ in range(copies)]
        for b in bufs:
            b.upload(np.full(nbytes // 4, 0x3f800000, np.uint32), stream=stream)
        best = None
        for wgs in (1024, 2048, 4096):
            sink = ctx.alloc(wgs * 256 * 4)
            enc = lambda i: _check(lib.er_hip_probe_stream_read(pctx.handle, stream.handle, bufs[i % copies].raw,
                                                                 nbytes, wgs, sink.raw))  # noqa: E731
            for i in range(5):
                enc(i)
            us = rotation_time_us(ctx, stream, enc, steps, copies)
            sink.free()
            if best is None or us < best[0]:
                best = (us, wgs)
        for b in bufs:
            b.free()
        out[name] = {"bytes": nbytes, **rotation_fields(copies, nbytes, steps), "us_per_call": best[0],
                     "workgroups": best[1],
                     "GBps": nbytes / (best[0] * 1e-6) / 1e9,
                     "frac_of_hbm_peak": nbytes / (best[0] * 1e-6) / 1e9 / HBM_PEAK_GBS}
        log(f"{name}: {best[0]:.2f} us, {out[name]['GBps']:.0f} GB/s ({best[1]} workgroups)")
    us = _graph_time_us(ctx, stream, lambda i: _check(lib.er_hip_probe_empty(pctx.handle, stream.handle)), steps)
    out["empty_kernel_in_graph"] = {"us_per_launch": us, "launches": steps}
    log(f"empty kernel in a graph: {us:.2f} us per launch")
    counter, res = ctx.alloc(16), ctx.alloc(16)
    e0, e1 = ctx.event(), ctx.event()
    rounds = 200
    for wgs in BARRIER_GRIDS:
        if wgs > ctx.compute_units:
            continue
        t = {}
        res.upload(np.zeros(4, np.uint32), stream=stream)  # the launches add to it
        for r in (0, rounds, 0, rounds):
            e0.record(stream)
            _check(lib.er_hip_probe_grid_barrier(pctx.handle, stream.handle, wgs, r, 1 << 20, counter.raw, res.raw))
            e1.record(stream)
            stream.synchronize()
            t[r] = min(t.get(r, 1e30), e0.elapsed_ms(e1) * 1000.0)
        polls, timeouts = (int(v) for v in res.download(np.uint32, 2))
        per = (t[rounds] - t[0]) / rounds
        out[f"grid_barrier_{wgs}"] = {"workgroups": wgs, "rounds": rounds, "us_per_barrier": per,
                                      "timeouts": timeouts, "polls": polls}
        log(f"grid barrier, {wgs} workgroups: {per:.2f} us per barrier ({timeouts} timed-out waits)")
    # per-CU rates of the prefill GEMM design: LDS reads in the A-fragment
    # layout with 4 / 8 / 16 waves per CU, and matrix-core / vector-ALU overlap
    sink = ctx.alloc(ctx.compute_units * 1024 * 4)

    def timed(launch) -> float:
        best = 1e30
        for _ in range(3):
            e0.record(stream)
            launch()
            e1.record(stream)
            stream.synchronize()
            best = min(best, e0.elapsed_ms(e1) * 1000.0)
        return best
    iters = 20000
    for waves in (4, 8, 16):
        us = timed(lambda: _check(lib.er_hip_probe_lds_read(pctx.handle, stream.handle, waves, iters, sink.raw)))
        per_cu = iters * 8 * 1024 * waves / (us * 1000.0)
        out[f"lds_read_{waves}_waves"] = {"us": us, "bytes_per_ns_per_cu": per_cu, "iters": iters}
        log(f"LDS reads, {waves} waves per CU: {per_cu:.0f} B/ns per CU")
    for mode, tag in enumerate(("mfma_alone", "fma_alone", "mfma_and_fma_two_waves", "mfma_and_fma_one_wave")):
        us = timed(lambda: _check(lib.er_hip_probe_mfma_valu(pctx.handle, stream.handle, mode, iters, sink.raw)))
        out[f"overlap_{tag}"] = {"us": us, "ns_per_iteration": us * 1000.0 / iters, "iters": iters}
        log(f"overlap {tag}: {us * 1000.0 / iters:.1f} ns per iteration (8 MFMA and/or 64 FMA per wave)")
    # int8 MFMAs for the Q8_0 prefill: alone, and each with the per-block
    # rescale of its int32 sums; the second prices the inner loop of such a
    # kernel at 512x14336x4096 (T/32 * N/32 * K/32 MFMAs over 4 SIMDs per CU)
    n_i8 = (512 // 32) * (14336 // 32) * (4096 // 32) / (4 * ctx.compute_units)
    for mode, tag in ((4, "i8_mfma_alone"), (5, "i8_mfma_with_block_rescale")):
        us = timed(lambda: _check(lib.er_hip_probe_mfma_valu(pctx.handle, stream.handle, mode, iters, sink.raw)))
        ns = us * 1000.0 / iters
        out[f"overlap_{tag}"] = {"us": us, "ns_per_iteration": ns, "iters": iters,
                                 "us_for_512x14336x4096": n_i8 * ns / 8 / 1000.0}
        log(f"overlap {tag}: {ns:.1f} ns per iteration (8 int8 MFMA per wave), "
            f"{n_i8 * ns / 8 / 1000.0:.1f} us of such iterations for Q8_0 512x14336x4096")
    sink.free()
    e0.destroy()
    e1.destroy()
    counter.free()
    res.free()
    stream.destroy()
    return out


def bench_chain_breakdown(ctx, steps: int) -> dict:
    """Where the decode chain's time goes: each distinct projection of a layer
    (and the head), and the fused triple / dual launches, timed alone like a
    GEMV workload (rotation_time_us over >= 768 MB of rotating weight copies,
    so each launch reads HBM as it does inside the 398 MB step).  The
    sums per step (x 28 layers + head) are set beside the measured chain."""
    import edgerunner_amd.synth as synth
    from edgerunner_amd import GEMVKernel
    from edgerunner_amd.chain import ChainSpec

    spec = ChainSpec()
    gemv = GEMVKernel(ctx)
    stream = ctx.stream()
    out = {}

    def rotating(fmt, M, K, t):
        W = synth.weights(fmt, synth.seed(5, 200 + t), M, K, **DSCALE[fmt])
        copies = max(2, -(-ROTATE_BYTES // W.nbytes))
        return [ctx.upload(W, stream) for _ in range(copies)], W.nbytes

    xs = {n: ctx.upload(synth.normal_f32(synth.seed(5, 300 + i), d), stream)
          for i, (n, d) in enumerate((("h", spec.hidden), ("a", spec.q_dim), ("f", spec.ffn)))}
    shapes = {}
    for name, fmt, M, K, src in spec.layer_projections() + [("head", spec.head_fmt, spec.vocab, spec.hidden, "h")]:
        shapes[name] = (fmt, M, K, src)
    for t, (name, (fmt, M, K, src)) in enumerate(shapes.items()):
        ws, wbytes = rotating(fmt, M, K, t)
        yb = ctx.alloc(4 * M)
        enc = getattr(gemv, ENCODE[fmt])
        f = lambda i: enc(stream, ws[i % len(ws)], xs[src], yb, M, K)  # noqa: E731
        for i in range(3):
            f(i)
        us = rotation_time_us(ctx, stream, f, steps, len(ws))
        out[name] = {"fmt": fmt, "M": M, "K": K, "weight_bytes": wbytes, **rotation_fields(len(ws), wbytes, steps),
                     "us_per_call": us, "GBps": wbytes / (us * 1e-6) / 1e9}
        for b in ws:
            b.free()
        yb.free()
        log(f"chain part {name} {fmt} {M}x{K}: {us:.2f} us ({out[name]['GBps']:.0f} GB/s)")
    # fused launches: q/k/v triple and gate/up dual over rotating layer copies
    tri = [rotating("q4_k", m, spec.hidden, 20 + j) for j, m in enumerate((spec.q_dim, spec.kv_dim, spec.kv_dim))]
    ys = [ctx.alloc(4 * m) for m in (spec.q_dim, spec.kv_dim, spec.kv_dim)]
    n = min(len(w[0]) for w in tri)
    f = lambda i: gemv.encodeQ4KWeightsTriple(stream, tri[0][0][i % n], tri[1][0][i % n], tri[2][0][i % n],  # noqa
                                              xs["h"], ys[0], ys[1], ys[2], spec.q_dim, spec.kv_dim, spec.kv_dim,
                                              spec.hidden)
    us = rotation_time_us(ctx, stream, f, steps, n)
    out["qkv_triple"] = {"us_per_call": us, "weight_bytes": sum(w[1] for w in tri),
                         **rotation_fields(n, sum(w[1] for w in tri), steps)}
    for w in tri:
        for b in w[0]:
            b.free()
    for b in ys:
        b.free()
    log(f"chain part qkv triple: {us:.2f} us")
    du = [rotating("q4_k", spec.ffn, spec.hidden, 30 + j) for j in range(2)]
    ys = [ctx.alloc(4 * spec.ffn) for _ in range(2)]
    n = min(len(w[0]) for w in du)
    f = lambda i: gemv.encodeQ4KWeightsDual(stream, du[0][0][i % n], du[1][0][i % n], xs["h"], ys[0], ys[1],  # noqa
                                            spec.ffn, spec.hidden)
    us = rotation_time_us(ctx, stream, f, steps, n)
    out["gate_up_dual"] = {"us_per_call": us, "weight_bytes": sum(w[1] for w in du),
                           **rotation_fields(n, sum(w[1] for w in du), steps)}
    for w in du:
        for b in w[0]:
            b.free()
    for b in ys:
        b.free()
    log(f"chain part gate/up dual: {us:.2f} us")
    L = spec.layers
    per = sum(out[k]["us_per_call"] for k in ("q", "k", "v", "o", "gate", "up", "down"))
    fused = sum(out[k]["us_per_call"] for k in ("qkv_triple", "o", "gate_up_dual", "down"))
    out["sum_per_projection_us"] = L * per + out["head"]["us_per_call"]
    out["sum_fused_us"] = L * fused + out["head"]["us_per_call"]
    for b in xs.values():
        b.free()
    stream.destroy()
    return out


def _check(status: int) -> None:
    from edgerunner_amd.runtime import check
    check(status)


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(fmt: str, M: int, K: int, cfg: int, budget_s: float) -> dict:
    """Times the CPU oracle (oracle/er_oracle.c, the reference's Swift CPU
    loop restated in C) on the same synthetic workload, all rows of the
    matrix per call: single-threaded for a third of `budget_s`, then with the
    rows split over every host thread this process may use for the rest.
    The GPU boxes give one GPU's process a 16-thread CPU share
    (OMP_NUM_THREADS=16, whatever nproc shows), so "all cores" is that share;
    nproc, the affinity mask and the CPU model are reported beside it."""
    import edgerunner_amd.synth as synth
    from oracle import ref

    W = synth.weights(fmt, synth.seed(cfg, 0), M, K, **DSCALE[fmt])
    x = synth.normal_f32(synth.seed(cfg, 1), K)
    nbytes = algorithmic_bytes(fmt, M, K)
    nproc = os.cpu_count() or 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or affinity
    threads = max(1, min(share, affinity, ref.max_threads()))

    def timed(nthreads: int, seconds: float):
        ref.gemv(fmt, W, x, M, K, threads=nthreads)  # warm
        calls, t0 = 0, time.perf_counter()
        while True:
            ref.gemv(fmt, W, x, M, K, threads=nthreads)
            calls += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                return calls, el

    c1, e1 = timed(1, budget_s / 3.0)
    cn, en = timed(threads, budget_s * 2.0 / 3.0)
    per1, pern = e1 / c1, en / cn
    return {
        "value": nbytes / pern / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
        "value_1thread": nbytes / per1 / 1e9,
        "nproc": nproc, "affinity_cpus": affinity, "cpu_model": _cpu_model(),
        "sample": f"full {fmt.upper()} GEMV calls {M}x{K}: {c1} single-threaded in {e1:.1f} s "
                  f"({per1 * 1e3:.1f} ms/call), {cn} with rows split over {threads} OpenMP threads "
                  f"(the process's CPU share; nproc {nproc}) in {en:.1f} s ({pern * 1e3:.2f} ms/call)",
        "us_per_call": pern * 1e6,
    }


TRAFFIC_FILE = ROOT / "profiles" / "gemv_hbm_traffic.txt"


def load_traffic(name: str):
    """HBM bytes per launch of workload `name` from the committed rocprofv3
    counter summary (lines `workload fetch_bytes write_bytes`), or None."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        f = line.split()
        if len(f) == 3 and f[0] == name and not line.startswith("#"):
            return int(float(f[1]) + float(f[2]))
    return None


COPY_CAL_BYTES = 64 << 20


def probe(ctx, todo, steps: int, gemm_todo=(), order_file=None, chain_steps: int = 0, dq_todo=(),
          fu_todo=()) -> None:
    """Counter-collection driver (run under `rocprofv3 --pmc ...`): three
    device-to-device copies of COPY_CAL_BYTES (the calibration kernel of known
    traffic), then for each GEMV workload (rotating weights) and each GEMM
    workload in `gemm_todo`, dequantisation in `dq_todo` and fused projection
    in `fu_todo`: one empty kernel (er_probe_empty) that marks
    where the workload's dispatches begin, then its `steps` calls; with
    chain_steps, the same for that many eager steps of the fused decode chain.  The workload names
    and step counts go to `order_file` (one `name steps` line each), which
    summarize() reads to label the dispatch groups."""
    import edgerunner_amd.synth as synth
    from edgerunner_amd import GEMVKernel

    stream = ctx.stream()
    src, dst = ctx.alloc(COPY_CAL_BYTES), ctx.alloc(COPY_CAL_BYTES)
    for _ in range(3):
        dst.copy_from(src, stream=stream)
    stream.synchronize()
    order = []
    pctx = probe_context(ctx)

    def separator():
        pctx.check(pctx.lib.er_hip_probe_empty(pctx.handle, stream.handle))
    gemv = GEMVKernel(ctx)
    for name, fmt, M, K, cfg in todo:
        W = synth.weights(fmt, synth.seed(cfg, 0), M, K, **DSCALE[fmt])
        x = synth.normal_f32(synth.seed(cfg, 1), K)
        copies = max(2, -(-ROTATE_BYTES // W.nbytes))
        wbufs = [ctx.upload(W, stream) for _ in range(copies)]
        xb, yb = ctx.upload(x, stream), ctx.alloc(4 * M)
        enc = getattr(gemv, ENCODE[fmt])
        stream.synchronize()
        separator()
        for i in range(steps):
            enc(stream, wbufs[i % copies], xb, yb, M, K)
        stream.synchronize()
        order.append((name, steps))
        log(f"probe {name}: {steps} launches")
        for b in wbufs:
            b.free()
        xb.free()
        yb.free()
    for name, fmt, M, K, cfg in dq_todo:
        import edgerunner_amd
        kern = getattr(edgerunner_amd, DEQUANT_KERNELS[fmt])(ctx)
        W = synth.weights(fmt, synth.seed(cfg, 0), M, K, **DSCALE[fmt])
        count = M * K // BLOCK[fmt][1]
        copies = max(2, -(-ROTATE_BYTES // W.nbytes))
        wbufs = [ctx.upload(W, stream) for _ in range(copies)]
        out = ctx.alloc(4 * M * K)
        stream.synchronize()
        separator()
        for i in range(steps):
            kern.encode(stream, wbufs[i % copies], count, out)
        stream.synchronize()
        order.append((name, steps))
        log(f"probe {name}: {steps} calls")
        for b in wbufs + [out]:
            b.free()
    for name, kind, fmt, rows, K, cfg in fu_todo:
        enc, copies, _, bufs = fused_calls(ctx, stream, kind, fmt, rows, K, cfg)
        stream.synchronize()
        separator()
        for i in range(steps):
            enc(i)
        stream.synchronize()
        order.append((name, steps))
        log(f"probe {name}: {steps} calls")
        for b in bufs:
            b.free()
    if gemm_todo:
        from edgerunner_amd import QuantGEMMKernel
        gemm = QuantGEMMKernel(ctx)
    for name, fmt, T, N, K, cfg in gemm_todo:
        W = synth.weights(fmt, synth.seed(cfg, 0), N, K, **DSCALE[fmt])
        X = synth.normal_bf16(synth.seed(cfg, 1), T * K)
        copies = max(2, -(-ROTATE_BYTES // W.nbytes))
        wbufs = [ctx.upload(W, stream) for _ in range(copies)]
        xb, yb = ctx.upload(X, stream), ctx.alloc(4 * T * N)
        enc = gemm.encodeQ4K if fmt == "q4_k" else gemm.encodeQ8_0
        stream.synchronize()
        separator()
        for i in range(steps):
            enc(stream, wbufs[i % copies], xb, yb, T, N, K)
        stream.synchronize()
        order.append((name, steps))
        log(f"probe {name}: {steps} calls")
        for b in wbufs + [xb, yb]:
            b.free()
    if chain_steps:
        # the decode chain's fused encodes, eagerly on the stream (no graph
        # capture): per-kernel durations of the chain under --kernel-trace
        from edgerunner_amd.chain import ChainSpec, DecodeChain, make_inputs, make_weights
        spec = ChainSpec()
        ch = DecodeChain(ctx, spec, make_weights(spec), make_inputs(spec), stream)
        stream.synchronize()
        separator()
        for _ in range(chain_steps):
            ch.encode(stream, True)
        stream.synchronize()
        order.append(("decode_chain_fused_eager", chain_steps))  # per call = per decode step
        log(f"probe decode_chain_fused_eager: {chain_steps} steps, {spec.launches(True)} launches each")
        ch.free()
    for b in (src, dst):
        b.free()
    stream.destroy()
    if order_file:
        Path(order_file).parent.mkdir(parents=True, exist_ok=True)
        Path(order_file).write_text("".join(f"{n} {k}\n" for n, k in order))


def _read_csv(path: Path):
    import csv
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


def summarize(root: Path) -> str:
    """Markdown summary of a rocprofv3 output tree holding three runs: kernel
    stats of the bench workloads (stats/, `--kernel-trace --stats`), and the
    FETCH_SIZE (fetch/) and WRITE_SIZE (write/) counter runs of `--probe`."""
    out = []
    stats = sorted(root.glob("stats/**/*kernel_stats.csv"))
    if stats:
        out.append("## Kernel statistics (rocprofv3 --kernel-trace --stats)\n")
        out.append("| kernel | calls | avg us | min us | max us | % time |")
        out.append("|---|---|---|---|---|---|")
        for r in _read_csv(stats[0]):
            out.append(f"| {r['Name']} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                       f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                       f"{float(r['Percentage']):.1f} |")
        out.append("")
    traces = sorted(root.glob("stats/**/*kernel_trace.csv"))
    if traces:
        import collections
        by = collections.defaultdict(list)
        for r in _read_csv(traces[0]):
            key = (r["Kernel_Name"], r.get("Grid_Size_X", r.get("Grid_Size", "")),
                   r.get("Grid_Size_Y", ""))
            by[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        # consecutive launches of one (kernel, grid) in dispatch order: the
        # workloads of a leg one after another (shapes that share a grid, such
        # as the two stream reads, stay apart here)
        runs = []
        for r in sorted(_read_csv(traces[0]), key=lambda r: int(r["Start_Timestamp"])):
            key = (r["Kernel_Name"], r.get("Grid_Size_X", r.get("Grid_Size", "")))
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            if runs and runs[-1][0] == key:
                runs[-1][1].append(d)
            else:
                runs.append((key, [d]))
        out.append("## Runs of consecutive launches (kernel trace, dispatch order, runs of 20 or more)\n")
        out.append("| # | kernel | grid x | launches | avg us | median us | min us |")
        out.append("|---|---|---|---|---|---|---|")
        for i, ((k, gx), v) in enumerate(r for r in runs if len(r[1]) >= 20):
            v = sorted(v)
            out.append(f"| {i} | {k} | {gx} | {len(v)} | {sum(v) / len(v):.2f} | {v[len(v) // 2]:.2f} | "
                       f"{v[0]:.2f} |")
        out.append("")
        out.append("## Per-launch-shape durations (kernel trace)\n")
        out.append("| kernel | grid x | grid y | launches | avg us | median us |")
        out.append("|---|---|---|---|---|---|")
        for (k, gx, gy), v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
            v = sorted(v)
            out.append(f"| {k} | {gx} | {gy} | {len(v)} | {sum(v) / len(v):.2f} | "
                       f"{v[len(v) // 2]:.2f} |")
        out.append("")
    per_workload = {}
    order_path = root / "probe_order.txt"
    order = ([(l.split()[0], int(l.split()[1])) for l in order_path.read_text().splitlines() if l.strip()]
             if order_path.exists() else [(w[0], None) for w in GEMV_WORKLOADS])
    for counter, sub in (("FETCH_SIZE", "fetch"), ("WRITE_SIZE", "write")):
        files = sorted(root.glob(f"{sub}/**/*counter_collection.csv"))
        if not files:
            continue
        rows = [r for r in _read_csv(files[0]) if r["Counter_Name"] == counter]
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        # calibration: the COPY_CAL_BYTES device copies are the largest copy dispatches
        copies = [float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]]
        big = [v for v in copies if copies and v >= 0.5 * max(copies)]
        measured = sum(big) / len(big) if big else float("nan")
        factor = (COPY_CAL_BYTES / 1024) / measured if big else float("nan")
        # dispatch groups: the kernels after each er_probe_empty marker
        # (copy kernels, which uploads use too, belong to no group)
        groups = []
        for r in rows:
            if r["Kernel_Name"].startswith("er_probe_empty"):
                groups.append([])
            elif "copyBuffer" not in r["Kernel_Name"] and groups:
                groups[-1].append(r)
        out.append(f"## {counter} per call, rocprofv3 --pmc {counter}\n")
        out.append(f"Calibration: a {COPY_CAL_BYTES >> 20} MiB device-to-device copy (reads and "
                   f"writes {COPY_CAL_BYTES >> 10} KiB) counts {measured:.0f} KiB per dispatch on "
                   f"this counter; scale factor {factor:.4f}.\n")
        out.append("| workload | kernels | dispatches | KiB per call | calibrated bytes per call |")
        out.append("|---|---|---|---|---|")
        for i, grp in enumerate(groups):
            name, steps = order[i] if i < len(order) else (f"group{i}", None)
            calls = steps or len(grp)
            kib = sum(float(r["Counter_Value"]) for r in grp) / calls
            cb = kib * 1024 * factor
            per_workload.setdefault(name, {})[counter] = cb
            kernels = ", ".join(sorted({r["Kernel_Name"] for r in grp}))
            out.append(f"| {name} | {kernels} | {len(grp)} | {kib:.1f} | {cb:.0f} |")
        out.append("")
    if per_workload:
        out.append("## HBM traffic per call vs algorithmic bytes\n")
        out.append("```")
        out.append("# workload fetch_bytes write_bytes  (calibrated FETCH_SIZE, WRITE_SIZE)")
        for name, v in per_workload.items():
            out.append(f"{name} {v.get('FETCH_SIZE', 0):.0f} {v.get('WRITE_SIZE', 0):.0f}")
        out.append("```\n")
        out.append("| workload | algorithmic bytes | measured bytes | ratio |")
        out.append("|---|---|---|---|")
        alg = {w[0]: algorithmic_bytes(w[1], w[2], w[3]) for w in GEMV_WORKLOADS}
        alg.update({w[0]: gemm_min_bytes(w[1], w[2], w[3], w[4]) for w in GEMM_WORKLOADS})
        alg.update({w[0]: dequant_bytes(w[1], w[2], w[3]) for w in DEQUANT_WORKLOADS})
        alg.update({w[0]: fused_bytes(w[1], w[2], w[3], w[4]) for w in FUSED_WORKLOADS})
        from edgerunner_amd.chain import ChainSpec
        alg["decode_chain_fused_eager"] = ChainSpec().weight_bytes()
        for name, v in per_workload.items():
            if name in alg:
                tot = v.get("FETCH_SIZE", 0) + v.get("WRITE_SIZE", 0)
                out.append(f"| {name} | {alg[name]} | {tot:.0f} | {tot / alg[name]:.3f} |")
        out.append("")
    return "\n".join(out)



def _rounded(v):
    if isinstance(v, dict):
        return {k: _rounded(x) for k, x in v.items()}
    if isinstance(v, float):
        return round(v, 4)
    return v


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workloads", default="all",
                    help="comma list of workload names, or 'all' / 'headline'")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--probe", action="store_true",
                    help="counter-collection driver for rocprofv3 --pmc (no JSON line)")
    ap.add_argument("--probe-order", metavar="FILE",
                    help="with --probe: write the workload order for --summarize")
    ap.add_argument("--summarize", metavar="DIR",
                    help="print a markdown summary of a rocprofv3 output tree and exit")
    args = ap.parse_args()
    if args.summarize:
        print(summarize(Path(args.summarize)))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not built)"}))
        return 2

    from edgerunner_amd import Context
    ctx = Context(0)
    log(f"device {ctx.info.name.decode()} arch={ctx.arch} CUs={ctx.compute_units} "
        f"LDS/workgroup={ctx.info.lds_per_workgroup} clock={ctx.info.clock_khz} kHz")

    head = GEMV_WORKLOADS[0]
    if args.workloads == "all":
        todo = GEMV_WORKLOADS
    elif args.workloads == "headline":
        todo = [head]
    else:
        names = set(args.workloads.split(","))
        todo = [w for w in GEMV_WORKLOADS if w[0] in names]
        if head not in todo:
            todo = [head] + todo
    if args.probe:
        gemm_todo = [w for w in GEMM_WORKLOADS if args.workloads not in ("all", "headline")
                     and w[0] in args.workloads.split(",")]
        dq_todo = [w for w in DEQUANT_WORKLOADS if args.workloads not in ("all", "headline")
                   and w[0] in args.workloads.split(",")]
        fu_todo = [w for w in FUSED_WORKLOADS if args.workloads not in ("all", "headline")
                   and w[0] in args.workloads.split(",")]
        chain_steps = 3 if "decode_chain" in args.workloads.split(",") else 0
        probe(ctx, todo, args.steps, gemm_todo, args.probe_order, chain_steps, dq_todo, fu_todo)
        return 0
    results = {}
    for name, fmt, M, K, cfg in todo:
        log(f"{name}: running")
        r = bench_gemv(ctx, fmt, M, K, cfg, args.steps, args.warmup)
        r["traffic_bytes"] = load_traffic(name)
        results[name] = r
        log(f"{name}: {r['us_per_call']:.2f} us/call, {r['GBps']:.0f} GB/s "
            f"({100 * r['frac_of_hbm_peak']:.1f}% of 8 TB/s); eager {r['us_per_call_eager']:.2f} us")

    for name, M, K, cfg in TOP1_WORKLOADS:
        if args.workloads not in ("all",) and name not in args.workloads.split(","):
            continue
        log(f"{name}: running")
        r = bench_top1(ctx, M, K, cfg, max(20, args.steps // 2), min(args.warmup, 5))
        results[name] = r
        log(f"{name}: {r['us_per_call']:.2f} us/call, {r['GBps']:.0f} GB/s "
            f"({100 * r['frac_of_hbm_peak']:.1f}% of 8 TB/s), row {r['index']}")

    for name, rows, K, cfg in QUANT_WORKLOADS:
        if args.workloads not in ("all",) and name not in args.workloads.split(","):
            continue
        log(f"{name}: running")
        r = bench_quant(ctx, rows, K, cfg, max(20, args.steps // 2), min(args.warmup, 5))
        results[name] = r
        log(f"{name}: {r['us_per_call']:.2f} us/call, {r['GBps']:.0f} GB/s "
            f"({100 * r['frac_of_hbm_peak']:.1f}% of 8 TB/s)")

    for name, fmt, M, K, cfg in DEQUANT_WORKLOADS:
        if args.workloads not in ("all",) and name not in args.workloads.split(","):
            continue
        log(f"{name}: running")
        r = bench_dequant(ctx, fmt, M, K, cfg, max(20, args.steps // 4), min(args.warmup, 5))
        r["traffic_bytes"] = load_traffic(name)
        results[name] = r
        log(f"{name}: {r['us_per_call']:.2f} us/call, {r['GBps']:.0f} GB/s "
            f"({100 * r['frac_of_hbm_peak']:.1f}% of 8 TB/s)")

    for name, kind, fmt, rows, K, cfg in FUSED_WORKLOADS:
        if args.workloads not in ("all",) and name not in args.workloads.split(","):
            continue
        log(f"{name}: running")
        r = bench_fused(ctx, kind, fmt, rows, K, cfg, max(20, args.steps // 4), min(args.warmup, 5))
        r["traffic_bytes"] = load_traffic(name)
        results[name] = r
        log(f"{name}: {r['us_per_call']:.2f} us/call, {r['GBps']:.0f} GB/s "
            f"({100 * r['frac_of_hbm_peak']:.1f}% of 8 TB/s)")

    for name, fmt, T, N, K, cfg in GEMM_WORKLOADS:
        if args.workloads not in ("all",) and name not in args.workloads.split(","):
            continue
        log(f"{name}: running")
        r = bench_gemm(ctx, fmt, T, N, K, cfg, max(20, args.steps // 4), min(args.warmup, 5))
        r["traffic_bytes"] = load_traffic(name)
        results[name] = r
        clk = (f"; workgroups ran at {r['sclk_mhz']:.0f} MHz (min {r['sclk_mhz_min']:.0f}), "
               f"{100 * r['frac_of_mfma_bf16_peak_at_clock']:.1f}% of the peak at that clock") if "sclk_mhz" in r else ""
        log(f"{name}: {r['us_per_call']:.2f} us/call, {r['TFLOPs']:.1f} TFLOP/s "
            f"({100 * r['frac_of_mfma_bf16_peak']:.1f}% of bf16 dense peak){clk}")

    if args.workloads == "all" or "gguf_upload" in args.workloads:
        log("gguf_upload_1gib: running")
        r = bench_gguf_upload(ctx, 1.0)
        results["gguf_upload_1gib"] = r
        log(f"gguf_upload_1gib: open {r['open_ms']:.1f} ms, upload {r['upload_ms']:.1f} ms, "
            f"{r['GBps']:.1f} GB/s host-to-HBM")

    if args.workloads in ("all", "chain") or "decode_chain" in args.workloads:
        log("decode_chain: running")
        r = bench_chain(ctx, max(20, args.steps // 4), 3)
        results["decode_chain_qwen3_0.6b_q4km"] = r
        for tag in ("per_projection", "fused"):
            v = r[tag]
            log(f"decode_chain {tag}: {v['launches']} launches, {v['us_per_step']:.1f} us/step, "
                f"{v['GBps']:.0f} GB/s ({100 * v['frac_of_hbm_peak']:.1f}% of 8 TB/s); "
                f"eager {v['us_per_step_eager']:.1f} us")

    if args.workloads in ("all", "chain") or "chain_breakdown" in args.workloads.split(","):
        log("chain_breakdown: running")
        results["chain_breakdown"] = bench_chain_breakdown(ctx, max(20, args.steps // 4))

    if args.workloads == "all" or "ceilings" in args.workloads.split(","):
        log("ceilings: running")
        results["ceilings"] = bench_ceilings(ctx, args.steps)

    h = results[head[0]]
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline: running")
        cpu = cpu_baseline(head[1], head[2], head[3], head[4], args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads, {cpu['value_1thread']:.2f} GB/s "
            f"single-threaded ({cpu['cpu_model']}, nproc {cpu['nproc']})")

    traffic = load_traffic(head[0])
    out = {
        "metric": METRIC,
        "value": round(h["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": h["us_per_call"] / 1000.0,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded xoshiro256**, BASELINE.json config distributions)",
        "config": {"workload": f"Q4_K decode GEMV, W 14336x4096 (BASELINE configs[1]), x fp32, "
                               f"y fp32, {h['copies']} rotating weight copies",
                   "M": head[2], "K": head[3], "format": "Q4_K"},
        "roofline": {
            "bound": "hbm",
            "achieved": round(h["GBps"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(h["frac_of_hbm_peak"], 4),
            "traffic": traffic,
        },
        "cpu_baseline": ({k: (round(v, 3) if isinstance(v, float) else v)
                          for k, v in cpu.items() if k != "us_per_call"} if cpu else None),
        "results": _rounded(results),
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
