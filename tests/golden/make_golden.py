"""Writes tests/golden/reference_cases.npz -- TEST INFRASTRUCTURE.

The reference (EdgeRunner, Swift + Metal) stores no literal golden vectors: its
kernel tests build their inputs with deterministic formula fillers and compare
against CPU helpers at test time.  This script restates those inputs and
records the CPU oracle's outputs for them, so that later changes to the oracle
or the kernels are checked against fixed numbers:

  q4k_9x512        makeQ4KWeights(9, 512), x[j] = ((j % 17) - 8) / 19
                   (Tests/EdgeRunnerMetalTests/GEMVTests.swift:136-151, 459-478)
  q4k_batch_7x512  makeQ4KWeights(7, 512), 3 tokens, x[j] = ((j % 37) - 18) / 23
                   (GEMVTests.swift:480-514)
  q6k_7x512        makeQ6KWeights(7, 512), x[j] = ((j % 23) - 11) / 29
  q6k_9x768        makeQ6KWeights(9, 768), same x formula
                   (GEMVTests.swift:153-170, 556-660)
  q8_0_64x128      packQ8_0Block of a seeded uniform[-0.5, 0.5] 64x128 matrix,
                   x = uniform[-1, 1] * (j + 1) / 128
                   (FusedKernelTests.swift:18-51, 89-126; the reference draws
                   unseeded Float.random, restated here with numpy's PCG64 seed 5)
  dq_*             dequantised fp32 values of the formula fillers' first blocks
                   and of the reference dequant tests' float patterns packed by
                   packQ*Block (DequantQ8_0Tests.swift:52, 75-77,
                   DequantQ4KMTests.swift:137, 160-162, DequantQ6KTests.swift)

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import ref  # noqa: E402

OUT = Path(__file__).resolve().parent / "reference_cases.npz"


def gemv_cases():
    cases = {}
    K = 512
    W = ref.make_q4k_weights(9, K)
    x = (((np.arange(K) % 17) - 8) / 19.0).astype(np.float32)
    cases["q4k_9x512"] = ("q4_k", 9, K, 1, W, x)
    W = ref.make_q4k_weights(7, K)
    x = (((np.arange(3 * K) % 37) - 18) / 23.0).astype(np.float32)
    cases["q4k_batch_7x512"] = ("q4_k", 7, K, 3, W, x)
    for M, K in ((7, 512), (9, 768)):
        W = ref.make_q6k_weights(M, K)
        x = (((np.arange(K) % 23) - 11) / 29.0).astype(np.float32)
        cases[f"q6k_{M}x{K}"] = ("q6_k", M, K, 1, W, x)
    rows, cols = 64, 128
    rng = np.random.default_rng(5)
    x = (rng.uniform(-1, 1, cols) * (np.arange(cols) + 1) / cols).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (rows, cols)).astype(np.float32)
    W = np.concatenate([ref.pack_block("q8_0", b) for b in w.reshape(-1, 32)])
    cases["q8_0_64x128"] = ("q8_0", rows, cols, 1, W, x)
    return cases


def dequant_cases():
    cases = {"dq_q4k_filler": ("q4_k", ref.make_q4k_weights(1, 256)),
             "dq_q6k_filler": ("q6_k", ref.make_q6k_weights(1, 256))}
    pat8 = [np.arange(32) * 0.1 - 1.6] + [((b * 31 + np.arange(32)) % 19 - 9) * 0.22 for b in range(8)]
    cases["dq_q8_0_patterns"] = ("q8_0", np.concatenate(
        [ref.pack_block("q8_0", np.asarray(p, np.float32)) for p in pat8]))
    patk = [np.arange(256) * 0.01 - 1.28] + [((b * 17 + np.arange(256)) % 29 - 14) * 0.14 for b in range(4)]
    for fmt in ("q4_k", "q6_k"):
        cases[f"dq_{fmt.replace('_', '')}_patterns"] = (fmt, np.concatenate(
            [ref.pack_block(fmt, np.asarray(p, np.float32)) for p in patk]))
    return cases


def main() -> None:
    arrays = {}
    for name, (fmt, M, K, T, W, x) in gemv_cases().items():
        arrays[f"{name}__fmt"] = np.array(fmt)
        arrays[f"{name}__shape"] = np.array([M, K, T], np.int64)
        arrays[f"{name}__W"] = np.asarray(W, np.uint8)
        arrays[f"{name}__x"] = x
        arrays[f"{name}__y"] = ref.gemv(fmt, W, x, M, K, tokens=T)
    for name, (fmt, blocks) in dequant_cases().items():
        arrays[f"{name}__fmt"] = np.array(fmt)
        arrays[f"{name}__blocks"] = np.asarray(blocks, np.uint8)
        arrays[f"{name}__values"] = ref.dequant(fmt, blocks)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
