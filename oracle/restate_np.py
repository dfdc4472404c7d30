"""Second, independent statement of the block layouts in numpy -- TEST
INFRASTRUCTURE (tests/ only).

Written from the bit-level layout, vectorised over blocks, with no shared code
with er_oracle.c, so that agreement between the two (bit-exact on dequantised
values) pins the byte layout:
  Q8_0 : DequantQ8_0Tests.swift:25-34
  Q4_K : DequantQ4KMTests.swift:84-119 (12-byte scale field read as a 96-bit
         little-endian integer: sc[j] = bits [6j, 6j+6) for j<4 ...)
  Q6_K : DequantQ6KTests.swift:80-113
"""
from __future__ import annotations

import numpy as np


def _f16(lo, hi):
    return (lo.astype(np.uint16) | (hi.astype(np.uint16) << 8)).view(np.float16).astype(np.float32)


def dequant_q8_0(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 34)
    d = _f16(b[:, 0], b[:, 1])
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d[:, None] * q).reshape(-1)


def q4k_scale_min(blocks: np.ndarray):
    """Per block and sub-block j (0..7): 6-bit scale and min, read bit-wise.
    Bytes s[0..11] = block[4..16).  For j<4: scale = low 6 bits of s[j],
    min = low 6 bits of s[j+4].  For j>=4: scale = low nibble of s[j+4] with
    the top two bits of s[j-4] above it; min = high nibble of s[j+4] with the
    top two bits of s[j] above it."""
    s = np.asarray(blocks, dtype=np.uint8).reshape(-1, 144)[:, 4:16].astype(np.int64)
    bits = lambda v, lo, n: (v >> lo) & ((1 << n) - 1)  # noqa: E731
    sc = np.zeros((s.shape[0], 8), dtype=np.int64)
    mn = np.zeros((s.shape[0], 8), dtype=np.int64)
    for j in range(4):
        sc[:, j] = bits(s[:, j], 0, 6)
        mn[:, j] = bits(s[:, j + 4], 0, 6)
        sc[:, j + 4] = bits(s[:, j + 8], 0, 4) + 16 * bits(s[:, j], 6, 2)
        mn[:, j + 4] = bits(s[:, j + 8], 4, 4) + 16 * bits(s[:, j + 4], 6, 2)
    return sc, mn


def dequant_q4_k(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 144)
    d = _f16(b[:, 0], b[:, 1])
    dmin = _f16(b[:, 2], b[:, 3])
    sc, mn = q4k_scale_min(b)
    qs = b[:, 16:].reshape(-1, 4, 32)            # [block, pair, l]
    lo = (qs & 0x0F).astype(np.float32)           # sub-block 2p
    hi = (qs >> 4).astype(np.float32)             # sub-block 2p+1
    q = np.stack([lo, hi], axis=2).reshape(-1, 8, 32)   # [block, j, l]
    scale = (d[:, None] * sc.astype(np.float32))[:, :, None]
    minv = (dmin[:, None] * mn.astype(np.float32))[:, :, None]
    return (scale * q - minv).astype(np.float32).reshape(-1)


def q6k_values(blocks: np.ndarray) -> np.ndarray:
    """6-bit quants in output order (0..63, before the -32 offset)."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 210)
    out = np.zeros((b.shape[0], 256), dtype=np.int64)
    for h in range(2):
        ql = b[:, 64 * h: 64 * h + 64].astype(np.int64)
        qh = b[:, 128 + 32 * h: 128 + 32 * h + 32].astype(np.int64)
        for k in range(4):  # output offset 32k
            nib = ql[:, 32 * (k & 1): 32 * (k & 1) + 32]
            nib = (nib & 15) if k < 2 else (nib >> 4)
            top = (qh >> (2 * k)) & 3
            out[:, 128 * h + 32 * k: 128 * h + 32 * k + 32] = nib | (top << 4)
    return out


def dequant_q6_k(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 210)
    d = _f16(b[:, 208], b[:, 209])
    sc = b[:, 192:208].view(np.int8).astype(np.float32)      # 16 scales, one per 16 outputs
    q = (q6k_values(b) - 32).astype(np.float32)
    scale = np.repeat(d[:, None] * sc, 16, axis=1)            # per output position
    return (scale * q).astype(np.float32).reshape(-1)


DEQUANT = {"q8_0": dequant_q8_0, "q4_k": dequant_q4_k, "q6_k": dequant_q6_k}
BLOCK = {"q8_0": (34, 32), "q4_k": (144, 256), "q6_k": (210, 256)}


def weights_f32(fmt: str, W: np.ndarray, M: int, K: int) -> np.ndarray:
    return DEQUANT[fmt](W).reshape(M, K)


def gemv_f64(fmt: str, W: np.ndarray, x: np.ndarray, M: int, K: int) -> np.ndarray:
    """float64 accumulation of the exactly-dequantised weights (diagnostic
    reference; independent of the fp32 summation order)."""
    w = weights_f32(fmt, W, M, K).astype(np.float64)
    return w @ np.asarray(x, dtype=np.float64).reshape(-1, K).T
