"""ctypes binding of liber_oracle.so (the C restatement in er_oracle.c).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# ER_ORACLE_LIB selects another build of the oracle (the sanitizer build)
LIB = Path(os.environ["ER_ORACLE_LIB"]) if os.environ.get("ER_ORACLE_LIB") else HERE / "liber_oracle.so"
_lib = None

u8p = C.POINTER(C.c_uint8)
f32p = C.POINTER(C.c_float)
u16p = C.POINTER(C.c_uint16)


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB.exists():
        build()
    lib = C.CDLL(str(LIB))
    lib.er_ref_f16_to_f32.argtypes = [C.c_uint16]
    lib.er_ref_f16_to_f32.restype = C.c_float
    lib.er_ref_f32_to_f16.argtypes = [C.c_float]
    lib.er_ref_f32_to_f16.restype = C.c_uint16
    lib.er_ref_f32_to_bf16.argtypes = [C.c_float]
    lib.er_ref_f32_to_bf16.restype = C.c_uint16
    for name in ("er_ref_dequant_q8_0", "er_ref_dequant_q4_k", "er_ref_dequant_q6_k"):
        f = getattr(lib, name)
        f.argtypes = [u8p, C.c_uint64, f32p]
        f.restype = None
    for name in ("er_ref_gemv_q8_0", "er_ref_gemv_q4_k", "er_ref_gemv_q6_k"):
        f = getattr(lib, name)
        f.argtypes = [u8p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int]
        f.restype = None
    lib.er_ref_gemm.argtypes = [C.c_int, u8p, u16p, f32p, C.c_int, C.c_int, C.c_int, C.c_int]
    lib.er_ref_gemm.restype = C.c_int
    lib.er_ref_quantize_q8_0_rows.argtypes = [f32p, u8p, C.c_uint32, C.c_uint32, C.c_uint32,
                                              C.c_uint32]
    lib.er_ref_quantize_q8_0_rows.restype = None
    for name in ("er_ref_pack_q8_0_block", "er_ref_pack_q4_k_block", "er_ref_pack_q6_k_block"):
        f = getattr(lib, name)
        f.argtypes = [f32p, u8p]
        f.restype = None
    for name in ("er_ref_make_q4k_weights", "er_ref_make_q6k_weights"):
        f = getattr(lib, name)
        f.argtypes = [C.c_int, C.c_int, u8p]
        f.restype = None
    lib.er_ref_gelu_tanh.argtypes = [C.c_float]
    lib.er_ref_gelu_tanh.restype = C.c_float
    lib.er_ref_argmax.argtypes = [f32p, C.c_uint32]
    lib.er_ref_argmax.restype = C.c_uint32
    lib.er_ref_rmsnorm.argtypes = [f32p, f32p, C.c_uint32, C.c_float, f32p]
    lib.er_ref_rmsnorm.restype = None
    lib.er_ref_silu.argtypes = [C.c_float]
    lib.er_ref_silu.restype = C.c_float
    lib.er_ref_top1.argtypes = [f32p, C.c_uint32]
    lib.er_ref_top1.restype = C.c_uint32
    lib.er_ref_max_threads.argtypes = []
    lib.er_ref_max_threads.restype = C.c_int
    _lib = lib
    return lib


BLOCK = {"q8_0": (34, 32), "q4_k": (144, 256), "q6_k": (210, 256)}
TYPE = {"q8_0": 8, "q4_k": 12, "q6_k": 14}


def _u8(a):
    a = np.ascontiguousarray(a, dtype=np.uint8).reshape(-1)
    return a, a.ctypes.data_as(u8p)


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    return a, a.ctypes.data_as(f32p)


def dequant(fmt: str, blocks) -> np.ndarray:
    bb, bw = BLOCK[fmt]
    b, bp = _u8(blocks)
    n = b.size // bb
    out = np.empty(n * bw, dtype=np.float32)
    getattr(load(), f"er_ref_dequant_{fmt}")(bp, n, out.ctypes.data_as(f32p))
    return out


def gemv(fmt: str, W, x, M: int, K: int, tokens: int = 1, threads: int = 1) -> np.ndarray:
    w, wp = _u8(W)
    xv, xp = _f32(x)
    assert xv.size == tokens * K
    y = np.empty(tokens * M, dtype=np.float32)
    getattr(load(), f"er_ref_gemv_{fmt}")(wp, xp, y.ctypes.data_as(f32p), M, K, tokens, threads)
    return y


def gemm(fmt: str, W, X_bf16, T: int, N: int, K: int, threads: int = 1) -> np.ndarray:
    w, wp = _u8(W)
    x = np.ascontiguousarray(X_bf16, dtype=np.uint16).reshape(-1)
    assert x.size == T * K
    y = np.empty(T * N, dtype=np.float32)
    rc = load().er_ref_gemm(TYPE[fmt], wp, x.ctypes.data_as(u16p), y.ctypes.data_as(f32p), T, N,
                            K, threads)
    assert rc == 0
    return y.reshape(T, N)


def quantize_q8_0_rows(src, rowCount: int, srcRowStride: int, dstRowBase: int,
                       blocksPerRow: int, dst=None) -> np.ndarray:
    s, sp = _f32(src)
    if dst is None:
        dst = np.zeros((dstRowBase + rowCount) * blocksPerRow * 34, dtype=np.uint8)
    d, dp = _u8(dst)
    load().er_ref_quantize_q8_0_rows(sp, dp, rowCount, srcRowStride, dstRowBase, blocksPerRow)
    return d


def pack_block(fmt: str, values) -> np.ndarray:
    v, vp = _f32(values)
    bb, bw = BLOCK[fmt]
    assert v.size == bw
    out = np.zeros(bb, dtype=np.uint8)
    getattr(load(), f"er_ref_pack_{fmt}_block")(vp, out.ctypes.data_as(u8p))
    return out


def make_q4k_weights(rows: int, cols: int) -> np.ndarray:
    out = np.zeros(rows * cols // 256 * 144, dtype=np.uint8)
    load().er_ref_make_q4k_weights(rows, cols, out.ctypes.data_as(u8p))
    return out


def make_q6k_weights(rows: int, cols: int) -> np.ndarray:
    out = np.zeros(rows * cols // 256 * 210, dtype=np.uint8)
    load().er_ref_make_q6k_weights(rows, cols, out.ctypes.data_as(u8p))
    return out


def gelu_tanh(v) -> np.ndarray:
    f = load().er_ref_gelu_tanh
    return np.array([f(float(t)) for t in np.asarray(v, np.float32).ravel()], np.float32)


def argmax(v) -> int:
    a, ap = _f32(v)
    return int(load().er_ref_argmax(ap, a.size))


def rmsnorm(x, w, eps: float) -> np.ndarray:
    a, ap = _f32(x)
    b, bp = _f32(w)
    assert a.size == b.size
    out = np.empty(a.size, np.float32)
    load().er_ref_rmsnorm(ap, bp, a.size, eps, out.ctypes.data_as(f32p))
    return out


def silu(v) -> np.ndarray:
    f = load().er_ref_silu
    return np.array([f(float(t)) for t in np.asarray(v, np.float32).ravel()], np.float32)


def top1(v) -> int:
    """Row chosen by the reference's two-stage top-1 (len(v) % 4 == 0)."""
    a, ap = _f32(v)
    assert a.size % 4 == 0
    return int(load().er_ref_top1(ap, a.size))


def f16_to_f32(h: int) -> float:
    return float(load().er_ref_f16_to_f32(h))


def f32_to_f16(f: float) -> int:
    return int(load().er_ref_f32_to_f16(f))


def f32_to_bf16(f: float) -> int:
    return int(load().er_ref_f32_to_bf16(f))


def max_threads() -> int:
    return int(load().er_ref_max_threads())
