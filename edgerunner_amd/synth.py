"""Seeded synthetic workloads for the BASELINE configurations (host side).

Thin ctypes binding of csrc/er_synth.c (xoshiro256** as in
Sources/EdgeRunnerCore/Sampling/SeededRandomSource.swift:3-30).  Seeds follow
seed(config c, tensor t) = 0xED6E0000 + 16*c + t.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_PATH = Path(__file__).resolve().parent / "liber_synth.so"
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not _PATH.exists():
            raise RuntimeError(f"{_PATH} is not built; run `python -m edgerunner_amd.build`")
        lib = C.CDLL(str(_PATH))
        u8p, f32p = C.POINTER(C.c_uint8), C.POINTER(C.c_float)
        lib.er_synth_q8_0.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_float, u8p]
        lib.er_synth_q4_k.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_float, C.c_float, u8p]
        lib.er_synth_q6_k.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_float, u8p]
        for f in (lib.er_synth_q8_0, lib.er_synth_q4_k, lib.er_synth_q6_k):
            f.restype = C.c_int
        lib.er_synth_normal_f32.argtypes = [C.c_uint64, C.c_uint64, f32p]
        lib.er_synth_normal_f32.restype = None
        lib.er_synth_normal_bf16.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint16)]
        lib.er_synth_normal_bf16.restype = None
        lib.er_synth_rng_outputs.argtypes = [C.c_uint64, C.POINTER(C.c_uint64), C.c_uint32]
        lib.er_synth_rng_outputs.restype = None
        _lib = lib
    return _lib


def seed(config: int, tensor: int) -> int:
    return 0xED6E0000 + 16 * config + tensor


def rng_outputs(s: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint64)
    _load().er_synth_rng_outputs(s, out.ctypes.data_as(C.POINTER(C.c_uint64)), n)
    return out


def q8_0(s: int, M: int, K: int, dscale: float = 0.02) -> np.ndarray:
    out = np.empty(M * (K // 32) * 34, dtype=np.uint8)
    if _load().er_synth_q8_0(s, M, K, dscale, out.ctypes.data_as(C.POINTER(C.c_uint8))) != 0:
        raise ValueError("K must be a positive multiple of 32")
    return out


def q4_k(s: int, M: int, K: int, dscale: float = 0.01, dminscale: float = 0.01) -> np.ndarray:
    out = np.empty(M * (K // 256) * 144, dtype=np.uint8)
    if _load().er_synth_q4_k(s, M, K, dscale, dminscale,
                             out.ctypes.data_as(C.POINTER(C.c_uint8))) != 0:
        raise ValueError("K must be a positive multiple of 256")
    return out


def q6_k(s: int, M: int, K: int, dscale: float = 0.005) -> np.ndarray:
    out = np.empty(M * (K // 256) * 210, dtype=np.uint8)
    if _load().er_synth_q6_k(s, M, K, dscale, out.ctypes.data_as(C.POINTER(C.c_uint8))) != 0:
        raise ValueError("K must be a positive multiple of 256")
    return out


def weights(fmt: str, s: int, M: int, K: int, **kw) -> np.ndarray:
    return {"q8_0": q8_0, "q4_k": q4_k, "q6_k": q6_k}[fmt](s, M, K, **kw)


def normal_f32(s: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _load().er_synth_normal_f32(s, n, out.ctypes.data_as(C.POINTER(C.c_float)))
    return out


def normal_bf16(s: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    _load().er_synth_normal_bf16(s, n, out.ctypes.data_as(C.POINTER(C.c_uint16)))
    return out
