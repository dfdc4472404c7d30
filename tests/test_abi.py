"""CPU checks of the C ABI: the library loads, exports exactly what
include/*.h declares, and validates shapes before touching a device
(GEMVKernel.swift:1415-1432 rules), so these run without a GPU."""
import ctypes as C
import re
from pathlib import Path

import pytest

from edgerunner_amd import _ffi

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b((?:er_hip|er_status|er_gguf)_\w+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "er_hip_create" in names and "er_hip_encode_q4k_weights" in names
    assert len(names) >= 25


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(str(_ffi.LIB_PATH))
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    assert set(declared_symbols()) <= set(_ffi.SIGNATURES)


def test_abi_version_and_status_strings():
    lib = _ffi.load()
    assert lib.er_hip_abi_version() == 1
    assert lib.er_status_string(4) == b"invalidMatrixShape"
    assert lib.er_status_string(5) == b"invalidVectorShape"


def _buf(n, ptr=0x1000):
    return _ffi.er_buffer(ptr, n)


@pytest.mark.parametrize("entry,block,per", [
    ("er_hip_encode_q4k_weights", 144, 256),
    ("er_hip_encode_q6k_weights", 210, 256),
    ("er_hip_encode_q8_0_weights", 34, 32),
])
def test_gemv_validation_without_device(entry, block, per):
    lib = _ffi.load()
    fn = getattr(lib, entry)
    M, K = 8, 2 * 256
    wbytes = M * (K // per) * block
    ok = lambda: fn(None, None, _buf(wbytes), _buf(K * 4), _buf(M * 4), M, K)  # noqa: E731
    # all shapes valid -> the null context is what fails
    assert ok() == 8
    # K not a multiple of the block width / zero -> invalidVectorShape
    assert fn(None, None, _buf(wbytes), _buf(K * 4), _buf(M * 4), M, K + per // 2) == 5
    assert fn(None, None, _buf(wbytes), _buf(K * 4), _buf(M * 4), M, 0) == 5
    # short weight buffer -> invalidMatrixShape
    assert fn(None, None, _buf(wbytes - 1), _buf(K * 4), _buf(M * 4), M, K) == 4
    # short input / output -> encodingFailed
    assert fn(None, None, _buf(wbytes), _buf(K * 4 - 4), _buf(M * 4), M, K) == 3
    assert fn(None, None, _buf(wbytes), _buf(K * 4), _buf(M * 4 - 4), M, K) == 3
    msg = _ffi.last_error()
    assert "too small" in msg


def test_batched_validation_without_device():
    lib = _ffi.load()
    M, K, T = 4, 256, 3
    f = lib.er_hip_encode_batched_q4k_weights
    assert f(None, None, _buf(M * 144), _buf(T * K * 4), _buf(T * M * 4), T, M, K) == 8
    assert f(None, None, _buf(M * 144), _buf(T * K * 4), _buf(T * M * 4), 0, M, K) == 3
    assert f(None, None, _buf(M * 144), _buf(T * K * 4 - 1), _buf(T * M * 4), T, M, K) == 3


@pytest.mark.parametrize("entry,block,per", [
    ("er_hip_dequant_q8_0", 34, 32), ("er_hip_dequant_q4_k", 144, 256),
    ("er_hip_dequant_q6_k", 210, 256)])
def test_dequant_validation_without_device(entry, block, per):
    fn = getattr(_ffi.load(), entry)
    n = 5
    assert fn(None, None, _buf(n * block), n, _buf(n * per * 4)) == 8
    assert fn(None, None, _buf(n * block - 1), n, _buf(n * per * 4)) == 6
    assert fn(None, None, _buf(n * block), n, _buf(n * per * 4 - 4)) == 7


def test_projection_rejects_unsupported_type():
    lib = _ffi.load()
    t = _ffi.er_tensor_storage()
    t.buffer = _buf(1 << 20)
    t.data_type = 0  # float32 is not on the quantized path
    t.ndim = 2
    t.shape[0], t.shape[1] = 256, 4
    assert lib.er_hip_encode_projection(None, None, C.byref(t), _buf(1024), _buf(16), 1) == 8
    t.data_type = 12
    t.ndim = 3
    assert lib.er_hip_encode_projection(None, None, C.byref(t), _buf(1024), _buf(16), 1) == 4


def test_top1_noalloc_validation_without_device():
    lib = _ffi.load()
    f = lib.er_hip_encode_q6k_weights_packed_top1_noalloc
    K = 256
    for M, want in ((1024, 8), (1022, 4), (262144, 8), (262148, 4)):
        # valid shapes reach the null-context check; M % 4 != 0 and heads
        # past ER_HIP_TOP1_NOALLOC_MAX_ROWS fail before it
        assert f(None, None, _buf(M * 210), _buf(4 * K), _buf(4), M, K) == want, M
    assert f(None, None, _buf(1024 * 210), _buf(4 * K), _buf(3), 1024, K) == 3


# The reference's alternative GEMVKernel encoders and the canonical entry
# each one is (GEMVKernel.swift:724, 745, 767, 789, 840, 1045, 1184).
ALIASES = {
    "er_hip_encode_q4k_weights_packed": "er_hip_encode_q4k_weights",
    "er_hip_encode_q4k_weights_packed_four_rows": "er_hip_encode_q4k_weights",
    "er_hip_encode_q4k_weights_llama_style": "er_hip_encode_q4k_weights",
    "er_hip_encode_q4k_weights_two_rows": "er_hip_encode_q4k_weights",
    "er_hip_encode_q6k_weights_packed": "er_hip_encode_q6k_weights",
    "er_hip_encode_q4k_weights_llama_style_dual": "er_hip_encode_q4k_weights_dual",
    "er_hip_encode_q4k_weights_triple_packed": "er_hip_encode_q4k_weights_triple",
}


def test_alias_table_matches_header():
    names = set(declared_symbols())
    for alias, canon in ALIASES.items():
        assert alias in names and canon in names
        assert _ffi.SIGNATURES[alias] == _ffi.SIGNATURES[canon], alias


@pytest.mark.parametrize("alias", [a for a, c in ALIASES.items() if c in (
    "er_hip_encode_q4k_weights", "er_hip_encode_q6k_weights")])
def test_alias_validation_equals_canonical(alias):
    lib = _ffi.load()
    a, c = getattr(lib, alias), getattr(lib, ALIASES[alias])
    block = 210 if "q6k" in alias else 144
    M, K = 8, 512
    wb = M * (K // 256) * block
    cases = [(wb, K * 4, M * 4, M, K), (wb, K * 4, M * 4, M, K + 128), (wb, K * 4, M * 4, M, 0),
             (wb - 1, K * 4, M * 4, M, K), (wb, K * 4 - 4, M * 4, M, K), (wb, K * 4, M * 4 - 4, M, K)]
    for w, xl, yl, m, k in cases:
        got = a(None, None, _buf(w), _buf(xl), _buf(yl), m, k)
        assert got == c(None, None, _buf(w), _buf(xl), _buf(yl), m, k)
    assert a(None, None, _buf(wb), _buf(K * 4), _buf(M * 4), M, K) == 8


def test_multi_alias_validation_equals_canonical():
    lib = _ffi.load()
    M, K = 4, 256
    for w in (M * 144, M * 144 - 1):
        args = (None, None, _buf(w), _buf(M * 144), _buf(K * 4), _buf(M * 4), _buf(M * 4), M, K)
        assert lib.er_hip_encode_q4k_weights_llama_style_dual(*args) == lib.er_hip_encode_q4k_weights_dual(*args)
    for k in (K, K + 1):
        args = (None, None, _buf(M * 144), _buf(M * 144), _buf(M * 144), _buf(K * 4), _buf(M * 4), _buf(M * 4),
                _buf(M * 4), M, M, M, k)
        assert lib.er_hip_encode_q4k_weights_triple_packed(*args) == lib.er_hip_encode_q4k_weights_triple(*args)


def test_execute_validation_without_device():
    """GEMVKernel.execute* rules (validateKQuantInputShape): x.count == K, K a
    positive multiple of 256, enough weight bytes, room for y; a valid call
    then fails on the null context."""
    import numpy as np
    lib = _ffi.load()
    M, K = 4, 256
    w = np.zeros(M * 144, np.uint8)
    x = np.zeros(K, np.float32)
    y = np.zeros(M, np.float32)
    f = lib.er_hip_execute_q4k_weights
    assert f(None, w.ctypes.data, w.size, x.ctypes.data, K, y.ctypes.data, M, M, K) == 8
    assert f(None, w.ctypes.data, w.size, x.ctypes.data, K - 1, y.ctypes.data, M, M, K) == 5
    assert f(None, w.ctypes.data, w.size - 1, x.ctypes.data, K, y.ctypes.data, M, M, K) == 4
    assert f(None, w.ctypes.data, w.size, x.ctypes.data, K, y.ctypes.data, M - 1, M, K) == 3
    g = lib.er_hip_execute_q6k_weights_with_weight_buffer
    assert g(None, _buf(M * 210), x.ctypes.data, K, y.ctypes.data, M, M, K) == 8
    assert g(None, _buf(M * 210 - 1), x.ctypes.data, K, y.ctypes.data, M, M, K) == 4
    assert g(None, _buf(M * 210), x.ctypes.data, K + 1, y.ctypes.data, M, M, K) == 5
    b = lib.er_hip_execute_batched_q4k_weights
    xb = np.zeros(3 * K, np.float32)
    yb = np.zeros(3 * M, np.float32)
    assert b(None, w.ctypes.data, w.size, xb.ctypes.data, 3 * K, yb.ctypes.data, 3 * M, 3, M, K) == 8
    assert b(None, w.ctypes.data, w.size, xb.ctypes.data, 3 * K, yb.ctypes.data, 3 * M, 0, M, K) == 5
    assert b(None, w.ctypes.data, w.size, xb.ctypes.data, 2 * K, yb.ctypes.data, 3 * M, 3, M, K) == 5
    # executeBatchedQ4KWeights (GEMVKernel.swift:623-640) runs the K and weight
    # rules before batchSeq / x.count: a short weight buffer is
    # invalidMatrixShape even when batchSeq or x.count is also wrong
    assert b(None, w.ctypes.data, w.size - 1, xb.ctypes.data, 3 * K, yb.ctypes.data, 3 * M, 0, M, K) == 4
    assert b(None, w.ctypes.data, w.size - 1, xb.ctypes.data, 2 * K, yb.ctypes.data, 3 * M, 3, M, K) == 4
    assert b(None, w.ctypes.data, w.size, xb.ctypes.data, 3 * K, yb.ctypes.data, 3 * M, 0, M, K + 32) == 5
    # the single-vector form checks x.count first (vectorCount == K)
    assert f(None, w.ctypes.data, w.size - 1, x.ctypes.data, K - 1, y.ctypes.data, M, M, K) == 5


def test_noalloc_top1_rejects_heads_past_the_array():
    """er_hip_encode_q6k_weights_packed_top1_noalloc: heads of more than
    ER_HIP_TOP1_NOALLOC_MAX_ROWS rows are INVALID_MATRIX_SHAPE, decided from
    the lengths before the context or any buffer is touched (null context,
    placeholder pointers never dereferenced)."""
    lib = _ffi.load()
    max_rows = 262144
    M, K = max_rows + 4, 256
    st = lib.er_hip_encode_q6k_weights_packed_top1_noalloc(None, None, _buf(M * 210), _buf(4 * K), _buf(4), M, K)
    assert st == 4 and "exceeds" in _ffi.last_error()
    # at the limit the shape passes and the null context is what fails
    M = max_rows
    st = lib.er_hip_encode_q6k_weights_packed_top1_noalloc(None, None, _buf(M * 210), _buf(4 * K), _buf(4), M, K)
    assert st == 8


def _exported(path):
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_product_library_exports_exactly_the_boundary():
    """libedgerunner_hip.so exports what include/*.h declares and nothing
    else: no measurement entry point (those live in libedgerunner_probe.so)."""
    exported = _exported(_ffi.LIB_PATH)
    declared = set(declared_symbols()) | {"er_status_string"}
    assert exported == declared, (sorted(exported - declared), sorted(declared - exported))


def test_probe_library_is_a_superset():
    if not _ffi.PROBE_LIB_PATH.exists():
        pytest.skip("measurement library not built")
    exported = _exported(_ffi.PROBE_LIB_PATH)
    assert set(declared_symbols()) <= exported
    assert set(_ffi.PROBE_SIGNATURES) <= exported
