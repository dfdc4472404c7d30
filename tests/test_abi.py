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
