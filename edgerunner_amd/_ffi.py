"""ctypes declarations of the C ABI in include/er_hip.h.

The library is loaded from this package directory (it is built in-tree by
``python -m edgerunner_amd.build``).  A missing library is an error: there is
no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
# ER_HIP_LIB selects another build of the same library (the sanitizer build
# of the host-side tests); by default the in-tree library.
LIB_PATH = Path(os.environ["ER_HIP_LIB"]) if os.environ.get("ER_HIP_LIB") else PKG / "libedgerunner_hip.so"
PROBE_LIB_PATH = PKG / "libedgerunner_probe.so"

ER_OK = 0
STATUS_NAMES = {
    0: "ok",
    1: "libraryNotFound",
    2: "functionNotFound",
    3: "encodingFailed",
    4: "invalidMatrixShape",
    5: "invalidVectorShape",
    6: "invalidBlockDataCount",
    7: "allocationFailed",
    8: "invalidArgument",
    9: "deviceError",
    10: "fileNotFound",
    11: "invalidFormat",
    12: "unsupportedVersion",
    13: "unsupportedDataType",
    14: "mmapFailed",
    15: "missingMetadata",
    16: "tensorNotFound",
}


class er_buffer(C.Structure):
    _fields_ = [("data", C.c_void_p), ("length", C.c_uint64)]


class er_tensor_storage(C.Structure):
    _fields_ = [
        ("buffer", er_buffer),
        ("byte_offset", C.c_uint64),
        ("data_type", C.c_uint32),
        ("ndim", C.c_uint32),
        ("shape", C.c_uint64 * 4),
    ]


class er_gguf_value(C.Structure):
    _fields_ = [
        ("type", C.c_uint32),
        ("elem_type", C.c_uint32),
        ("count", C.c_uint64),
        ("u", C.c_uint64),
        ("i", C.c_int64),
        ("f", C.c_double),
        ("str", C.c_void_p),   # count bytes of UTF-8 (may hold NULs)
        ("node", C.c_void_p),
    ]


class er_gguf_tensor_info(C.Structure):
    _fields_ = [
        ("name", C.c_char_p),
        ("ndim", C.c_uint32),
        ("ggml_type", C.c_uint32),
        ("dims", C.c_uint64 * 8),
        ("offset", C.c_uint64),
        ("element_count", C.c_uint64),
        ("byte_count", C.c_uint64),
        ("data_type", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


class er_device_info(C.Structure):
    _fields_ = [
        ("device", C.c_int),
        ("compute_units", C.c_int),
        ("clock_khz", C.c_int),
        ("memory_clock_khz", C.c_int),
        ("memory_bus_width", C.c_int),
        ("total_memory", C.c_uint64),
        ("lds_per_workgroup", C.c_uint64),
        ("name", C.c_char * 64),
        ("arch", C.c_char * 64),
    ]


_ctx_p = C.c_void_p
_stream = C.c_void_p
_event = C.c_void_p
_graph = C.c_void_p
_u32 = C.c_uint32
_u64 = C.c_uint64

# name -> (restype, argtypes)
SIGNATURES = {
    "er_hip_abi_version": (C.c_int, []),
    "er_hip_create": (C.c_int, [C.c_int, C.POINTER(_ctx_p)]),
    "er_hip_destroy": (None, [_ctx_p]),
    "er_hip_get_device_info": (C.c_int, [_ctx_p, C.POINTER(er_device_info)]),
    "er_hip_last_error": (C.c_char_p, []),
    "er_status_string": (C.c_char_p, [C.c_int]),
    "er_hip_alloc": (C.c_int, [_ctx_p, _u64, C.POINTER(er_buffer)]),
    "er_hip_free": (C.c_int, [_ctx_p, er_buffer]),
    "er_hip_upload": (C.c_int, [_ctx_p, _stream, er_buffer, _u64, C.c_void_p, _u64]),
    "er_hip_download": (C.c_int, [_ctx_p, _stream, C.c_void_p, er_buffer, _u64, _u64]),
    "er_hip_copy": (C.c_int, [_ctx_p, _stream, er_buffer, _u64, er_buffer, _u64, _u64]),
    "er_hip_stream_create": (C.c_int, [_ctx_p, C.POINTER(_stream)]),
    "er_hip_stream_destroy": (C.c_int, [_ctx_p, _stream]),
    "er_hip_synchronize": (C.c_int, [_ctx_p, _stream]),
    "er_hip_event_create": (C.c_int, [_ctx_p, C.POINTER(_event)]),
    "er_hip_event_destroy": (C.c_int, [_ctx_p, _event]),
    "er_hip_event_record": (C.c_int, [_ctx_p, _event, _stream]),
    "er_hip_event_elapsed_ms": (C.c_int, [_ctx_p, _event, _event, C.POINTER(C.c_float)]),
    "er_hip_graph_begin": (C.c_int, [_ctx_p, _stream]),
    "er_hip_graph_end": (C.c_int, [_ctx_p, _stream, C.POINTER(_graph)]),
    "er_hip_graph_launch": (C.c_int, [_ctx_p, _graph, _stream]),
    "er_hip_graph_destroy": (C.c_int, [_ctx_p, _graph]),
    "er_hip_dequant_q8_0": (C.c_int, [_ctx_p, _stream, er_buffer, _u64, er_buffer]),
    "er_hip_dequant_q4_k": (C.c_int, [_ctx_p, _stream, er_buffer, _u64, er_buffer]),
    "er_hip_dequant_q6_k": (C.c_int, [_ctx_p, _stream, er_buffer, _u64, er_buffer]),
    "er_hip_encode_q4k_weights": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q6k_weights": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q8_0_weights": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q4k_weights_dual": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q4k_weights_triple": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, er_buffer, er_buffer, er_buffer,
                  er_buffer, _u32, _u32, _u32, _u32]),
    "er_hip_encode_q4k_weights_dual_geglu": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q6k_weights_packed_top1": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q4k_weights_packed": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q4k_weights_packed_four_rows": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q4k_weights_llama_style": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q4k_weights_two_rows": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q6k_weights_packed": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q4k_weights_llama_style_dual": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_encode_q4k_weights_triple_packed": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, er_buffer, er_buffer, er_buffer,
                  er_buffer, _u32, _u32, _u32, _u32]),
    "er_hip_execute_q4k_weights": (
        C.c_int, [_ctx_p, C.c_void_p, _u64, C.c_void_p, _u64, C.c_void_p, _u64, _u32, _u32]),
    "er_hip_execute_q6k_weights": (
        C.c_int, [_ctx_p, C.c_void_p, _u64, C.c_void_p, _u64, C.c_void_p, _u64, _u32, _u32]),
    "er_hip_execute_q4k_weights_with_weight_buffer": (
        C.c_int, [_ctx_p, er_buffer, C.c_void_p, _u64, C.c_void_p, _u64, _u32, _u32]),
    "er_hip_execute_q6k_weights_with_weight_buffer": (
        C.c_int, [_ctx_p, er_buffer, C.c_void_p, _u64, C.c_void_p, _u64, _u32, _u32]),
    "er_hip_execute_batched_q4k_weights": (
        C.c_int, [_ctx_p, C.c_void_p, _u64, C.c_void_p, _u64, C.c_void_p, _u64, _u32, _u32, _u32]),
    "er_hip_encode_q6k_weights_packed_top1_noalloc": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_quantize_q8_0_rows": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, _u32, _u32, _u32, _u32]),
    "er_hip_q8_0_fused_qkv": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, er_buffer,
                                        er_buffer, er_buffer, er_buffer, er_buffer, _u32, _u32, _u32,
                                        _u32, C.c_float]),
    "er_hip_q8_0_fused_qkv_turbo": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, er_buffer,
                                              er_buffer, er_buffer, er_buffer, er_buffer, _u32, _u32, _u32,
                                              _u32, C.c_float]),
    "er_hip_q8_0_fused_gate_up_silu": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer,
                                                 er_buffer, er_buffer, _u32, _u32, _u32, C.c_float]),
    "er_hip_q8_0_fused_final_norm_gemv": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer,
                                                    er_buffer, _u32, _u32, C.c_float]),
    "er_hip_q8_0_gemv_f16out": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32]),
    "er_hip_q8_0_gemv_add": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, er_buffer,
                                       _u32, _u32]),
    "er_hip_encode_batched_q4k_weights": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32, _u32]),
    "er_hip_encode_batched_q6k_weights": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32, _u32]),
    "er_hip_encode_batched_q8_0_weights": (
        C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32, _u32]),
    "er_hip_gemm_q4_k": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32, _u32]),
    "er_hip_gemm_q8_0": (C.c_int, [_ctx_p, _stream, er_buffer, er_buffer, er_buffer, _u32, _u32, _u32]),
    "er_gguf_parse_memory": (C.c_int, [C.c_void_p, C.c_uint64, _u32, C.POINTER(C.c_void_p)]),
    "er_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "er_gguf_close": (None, [C.c_void_p]),
    "er_gguf_header": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                                 C.POINTER(C.c_uint64)]),
    "er_gguf_metadata_count": (C.c_uint64, [C.c_void_p]),
    "er_gguf_metadata_key": (C.c_int, [C.c_void_p, C.c_uint64, C.POINTER(C.c_char_p)]),
    "er_gguf_metadata_value": (C.c_int, [C.c_void_p, C.c_uint64, C.POINTER(er_gguf_value)]),
    "er_gguf_find_metadata": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint64)]),
    "er_gguf_array_get": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(er_gguf_value)]),
    "er_gguf_tensor_count": (C.c_uint64, [C.c_void_p]),
    "er_gguf_tensor_info_at": (C.c_int, [C.c_void_p, C.c_uint64, C.POINTER(er_gguf_tensor_info)]),
    "er_gguf_find_tensor": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint64)]),
    "er_gguf_data_section": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "er_gguf_tensor_host_data": (C.c_int, [C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p),
                                           C.POINTER(C.c_uint64)]),
    "er_hip_gguf_upload": (C.c_int, [_ctx_p, _stream, C.c_void_p, C.POINTER(er_buffer)]),
    "er_gguf_tensor_storage": (C.c_int, [C.c_void_p, C.c_uint64, er_buffer,
                                         C.POINTER(er_tensor_storage)]),
    "er_hip_encode_projection": (
        C.c_int, [_ctx_p, _stream, C.POINTER(er_tensor_storage), er_buffer, er_buffer, _u32]),
}

# The measurement library's extra entry points (csrc/er_hip_probe.h).
PROBE_SIGNATURES = {
    "er_hip_probe_stream_read": (C.c_int, [_ctx_p, _stream, er_buffer, _u64, _u32, er_buffer]),
    "er_hip_probe_empty": (C.c_int, [_ctx_p, _stream]),
    "er_hip_probe_grid_barrier": (C.c_int, [_ctx_p, _stream, _u32, _u32, _u32, er_buffer, er_buffer]),
    "er_hip_probe_lds_read": (C.c_int, [_ctx_p, _stream, _u32, _u32, er_buffer]),
    "er_hip_probe_mfma_valu": (C.c_int, [_ctx_p, _stream, _u32, _u32, er_buffer]),
    "er_hip_probe_gemm_clock": (C.c_int, [_ctx_p, _stream, C.c_int, er_buffer, er_buffer, er_buffer, _u32, _u32, _u32,
                                          er_buffer, C.POINTER(C.c_uint32)]),
}

_lib = None
_probe_lib = None


class LibraryMissing(RuntimeError):
    pass


def _bind(path: Path, signatures: dict) -> C.CDLL:
    if not path.exists():
        raise LibraryMissing(
            f"{path} is not built; run `python -m edgerunner_amd.build` "
            "(the HIP library is required, there is no CPU fallback)")
    lib = C.CDLL(str(path))
    for name, (res, args) in signatures.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def load() -> C.CDLL:
    """Load libedgerunner_hip.so and bind every declared entry point."""
    global _lib
    if _lib is None:
        _lib = _bind(LIB_PATH, SIGNATURES)
    return _lib


def load_probe() -> C.CDLL:
    """Load the measurement library (libedgerunner_probe.so: every entry point
    of the product library plus the probes), for bench.py's ceilings and GEMM
    clock legs.  Its contexts, like its entry points, are its own; device
    buffers are plain device memory and pass between the two."""
    global _probe_lib
    if _probe_lib is None:
        _probe_lib = _bind(PROBE_LIB_PATH, {**SIGNATURES, **PROBE_SIGNATURES})
    return _probe_lib


def last_error(lib: C.CDLL | None = None) -> str:
    """The calling thread's last error message of `lib` (default: the product
    library)."""
    msg = (lib or load()).er_hip_last_error()
    return msg.decode() if msg else ""
