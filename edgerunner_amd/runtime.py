"""Python host layer over the EdgeRunnerHIP C ABI.

Mirrors the Swift host objects the Metal path is driven by:
  - ``Context``     : the device + loaded code object (MetalBackend/KernelRegistry)
  - ``Buffer``      : device memory with a length (MTLBuffer)
  - ``Stream``      : the ordered work queue encodes go to (MTLCommandBuffer)
  - ``Event``       : GPU timestamps (commandBuffer.gpuStartTime/gpuEndTime)
  - ``GEMVError`` / ``DequantKernelError`` : the reference's Swift error enums
    (Sources/EdgeRunnerMetal/GEMVKernel.swift:1435-1441,
     Sources/EdgeRunnerIO/DequantKernel.swift:19-25).
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np

from . import _ffi


# --------------------------------------------------------------------------- errors
class EdgeRunnerHIPError(Exception):
    status = -1

    def __init__(self, message: str = ""):
        super().__init__(message)
        self.message = message


class GEMVError(EdgeRunnerHIPError):
    """GEMVError (GEMVKernel.swift:1435-1441)."""


class LibraryNotFound(GEMVError):
    status = 1


class FunctionNotFound(GEMVError):
    status = 2


class EncodingFailed(GEMVError):
    status = 3


class InvalidMatrixShape(GEMVError):
    status = 4


class InvalidVectorShape(GEMVError):
    status = 5


class DequantKernelError(EdgeRunnerHIPError):
    """DequantKernelError (DequantKernel.swift:19-25)."""


class InvalidBlockDataCount(DequantKernelError):
    status = 6

    def __init__(self, message: str = "", expected: Optional[int] = None,
                 actual: Optional[int] = None):
        super().__init__(message)
        self.expected = expected
        self.actual = actual


class AllocationFailed(DequantKernelError):
    status = 7


class InvalidArgument(EdgeRunnerHIPError):
    status = 8


class DeviceError(EdgeRunnerHIPError):
    status = 9


class WeightLoaderError(EdgeRunnerHIPError):
    """WeightLoaderError (Sources/EdgeRunnerIO/WeightLoaderError.swift:3-15)."""


class FileNotFound(WeightLoaderError):
    status = 10


class InvalidFormat(WeightLoaderError):
    status = 11


class UnsupportedVersion(WeightLoaderError):
    status = 12


class UnsupportedDataType(WeightLoaderError):
    status = 13


class MmapFailed(WeightLoaderError):
    status = 14


class MissingMetadata(WeightLoaderError):
    status = 15


class TensorNotFound(WeightLoaderError):
    status = 16


_BY_STATUS = {cls.status: cls for cls in (
    LibraryNotFound, FunctionNotFound, EncodingFailed, InvalidMatrixShape, InvalidVectorShape,
    InvalidBlockDataCount, AllocationFailed, InvalidArgument, DeviceError, FileNotFound,
    InvalidFormat, UnsupportedVersion, UnsupportedDataType, MmapFailed, MissingMetadata,
    TensorNotFound)}


def check(status: int, lib=None) -> None:
    """Raise the error class of a non-OK status with the message `lib` (the
    library that returned it; default the product library) recorded."""
    if status == _ffi.ER_OK:
        return
    cls = _BY_STATUS.get(status, EdgeRunnerHIPError)
    raise cls(f"{_ffi.STATUS_NAMES.get(status, status)}: {_ffi.last_error(lib)}")


# --------------------------------------------------------------------------- objects
class Buffer:
    """Device memory plus its byte length (the MTLBuffer analogue)."""

    def __init__(self, ctx: "Context", raw: _ffi.er_buffer, owned: bool = True):
        self.ctx = ctx
        self.raw = raw
        self.owned = owned

    @property
    def length(self) -> int:
        return int(self.raw.length)

    @property
    def ptr(self) -> int:
        return int(self.raw.data or 0)

    def view(self, offset: int = 0, length: Optional[int] = None) -> "Buffer":
        """A non-owning sub-range (for byteOffset-style tensor views)."""
        if length is None:
            length = self.length - offset
        if offset < 0 or length < 0 or offset + length > self.length:
            raise InvalidArgument("view out of range")
        return Buffer(self.ctx, _ffi.er_buffer(self.ptr + offset, length), owned=False)

    def upload(self, host: np.ndarray, offset: int = 0, stream: "Optional[Stream]" = None) -> None:
        a = np.ascontiguousarray(host)
        self.ctx.check(self.ctx.lib.er_hip_upload(self.ctx.handle, _sh(stream), self.raw, offset,
                                         a.ctypes.data_as(C.c_void_p), a.nbytes))

    def download(self, dtype, count: Optional[int] = None, offset: int = 0,
                 stream: "Optional[Stream]" = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.length - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        self.ctx.check(self.ctx.lib.er_hip_download(self.ctx.handle, _sh(stream),
                                           out.ctypes.data_as(C.c_void_p), self.raw, offset,
                                           out.nbytes))
        return out

    def copy_from(self, src: "Buffer", nbytes: Optional[int] = None, dst_offset: int = 0,
                  src_offset: int = 0, stream: "Optional[Stream]" = None) -> None:
        """Device-to-device copy enqueued on `stream`."""
        n = src.length - src_offset if nbytes is None else nbytes
        self.ctx.check(self.ctx.lib.er_hip_copy(self.ctx.handle, _sh(stream), self.raw, dst_offset, src.raw,
                                       src_offset, n))

    def free(self) -> None:
        if self.owned and self.raw.data:
            self.ctx.check(self.ctx.lib.er_hip_free(self.ctx.handle, self.raw))
        self.raw = _ffi.er_buffer(None, 0)

    def __del__(self):
        try:
            if self.owned and self.raw.data and self.ctx.handle:
                self.ctx.lib.er_hip_free(self.ctx.handle, self.raw)
        except Exception:
            pass


class Stream:
    def __init__(self, ctx: "Context"):
        self.ctx = ctx
        h = C.c_void_p()
        ctx.check(ctx.lib.er_hip_stream_create(ctx.handle, C.byref(h)))
        self.handle = h

    def synchronize(self) -> None:
        self.ctx.check(self.ctx.lib.er_hip_synchronize(self.ctx.handle, self.handle))

    def destroy(self) -> None:
        if self.handle:
            self.ctx.check(self.ctx.lib.er_hip_stream_destroy(self.ctx.handle, self.handle))
            self.handle = C.c_void_p()


class Event:
    def __init__(self, ctx: "Context"):
        self.ctx = ctx
        h = C.c_void_p()
        ctx.check(ctx.lib.er_hip_event_create(ctx.handle, C.byref(h)))
        self.handle = h

    def record(self, stream: "Optional[Stream]" = None) -> None:
        self.ctx.check(self.ctx.lib.er_hip_event_record(self.ctx.handle, self.handle, _sh(stream)))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        self.ctx.check(self.ctx.lib.er_hip_event_elapsed_ms(self.ctx.handle, self.handle, end.handle,
                                                   C.byref(ms)))
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            self.ctx.check(self.ctx.lib.er_hip_event_destroy(self.ctx.handle, self.handle))
            self.handle = C.c_void_p()


class Graph:
    """A recorded sequence of encodes, replayed with launch() (hipGraphExec)."""

    def __init__(self, ctx: "Context", handle):
        self.ctx = ctx
        self.handle = handle

    def launch(self, stream: "Optional[Stream]" = None) -> None:
        self.ctx.check(self.ctx.lib.er_hip_graph_launch(self.ctx.handle, self.handle, _sh(stream)))

    def destroy(self) -> None:
        if self.handle:
            self.ctx.check(self.ctx.lib.er_hip_graph_destroy(self.ctx.handle, self.handle))
            self.handle = C.c_void_p()


class Capture:
    """Context manager recording every encode on `stream` into a Graph:

        with Capture(ctx, stream) as cap:
            gemv.encodeQ4KWeights(stream, ...)
        cap.graph.launch(stream)
    """

    def __init__(self, ctx: "Context", stream: "Stream"):
        self.ctx = ctx
        self.stream = stream
        self.graph: Optional[Graph] = None

    def __enter__(self) -> "Capture":
        self.ctx.check(self.ctx.lib.er_hip_graph_begin(self.ctx.handle, self.stream.handle))
        return self

    def __exit__(self, exc_type, exc, tb) -> bool:
        h = C.c_void_p()
        st = self.ctx.lib.er_hip_graph_end(self.ctx.handle, self.stream.handle, C.byref(h))
        if exc_type is None:
            self.ctx.check(st)
            self.graph = Graph(self.ctx, h)
        elif st == _ffi.ER_OK and h:
            self.ctx.lib.er_hip_graph_destroy(self.ctx.handle, h)
        return False


def _sh(stream: Optional[Stream]):
    return stream.handle if stream is not None else None


class Context:
    """One GPU with the gfx950 code object loaded and every kernel resolved."""

    def __init__(self, device: int = 0, probes: bool = False):
        # probes: a context of the measurement library (libedgerunner_probe.so)
        self.lib = _ffi.load_probe() if probes else _ffi.load()
        h = C.c_void_p()
        self.check(self.lib.er_hip_create(device, C.byref(h)))
        self.handle = h
        info = _ffi.er_device_info()
        self.check(self.lib.er_hip_get_device_info(self.handle, C.byref(info)))
        self.info = info

    def check(self, status: int) -> None:
        check(status, self.lib)

    @property
    def compute_units(self) -> int:
        return int(self.info.compute_units)

    @property
    def arch(self) -> str:
        return self.info.arch.decode()

    def alloc(self, nbytes: int) -> Buffer:
        raw = _ffi.er_buffer()
        self.check(self.lib.er_hip_alloc(self.handle, nbytes, C.byref(raw)))
        return Buffer(self, raw)

    def upload(self, host: np.ndarray, stream: Optional[Stream] = None) -> Buffer:
        a = np.ascontiguousarray(host)
        buf = self.alloc(a.nbytes)
        buf.upload(a, stream=stream)
        return buf

    def stream(self) -> Stream:
        return Stream(self)

    def event(self) -> Event:
        return Event(self)

    def synchronize(self, stream: Optional[Stream] = None) -> None:
        self.check(self.lib.er_hip_synchronize(self.handle, _sh(stream)))

    def close(self) -> None:
        if self.handle:
            self.lib.er_hip_destroy(self.handle)
            self.handle = C.c_void_p()


_default: Optional[Context] = None


def default_context() -> Context:
    global _default
    if _default is None:
        _default = Context(0)
    return _default
