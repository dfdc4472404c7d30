"""GGUF weights into HBM: the host-side mirror of the reference's GGUF
reader and loader (Sources/EdgeRunnerIO/GGUF/GGUFParser.swift,
GGUFLoader.swift, GGUFTypes.swift), over the native parser and uploader of
include/er_gguf.h.

    loader = GGUFLoader(path)           # map + parse + the loader's checks
    weights = loader.load(ctx)          # data section -> one HBM buffer
    t = weights["blk.0.attn_q.weight"]  # TensorStorage view (dataType, shape)
    GEMVKernel(ctx).encodeTensor(stream, t, x, y)

`GGUFReader(data)` parses bytes in memory step by step (readHeader,
readMetadata, readTensorInfos) with the reference reader's errors;
`write_gguf` writes a GGUF file (synthetic models for tests and benches).
"""
from __future__ import annotations

import ctypes as C
import enum
import struct
from dataclasses import dataclass, field
from pathlib import Path
from typing import Dict, Iterable, List, Optional, Sequence, Tuple, Union

import numpy as np

from . import _ffi
from .runtime import Buffer, Context, Stream, _sh, check, default_context

GGUF_MAGIC = 0x46554747
GGUF_DEFAULT_ALIGNMENT = 32


class GGUFMetadataValueType(enum.IntEnum):
    """GGUFTypes.swift:6-20."""
    uint8 = 0
    int8 = 1
    uint16 = 2
    int16 = 3
    uint32 = 4
    int32 = 5
    float32 = 6
    bool = 7
    string = 8
    array = 9
    uint64 = 10
    int64 = 11
    float64 = 12


class TensorDataType(enum.IntEnum):
    """WeightMap.swift:69-91."""
    float32 = 0
    float16 = 1
    q4_0 = 2
    q4_1 = 3
    q5_0 = 6
    q5_1 = 7
    q8_0 = 8
    q8_1 = 9
    q2_K = 10
    q3_K = 11
    q4_K = 12
    q5_K = 13
    q6_K = 14
    q8_K = 15
    i8 = 16
    i16 = 17
    i32 = 18
    i64 = 19
    f64 = 20
    bfloat16 = 30
    q1_0_g128 = 41


class GGUFTensorType(enum.IntEnum):
    """GGUFTypes.swift:22-57."""
    f32 = 0
    f16 = 1
    q4_0 = 2
    q4_1 = 3
    q5_0 = 6
    q5_1 = 7
    q8_0 = 8
    q8_1 = 9
    q2_K = 10
    q3_K = 11
    q4_K = 12
    q5_K = 13
    q6_K = 14
    q8_K = 15
    iq2_xxs = 16
    iq2_xs = 17
    iq3_xxs = 18
    iq1_s = 19
    iq4_nl = 20
    iq3_s = 21
    iq2_s = 22
    iq4_xs = 23
    i8 = 24
    i16 = 25
    i32 = 26
    i64 = 27
    f64 = 28
    iq1_m = 29
    bf16 = 30
    tq1_0 = 34
    tq2_0 = 35
    mxfp4 = 39
    nvfp4 = 40
    q1_0_g128 = 41

    @property
    def tensorDataType(self) -> Optional[TensorDataType]:
        """GGUFTypes.swift:59-85: None for the deferred upstream types."""
        return _DATA_TYPE.get(self)

    @property
    def diagnosticName(self) -> str:
        return _DIAG.get(self, self.name.upper())

    @property
    def block(self) -> Optional[Tuple[int, int]]:
        """(elements, bytes) per block as GGUFLoader.tensorByteCount sizes it."""
        return _BLOCK.get(self)


_DATA_TYPE = {
    GGUFTensorType.f32: TensorDataType.float32, GGUFTensorType.f16: TensorDataType.float16,
    GGUFTensorType.q4_0: TensorDataType.q4_0, GGUFTensorType.q4_1: TensorDataType.q4_1,
    GGUFTensorType.q5_0: TensorDataType.q5_0, GGUFTensorType.q5_1: TensorDataType.q5_1,
    GGUFTensorType.q8_0: TensorDataType.q8_0, GGUFTensorType.q8_1: TensorDataType.q8_1,
    GGUFTensorType.q2_K: TensorDataType.q2_K, GGUFTensorType.q3_K: TensorDataType.q3_K,
    GGUFTensorType.q4_K: TensorDataType.q4_K, GGUFTensorType.q5_K: TensorDataType.q5_K,
    GGUFTensorType.q6_K: TensorDataType.q6_K, GGUFTensorType.q8_K: TensorDataType.q8_K,
    GGUFTensorType.i8: TensorDataType.i8, GGUFTensorType.i16: TensorDataType.i16,
    GGUFTensorType.i32: TensorDataType.i32, GGUFTensorType.i64: TensorDataType.i64,
    GGUFTensorType.f64: TensorDataType.f64, GGUFTensorType.bf16: TensorDataType.bfloat16,
    GGUFTensorType.q1_0_g128: TensorDataType.q1_0_g128,
}
_DIAG = {GGUFTensorType.q2_K: "Q2_K", GGUFTensorType.q3_K: "Q3_K", GGUFTensorType.q4_K: "Q4_K",
         GGUFTensorType.q5_K: "Q5_K", GGUFTensorType.q6_K: "Q6_K", GGUFTensorType.q8_K: "Q8_K"}
_BLOCK = {
    GGUFTensorType.f32: (1, 4), GGUFTensorType.f16: (1, 2), GGUFTensorType.q4_0: (32, 18),
    GGUFTensorType.q4_1: (32, 20), GGUFTensorType.q5_0: (32, 22), GGUFTensorType.q5_1: (32, 24),
    GGUFTensorType.q8_0: (32, 34), GGUFTensorType.q8_1: (32, 36), GGUFTensorType.q2_K: (256, 84),
    GGUFTensorType.q3_K: (256, 110), GGUFTensorType.q4_K: (256, 144),
    GGUFTensorType.q5_K: (256, 176), GGUFTensorType.q6_K: (256, 210),
    GGUFTensorType.q8_K: (256, 292), GGUFTensorType.i8: (1, 1), GGUFTensorType.i16: (1, 2),
    GGUFTensorType.i32: (1, 4), GGUFTensorType.i64: (1, 8), GGUFTensorType.f64: (1, 8),
    GGUFTensorType.bf16: (1, 2), GGUFTensorType.q1_0_g128: (128, 18),
}


@dataclass(frozen=True)
class GGUFHeader:
    """GGUFTypes.swift:124-133."""
    version: int
    tensorCount: int
    metadataKVCount: int

    @staticmethod
    def parse(data: bytes) -> "GGUFHeader":
        return GGUFReader(data).readHeader()


@dataclass(frozen=True)
class GGUFTensorInfo:
    """GGUFTypes.swift:135-149."""
    name: str
    dimensions: Tuple[int, ...]
    type: GGUFTensorType
    offset: int

    @property
    def elementCount(self) -> int:
        n = 1
        for d in self.dimensions:
            n *= d
        return n


@dataclass
class TensorStorage:
    """TensorStorage (WeightMap.swift:93-127): a view into the device copy of
    the data section.  `storage` is the er_tensor_storage encodeProjection takes."""
    buffer: Buffer
    byteOffset: int
    dataType: TensorDataType
    shape: Tuple[int, ...]
    name: str
    byteCount: int
    storage: _ffi.er_tensor_storage = field(repr=False, default=None)

    @property
    def elementCount(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


class _Handle:
    """Owns one native er_gguf."""

    def __init__(self, ptr: int):
        self.lib = _ffi.load()
        self.ptr = ptr

    def close(self) -> None:
        if self.ptr:
            self.lib.er_gguf_close(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def header(self) -> GGUFHeader:
        v, t, k = C.c_uint32(), C.c_uint64(), C.c_uint64()
        check(self.lib.er_gguf_header(self.ptr, C.byref(v), C.byref(t), C.byref(k)))
        return GGUFHeader(v.value, t.value, k.value)

    def _value(self, v: _ffi.er_gguf_value):
        t = GGUFMetadataValueType(v.type)
        if t == GGUFMetadataValueType.string:
            return C.string_at(v.str, v.count).decode("utf-8") if v.count else ""
        if t == GGUFMetadataValueType.array:
            out = []
            e = _ffi.er_gguf_value()
            for j in range(v.count):
                check(self.lib.er_gguf_array_get(self.ptr, v.node, j, C.byref(e)))
                out.append(self._value(e))
            return out
        if t == GGUFMetadataValueType.bool:
            return bool(v.u)
        if t in (GGUFMetadataValueType.float32, GGUFMetadataValueType.float64):
            return float(v.f)
        if t in (GGUFMetadataValueType.int8, GGUFMetadataValueType.int16,
                 GGUFMetadataValueType.int32, GGUFMetadataValueType.int64):
            return int(v.i)
        return int(v.u)

    def metadata(self) -> Dict[str, object]:
        out = {}
        key = C.c_char_p()
        v = _ffi.er_gguf_value()
        for i in range(self.lib.er_gguf_metadata_count(self.ptr)):
            check(self.lib.er_gguf_metadata_key(self.ptr, i, C.byref(key)))
            check(self.lib.er_gguf_metadata_value(self.ptr, i, C.byref(v)))
            out[key.value.decode("utf-8")] = self._value(v)
        return out

    def metadata_types(self) -> Dict[str, GGUFMetadataValueType]:
        out = {}
        key = C.c_char_p()
        v = _ffi.er_gguf_value()
        for i in range(self.lib.er_gguf_metadata_count(self.ptr)):
            check(self.lib.er_gguf_metadata_key(self.ptr, i, C.byref(key)))
            check(self.lib.er_gguf_metadata_value(self.ptr, i, C.byref(v)))
            out[key.value.decode("utf-8")] = GGUFMetadataValueType(v.type)
        return out

    def tensor_infos(self) -> List[Tuple[GGUFTensorInfo, _ffi.er_gguf_tensor_info]]:
        out = []
        for i in range(self.lib.er_gguf_tensor_count(self.ptr)):
            ti = _ffi.er_gguf_tensor_info()
            check(self.lib.er_gguf_tensor_info_at(self.ptr, i, C.byref(ti)))
            info = GGUFTensorInfo(ti.name.decode("utf-8"), tuple(ti.dims[d] for d in range(ti.ndim)),
                                  GGUFTensorType(ti.ggml_type), ti.offset)
            out.append((info, ti))
        return out


class GGUFReader:
    """GGUFReader (GGUFParser.swift:3-205) over bytes in memory.  Each step
    parses from the start up to that part, so errors surface at the step the
    reference raises them."""

    def __init__(self, data: bytes):
        self.data = bytes(data)
        self._header: Optional[GGUFHeader] = None

    def _parse(self, parts: int) -> _Handle:
        lib = _ffi.load()
        buf = C.create_string_buffer(self.data, len(self.data)) if self.data else None
        out = C.c_void_p()
        check(lib.er_gguf_parse_memory(buf, len(self.data), parts, C.byref(out)))
        return _Handle(out.value)

    def readHeader(self) -> GGUFHeader:
        h = self._parse(1)
        try:
            self._header = h.header()
            return self._header
        finally:
            h.close()

    def readMetadata(self, count: Optional[int] = None) -> Dict[str, object]:
        h = self._parse(2)
        try:
            return h.metadata()
        finally:
            h.close()

    def readTensorInfos(self, count: Optional[int] = None) -> List[GGUFTensorInfo]:
        h = self._parse(3)
        try:
            return [info for info, _ in h.tensor_infos()]
        finally:
            h.close()

    def metadataTypes(self) -> Dict[str, GGUFMetadataValueType]:
        h = self._parse(2)
        try:
            return h.metadata_types()
        finally:
            h.close()


def tensorByteCount(info: GGUFTensorInfo) -> int:
    """GGUFLoader.tensorByteCount (GGUFLoader.swift:125-179)."""
    from .runtime import UnsupportedDataType
    blk = info.type.block
    if blk is None:
        raise UnsupportedDataType(f"unsupportedDataType({int(info.type)})")
    per, nbytes = blk
    return -(-info.elementCount // per) * nbytes


class GGUFLoader:
    """GGUFLoader (GGUFLoader.swift:4-123) for an MI355X host: the file is
    mapped and checked at construction (prepare + load's per-tensor checks);
    load() copies the data section into one HBM buffer and returns the
    tensors as TensorStorage views (a WeightMap as a dict)."""

    def __init__(self, url: Union[str, Path, None] = None):
        self.url = None if url is None else Path(url)
        self._h: Optional[_Handle] = None
        if self.url is not None:
            self._h = self._open(self.url)

    @staticmethod
    def _open(url: Path) -> _Handle:
        lib = _ffi.load()
        out = C.c_void_p()
        check(lib.er_gguf_open(str(url).encode(), C.byref(out)))
        return _Handle(out.value)

    @staticmethod
    def canLoad(url: Union[str, Path]) -> bool:
        return Path(url).suffix.lower() == ".gguf"

    @property
    def header(self) -> GGUFHeader:
        return self._h.header()

    @property
    def metadata(self) -> Dict[str, object]:
        return self._h.metadata()

    @property
    def architectureName(self) -> str:
        return str(self.metadata.get("general.architecture", ""))

    @property
    def tensorInfos(self) -> List[GGUFTensorInfo]:
        return [info for info, _ in self._h.tensor_infos()]

    def dataSection(self) -> Tuple[int, int]:
        off, n = C.c_uint64(), C.c_uint64()
        check(self._h.lib.er_gguf_data_section(self._h.ptr, C.byref(off), C.byref(n)))
        return off.value, n.value

    def hostTensor(self, name: str) -> np.ndarray:
        """The tensor's raw bytes from the mapping (no device involved)."""
        idx = C.c_uint64()
        check(self._h.lib.er_gguf_find_tensor(self._h.ptr, name.encode(), C.byref(idx)))
        p, n = C.c_void_p(), C.c_uint64()
        check(self._h.lib.er_gguf_tensor_host_data(self._h.ptr, idx.value, C.byref(p), C.byref(n)))
        return np.frombuffer(C.string_at(p.value, n.value), dtype=np.uint8).copy()

    def load(self, ctx: Optional[Context] = None, stream: Optional[Stream] = None,
             url: Union[str, Path, None] = None) -> Dict[str, TensorStorage]:
        if url is not None and (self.url is None or Path(url) != self.url):
            self.url = Path(url)
            self._h = self._open(self.url)
        if self._h is None:
            raise ValueError("GGUFLoader.load needs a file")
        ctx = ctx or default_context()
        lib = self._h.lib
        raw = _ffi.er_buffer()
        check(lib.er_hip_gguf_upload(ctx.handle, _sh(stream), self._h.ptr, C.byref(raw)))
        data = Buffer(ctx, raw, owned=True)
        self.deviceData = data
        out: Dict[str, TensorStorage] = {}
        for i, (info, ti) in enumerate(self._h.tensor_infos()):
            st = _ffi.er_tensor_storage()
            check(lib.er_gguf_tensor_storage(self._h.ptr, i, raw, C.byref(st)))
            view = data.view(ti.offset, ti.byte_count)
            view._owner = data  # the views keep the data-section allocation alive
            out.setdefault(info.name, TensorStorage(view, ti.offset, TensorDataType(ti.data_type),
                                                    info.dimensions, info.name, ti.byte_count, st))
        return out

    def close(self) -> None:
        if self._h is not None:
            self._h.close()
            self._h = None


# --------------------------------------------------------------------------- writer
def _pack_value(t: GGUFMetadataValueType, v) -> bytes:
    T = GGUFMetadataValueType
    if t == T.string:
        b = v.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if t == T.array:
        et, items = v
        return struct.pack("<IQ", int(et), len(items)) + b"".join(_pack_value(et, x) for x in items)
    fmt = {T.uint8: "<B", T.int8: "<b", T.uint16: "<H", T.int16: "<h", T.uint32: "<I",
           T.int32: "<i", T.float32: "<f", T.bool: "<B", T.uint64: "<Q", T.int64: "<q",
           T.float64: "<d"}[t]
    return struct.pack(fmt, int(v) if t == T.bool else v)


def build_gguf(metadata: Sequence[Tuple[str, GGUFMetadataValueType, object]],
               tensors: Sequence[Tuple[str, Sequence[int], GGUFTensorType, bytes]],
               version: int = 3, alignment: int = GGUF_DEFAULT_ALIGNMENT) -> bytes:
    """GGUF bytes: header, metadata (array values as (elementType, items)),
    tensor table with offsets laid out at `alignment`, padding, data."""
    head = struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(metadata))
    for k, t, v in metadata:
        head += _pack_value(GGUFMetadataValueType.string, k) + struct.pack("<I", int(t)) + _pack_value(t, v)
    offsets, off = [], 0
    for _, _, _, payload in tensors:
        offsets.append(off)
        off += len(payload)
        off = -(-off // alignment) * alignment
    for (name, dims, ttype, _), o in zip(tensors, offsets):
        head += _pack_value(GGUFMetadataValueType.string, name)
        head += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", int(ttype), o)
    head += b"\0" * (-len(head) % alignment)
    body = bytearray()
    for (_, _, _, payload), o in zip(tensors, offsets):
        body += b"\0" * (o - len(body))
        body += payload
    return bytes(head) + bytes(body)


def write_gguf(path: Union[str, Path], metadata, tensors, version: int = 3,
               alignment: int = GGUF_DEFAULT_ALIGNMENT) -> Path:
    path = Path(path)
    path.write_bytes(build_gguf(metadata, tensors, version, alignment))
    return path
