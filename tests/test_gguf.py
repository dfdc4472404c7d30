"""GGUF parsing and loader checks on the CPU (host code of er_gguf.cpp; no
device needed).  The cases restate the reference's parser and loader tests
(Tests/EdgeRunnerIOTests/GGUFHeaderTests.swift, GGUFTensorTableTests.swift)
on bytes built the way their GGUFBuilder builds them, plus the limits and
error paths of GGUFParser.swift and GGUFLoader.swift, and truncation at
every byte of a small file (each prefix parses or raises WeightLoaderError,
never anything else)."""
import struct

import pytest

from edgerunner_amd import (FileNotFound, InvalidFormat, MissingMetadata, UnsupportedDataType,
                            UnsupportedVersion, WeightLoaderError)
from edgerunner_amd.gguf import (GGUFHeader, GGUFLoader, GGUFMetadataValueType as VT, GGUFReader,
                                 GGUFTensorType as TT, TensorDataType, build_gguf, tensorByteCount,
                                 write_gguf)

MAGIC = 0x46554747


class Builder:
    """The reference tests' GGUFBuilder (GGUFTensorTableTests.swift:346-363)."""

    def __init__(self):
        self.data = bytearray()

    def u32(self, v):
        self.data += struct.pack("<I", v)
        return self

    def u64(self, v):
        self.data += struct.pack("<Q", v)
        return self

    def raw(self, b):
        self.data += b
        return self

    def string(self, s):
        b = s.encode() if isinstance(s, str) else s
        return self.u64(len(b)).raw(b)


def header(version=3, tensors=0, kvs=0):
    return Builder().u32(MAGIC).u32(version).u64(tensors).u64(kvs)


# ---- GGUFHeaderTests ---------------------------------------------------------
def test_parse_magic_and_version():
    h = GGUFHeader.parse(bytes(header().data))
    assert (h.version, h.tensorCount, h.metadataKVCount) == (3, 0, 0)


def test_reject_invalid_magic():
    with pytest.raises(InvalidFormat):
        GGUFHeader.parse(bytes(Builder().u32(0xDEADBEEF).u32(3).u64(0).u64(0).data))


@pytest.mark.parametrize("version", [1, 4, 0xFFFFFFFF])
def test_reject_unsupported_version(version):
    with pytest.raises(UnsupportedVersion):
        GGUFHeader.parse(bytes(header(version).data))


def test_parse_version2_header_only():
    h = GGUFHeader.parse(bytes(header(2, 5, 2).data))
    assert (h.version, h.tensorCount, h.metadataKVCount) == (2, 5, 2)


def kv(b, key, vtype, payload: bytes):
    return b.string(key).u32(int(vtype)).raw(payload)


@pytest.mark.parametrize("vtype,payload,expected", [
    (VT.string, struct.pack("<Q", 5) + b"llama", "llama"),
    (VT.uint32, struct.pack("<I", 4096), 4096),
    (VT.int32, struct.pack("<i", -42), -42),
    (VT.float32, struct.pack("<f", 500000.0), 500000.0),
    (VT.bool, b"\x01", True),
    (VT.uint64, struct.pack("<Q", 1_234_567_890), 1_234_567_890),
    (VT.int64, struct.pack("<q", -99), -99),
    (VT.float64, struct.pack("<d", 3.5), 3.5),
    (VT.uint8, b"\xff", 255), (VT.int8, b"\x80", -128),
    (VT.uint16, struct.pack("<H", 65535), 65535), (VT.int16, struct.pack("<h", -2), -2),
])
def test_parse_scalar_metadata(vtype, payload, expected):
    b = kv(header(kvs=1), "k", vtype, payload)
    md = GGUFReader(bytes(b.data)).readMetadata()
    assert md == {"k": expected}
    assert GGUFReader(bytes(b.data)).metadataTypes()["k"] == vtype


def test_parse_array_metadata():
    arr = struct.pack("<IQ", int(VT.uint32), 4) + b"".join(struct.pack("<I", v) for v in (1, 2, 3, 4))
    md = GGUFReader(bytes(kv(header(kvs=1), "a", VT.array, arr).data)).readMetadata()
    assert md == {"a": [1, 2, 3, 4]}


def test_parse_string_and_nested_arrays():
    strs = struct.pack("<IQ", int(VT.string), 3) + b"".join(
        struct.pack("<Q", len(s)) + s for s in (b"a", b"", "é中".encode()))
    inner = struct.pack("<IQ", int(VT.int8), 2) + b"\x01\xff"
    nested = struct.pack("<IQ", int(VT.array), 2) + inner + inner
    b = kv(kv(header(kvs=2), "tok", VT.array, strs), "nest", VT.array, nested)
    md = GGUFReader(bytes(b.data)).readMetadata()
    assert md == {"tok": ["a", "", "é中"], "nest": [[1, -1], [1, -1]]}


def test_parse_multiple_metadata_entries_and_model_config_keys():
    b = header(kvs=3)
    kv(b, "general.architecture", VT.string, struct.pack("<Q", 5) + b"llama")
    kv(b, "llama.block_count", VT.uint32, struct.pack("<I", 32))
    kv(b, "llama.attention.head_count", VT.uint32, struct.pack("<I", 32))
    md = GGUFReader(bytes(b.data)).readMetadata()
    assert md == {"general.architecture": "llama", "llama.block_count": 32,
                  "llama.attention.head_count": 32}


def test_repeated_key_keeps_last_value():
    b = header(kvs=2)
    kv(b, "x", VT.uint32, struct.pack("<I", 1))
    kv(b, "x", VT.int32, struct.pack("<i", -7))
    assert GGUFReader(bytes(b.data)).readMetadata() == {"x": -7}


@pytest.mark.parametrize("mutate", ["type", "string_len", "utf8", "elem_type", "truncated"])
def test_metadata_errors_are_invalid_format(mutate):
    b = header(kvs=1)
    if mutate == "type":
        kv(b, "k", 13, b"\0" * 8)
    elif mutate == "string_len":
        b.string("k").u32(int(VT.string)).u64(1_000_001)
    elif mutate == "utf8":
        kv(b, "k", VT.string, struct.pack("<Q", 2) + b"\xc3\x28")
    elif mutate == "elem_type":
        kv(b, "k", VT.array, struct.pack("<IQ", 99, 1))
    else:
        kv(b, "k", VT.uint64, b"\0\0\0")
    with pytest.raises(InvalidFormat):
        GGUFReader(bytes(b.data)).readMetadata()


def test_huge_array_count_fails_without_allocating():
    b = kv(header(kvs=1), "k", VT.array, struct.pack("<IQ", int(VT.uint8), 2 ** 62) + b"\0" * 16)
    with pytest.raises(InvalidFormat):
        GGUFReader(bytes(b.data)).readMetadata()


# ---- GGUFTensorTableTests ----------------------------------------------------
def tensor_entry(b, name, dims, ttype, offset):
    b.string(name).u32(len(dims))
    for d in dims:
        b.u64(d)
    return b.u32(int(ttype)).u64(offset)


def test_parse_single_tensor_info():
    b = tensor_entry(header(tensors=1), "output.weight", [4096, 32000], TT.f16, 0)
    r = GGUFReader(bytes(b.data))
    assert r.readMetadata() == {}
    infos = r.readTensorInfos()
    assert len(infos) == 1
    i = infos[0]
    assert (i.name, i.dimensions, i.type, i.offset) == ("output.weight", (4096, 32000), TT.f16, 0)


def test_parse_multiple_tensor_infos():
    b = header(tensors=3)
    tensor_entry(b, "token_embd.weight", [32000, 4096], TT.f16, 0)
    tensor_entry(b, "blk.0.attn_q.weight", [4096, 4096], TT.q8_0, 262_144_000)
    tensor_entry(b, "blk.0.ffn_gate.weight", [4096, 11008], TT.q4_0, 295_698_432)
    infos = GGUFReader(bytes(b.data)).readTensorInfos()
    assert [(i.name, i.type) for i in infos] == [
        ("token_embd.weight", TT.f16), ("blk.0.attn_q.weight", TT.q8_0),
        ("blk.0.ffn_gate.weight", TT.q4_0)]


def test_modern_tensor_type_ordering():
    assert TT(16) == TT.iq2_xxs and TT(23) == TT.iq4_xs and TT(24) == TT.i8
    assert TT(28) == TT.f64 and TT(29) == TT.iq1_m and TT(30) == TT.bf16
    assert TT(34) == TT.tq1_0 and TT(35) == TT.tq2_0 and TT(39) == TT.mxfp4 and TT(40) == TT.nvfp4
    assert TT.bf16.tensorDataType == TensorDataType.bfloat16


DEFERRED = [(TT.iq2_xxs, "IQ2_XXS"), (TT.iq2_xs, "IQ2_XS"), (TT.iq3_xxs, "IQ3_XXS"),
            (TT.iq1_s, "IQ1_S"), (TT.iq4_nl, "IQ4_NL"), (TT.iq3_s, "IQ3_S"), (TT.iq2_s, "IQ2_S"),
            (TT.iq4_xs, "IQ4_XS"), (TT.iq1_m, "IQ1_M"), (TT.tq1_0, "TQ1_0"), (TT.tq2_0, "TQ2_0"),
            (TT.mxfp4, "MXFP4"), (TT.nvfp4, "NVFP4")]


def test_deferred_types_are_explicitly_unsupported():
    for t, name in DEFERRED:
        assert t.tensorDataType is None and t.diagnosticName == name


def test_parse_bf16_tensor_info():
    b = tensor_entry(header(tensors=1), "per_layer_model_proj.weight", [2560, 10752], 30, 0)
    i = GGUFReader(bytes(b.data)).readTensorInfos()[0]
    assert i.type == TT.bf16 and i.type.tensorDataType == TensorDataType.bfloat16


@pytest.mark.parametrize("raw", [0xFF, 4, 5, 31, 36, 42])
def test_reject_unknown_tensor_type(raw):
    b = tensor_entry(header(tensors=1), "bad.weight", [100], raw, 0)
    with pytest.raises(UnsupportedDataType):
        GGUFReader(bytes(b.data)).readTensorInfos()


def test_reject_too_many_dimensions():
    b = tensor_entry(header(tensors=1), "t", [1] * 9, TT.f32, 0)
    with pytest.raises(InvalidFormat):
        GGUFReader(bytes(b.data)).readTensorInfos()


# ---- loader (GGUFLoader.load checks) --------------------------------------------
ARCH = [("general.architecture", VT.string, "llama")]
MOBILE = [(TT.f16, [256], 512), (TT.bf16, [256], 512), (TT.q2_K, [256], 84),
          (TT.q3_K, [256], 110), (TT.q4_K, [256], 144), (TT.q5_K, [256], 176),
          (TT.q6_K, [256], 210), (TT.q8_0, [32], 34)]


def single_tensor_file(tmp_path, ttype, dims, payload_bytes, metadata=ARCH):
    """writeSingleTensorGGUF (GGUFTensorTableTests.swift:242-273)."""
    return write_gguf(tmp_path / f"t_{int(ttype)}.gguf", metadata,
                      [("test.weight", dims, ttype, bytes(payload_bytes))])


@pytest.mark.parametrize("ttype,dims,nbytes", MOBILE)
def test_loader_accepts_mobile_quant_byte_counts(tmp_path, ttype, dims, nbytes):
    ld = GGUFLoader(single_tensor_file(tmp_path, ttype, dims, nbytes))
    (info,) = ld.tensorInfos
    assert info.type.tensorDataType == ttype.tensorDataType
    assert info.elementCount == dims[0]
    assert tensorByteCount(info) == nbytes
    assert ld.architectureName == "llama"


@pytest.mark.parametrize("ttype,dims,nbytes", MOBILE)
def test_loader_rejects_truncated_payloads(tmp_path, ttype, dims, nbytes):
    with pytest.raises(InvalidFormat):
        GGUFLoader(single_tensor_file(tmp_path, ttype, dims, nbytes - 1))


@pytest.mark.parametrize("ttype", [t for t, _ in DEFERRED])
def test_loader_rejects_deferred_types(tmp_path, ttype):
    with pytest.raises(UnsupportedDataType) as e:
        GGUFLoader(single_tensor_file(tmp_path, ttype, [256], 0))
    assert f"({int(ttype)})" in str(e.value)


def test_loader_requires_architecture(tmp_path):
    with pytest.raises(MissingMetadata):
        GGUFLoader(single_tensor_file(tmp_path, TT.q8_0, [32], 34, metadata=[]))


def test_loader_rejects_uint64_metadata_beyond_int(tmp_path):
    md = ARCH + [("general.size", VT.uint64, 2 ** 63)]
    with pytest.raises(InvalidFormat):
        GGUFLoader(single_tensor_file(tmp_path, TT.q8_0, [32], 34, metadata=md))


def test_loader_file_not_found_and_can_load(tmp_path):
    with pytest.raises(FileNotFound):
        GGUFLoader(tmp_path / "missing.gguf")
    assert GGUFLoader.canLoad("/tmp/model.gguf") and GGUFLoader.canLoad("/x/M.GGUF")
    assert not GGUFLoader.canLoad("/tmp/model.safetensors")


def test_loader_offsets_host_bytes_and_alignment(tmp_path):
    """Tensor bytes come back from their offsets in the data section; the
    data section starts at 32 by default and at general.alignment when set."""
    pay = [bytes((i * 7 + k) % 251 for i in range(n)) for k, n in enumerate((34 * 3, 144, 210 * 2))]
    tensors = [("a", [96], TT.q8_0, pay[0]), ("b", [256], TT.q4_K, pay[1]),
               ("c", [256, 2], TT.q6_K, pay[2])]
    for align in (32, 64, 4096):
        md = ARCH + ([("general.alignment", VT.uint32, align)] if align != 32 else [])
        p = write_gguf(tmp_path / f"m{align}.gguf", md, tensors, alignment=align)
        ld = GGUFLoader(p)
        off, n = ld.dataSection()
        assert off % align == 0 and off + n == p.stat().st_size
        for (name, _, _, b) in tensors:
            assert bytes(ld.hostTensor(name)) == b
        infos = {i.name: i for i in ld.tensorInfos}
        assert infos["c"].dimensions == (256, 2) and infos["b"].offset % align == 0


def test_bad_general_alignment_is_rejected(tmp_path):
    md = ARCH + [("general.alignment", VT.uint32, 48)]
    with pytest.raises(InvalidFormat):
        GGUFLoader(write_gguf(tmp_path / "bad.gguf", md, [("a", [32], TT.q8_0, bytes(34))]))


def test_every_truncation_raises_loader_error(tmp_path):
    data = build_gguf(ARCH + [("tok", VT.array, (VT.string, ["x", "yz"]))],
                      [("a", [32], TT.q8_0, bytes(range(34))), ("b", [256], TT.q4_K, bytes(144))])
    for cut in range(0, len(data)):
        p = tmp_path / "cut.gguf"
        p.write_bytes(data[:cut])
        with pytest.raises(WeightLoaderError):
            GGUFLoader(p)
    p.write_bytes(data)
    assert [i.name for i in GGUFLoader(p).tensorInfos] == ["a", "b"]
