// er_gguf.cpp -- GGUF parsing and HBM upload (include/er_gguf.h).
//
// Parser: a bounds-checked little-endian cursor over the mapped bytes with
// the reference's limits and error cases (GGUFReader,
// Sources/EdgeRunnerIO/GGUF/GGUFParser.swift:3-205).  Loader checks follow
// GGUFLoader.prepare / load / tensorByteCount (GGUFLoader.swift:35-179).
// Upload: the data section goes to HBM in one allocation through a ring of
// two pinned staging buffers; each chunk's page copy is split over host
// threads and overlaps the previous chunk's DMA.
#include "er_gguf.h"
#include "er_error.h"

#include <hip/hip_runtime_api.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

using er_detail::fail;

namespace {

struct Value {
    uint32_t type = 0, elemType = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string str;
    std::vector<Value> items;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
};

// GGUFTensorType (GGUFTypes.swift:22-57): per raw value, whether the enum
// knows it, the block (elements, bytes) GGUFLoader.tensorByteCount uses
// (0 bytes: a type it refuses to size), and the TensorDataType raw value.
struct TypeRow {
    bool known;
    uint32_t blockElems, blockBytes, dataType;
};

TypeRow type_row(uint32_t t) {
    const uint32_t N = ER_DATA_TYPE_NONE;
    switch (t) {
        case 0: return {true, 1, 4, 0};        // f32
        case 1: return {true, 1, 2, 1};        // f16
        case 2: return {true, 32, 18, 2};      // q4_0
        case 3: return {true, 32, 20, 3};      // q4_1
        case 6: return {true, 32, 22, 6};      // q5_0
        case 7: return {true, 32, 24, 7};      // q5_1
        case 8: return {true, 32, 34, 8};      // q8_0
        case 9: return {true, 32, 36, 9};      // q8_1
        case 10: return {true, 256, 84, 10};   // q2_K
        case 11: return {true, 256, 110, 11};  // q3_K
        case 12: return {true, 256, 144, 12};  // q4_K
        case 13: return {true, 256, 176, 13};  // q5_K
        case 14: return {true, 256, 210, 14};  // q6_K
        case 15: return {true, 256, 292, 15};  // q8_K
        case 24: return {true, 1, 1, 16};      // i8
        case 25: return {true, 1, 2, 17};      // i16
        case 26: return {true, 1, 4, 18};      // i32
        case 27: return {true, 1, 8, 19};      // i64
        case 28: return {true, 1, 8, 20};      // f64
        case 30: return {true, 1, 2, 30};      // bf16
        case 41: return {true, 128, 18, 41};   // q1_0_g128
        // deferred upstream types: known, never sized or loaded
        case 16: case 17: case 18: case 19: case 20: case 21: case 22: case 23:
        case 29: case 34: case 35: case 39: case 40:
            return {true, 0, 0, N};
        default: return {false, 0, 0, N};
    }
}

// RFC 3629 UTF-8 (no overlongs, no surrogates, at most U+10FFFF).
bool valid_utf8(const uint8_t *p, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = p[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        uint32_t len, cp;
        if ((c & 0xe0) == 0xc0) len = 2, cp = c & 0x1f;
        else if ((c & 0xf0) == 0xe0) len = 3, cp = c & 0x0f;
        else if ((c & 0xf8) == 0xf0) len = 4, cp = c & 0x07;
        else return false;
        if (n - i < len) return false;
        for (uint32_t k = 1; k < len; ++k) {
            if ((p[i + k] & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (p[i + k] & 0x3f);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
            cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff))
            return false;
        i += len;
    }
    return true;
}

constexpr int kMaxArrayDepth = 64;

// Little-endian cursor; every read reports "Unexpected end" as the
// reference's readInteger / readBytes do (GGUFParser.swift:187-204).
struct Reader {
    const uint8_t *p;
    uint64_t n, off = 0;

    er_status need(uint64_t k) const {
        if (k > n - off)
            return fail(ER_ERR_INVALID_FORMAT, "Unexpected end of GGUF data at offset %llu",
                        (unsigned long long)off);
        return ER_OK;
    }
    template <typename T>
    er_status get(T &v) {
        er_status st = need(sizeof(T));
        if (st != ER_OK) return st;
        std::memcpy(&v, p + off, sizeof(T));  // x86-64 and the GGUF format are little-endian
        off += sizeof(T);
        return ER_OK;
    }
    er_status string(std::string &s) {
        uint64_t len = 0;
        er_status st = get(len);
        if (st != ER_OK) return st;
        if (len > ER_GGUF_MAX_STRING)
            return fail(ER_ERR_INVALID_FORMAT, "Unreasonable string length %llu at offset %llu",
                        (unsigned long long)len, (unsigned long long)off);
        st = need(len);
        if (st != ER_OK) return st;
        if (!valid_utf8(p + off, len))
            return fail(ER_ERR_INVALID_FORMAT, "Invalid UTF-8 string at offset %llu", (unsigned long long)off);
        s.assign((const char *)(p + off), (size_t)len);
        off += len;
        return ER_OK;
    }
    er_status value(uint32_t type, Value &v, int depth) {
        v.type = type;
        switch (type) {
            case ER_GGUF_UINT8: { uint8_t x = 0; er_status s = get(x); v.u = x; return s; }
            case ER_GGUF_INT8: { int8_t x = 0; er_status s = get(x); v.i = x; return s; }
            case ER_GGUF_UINT16: { uint16_t x = 0; er_status s = get(x); v.u = x; return s; }
            case ER_GGUF_INT16: { int16_t x = 0; er_status s = get(x); v.i = x; return s; }
            case ER_GGUF_UINT32: { uint32_t x = 0; er_status s = get(x); v.u = x; return s; }
            case ER_GGUF_INT32: { int32_t x = 0; er_status s = get(x); v.i = x; return s; }
            case ER_GGUF_FLOAT32: { float x = 0; er_status s = get(x); v.f = x; return s; }
            case ER_GGUF_BOOL: { uint8_t x = 0; er_status s = get(x); v.u = x != 0; return s; }
            case ER_GGUF_STRING: return string(v.str);
            case ER_GGUF_UINT64: return get(v.u);
            case ER_GGUF_INT64: return get(v.i);
            case ER_GGUF_FLOAT64: return get(v.f);
            case ER_GGUF_ARRAY: {
                uint32_t et = 0;
                er_status st = get(et);
                if (st != ER_OK) return st;
                if (et > ER_GGUF_FLOAT64)
                    return fail(ER_ERR_INVALID_FORMAT, "Unknown GGUF array element type: %u", et);
                if (depth >= kMaxArrayDepth)
                    return fail(ER_ERR_INVALID_FORMAT, "GGUF arrays nested deeper than %d", kMaxArrayDepth);
                uint64_t count = 0;
                st = get(count);
                if (st != ER_OK) return st;
                v.elemType = et;
                // every element takes at least one byte: a count beyond the
                // remaining bytes fails below without a huge reservation
                v.items.reserve((size_t)std::min<uint64_t>(count, n - off));
                for (uint64_t k = 0; k < count; ++k) {
                    v.items.emplace_back();
                    st = value(et, v.items.back(), depth + 1);
                    if (st != ER_OK) return st;
                }
                return ER_OK;
            }
            default:
                return fail(ER_ERR_INVALID_FORMAT, "Unknown GGUF metadata type: %u", type);
        }
    }
};

void fill_value(const Value &v, er_gguf_value *out) {
    *out = er_gguf_value{};
    out->type = v.type;
    out->u = v.u;
    out->i = v.i;
    out->f = v.f;
    if (v.type == ER_GGUF_STRING) {
        out->str = v.str.c_str();
        out->count = v.str.size();
    } else if (v.type == ER_GGUF_ARRAY) {
        out->elem_type = v.elemType;
        out->count = v.items.size();
        out->node = &v;
    }
}

uint64_t align_up(uint64_t x, uint64_t a) { return a <= 1 ? x : (x + a - 1) / a * a; }

}  // namespace

struct er_gguf {
    // backing bytes: a read-only file mapping, or a private copy (parse_memory)
    const uint8_t *base = nullptr;
    uint64_t size = 0;
    void *map = nullptr;
    std::vector<uint8_t> copy;

    uint32_t version = 0;
    uint64_t tensorCountHdr = 0, kvCountHdr = 0;
    std::vector<std::string> keys;
    std::vector<Value> values;
    std::unordered_map<std::string, size_t> keyIndex;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensorIndex;
    uint64_t tableEnd = 0, dataOffset = 0, alignment = ER_GGUF_DEFAULT_ALIGNMENT;

    ~er_gguf() {
        if (map) munmap(map, (size_t)size);
    }
};

namespace {

// readHeader, then readMetadata, then readTensorInfos (GGUFParser.swift:11-75);
// `parts` (1..3) says how many of the three to read.
er_status parse(er_gguf *g, uint32_t parts = 3) {
    Reader r{g->base, g->size};
    uint32_t magic = 0;
    er_status st = r.get(magic);
    if (st != ER_OK) return st;
    if (magic != ER_GGUF_MAGIC) return fail(ER_ERR_INVALID_FORMAT, "Invalid GGUF magic: 0x%x", magic);
    st = r.get(g->version);
    if (st != ER_OK) return st;
    if (g->version < 2 || g->version > 3)
        return fail(ER_ERR_UNSUPPORTED_VERSION, "unsupportedVersion(%u)", g->version);
    if ((st = r.get(g->tensorCountHdr)) != ER_OK || (st = r.get(g->kvCountHdr)) != ER_OK) return st;
    g->tableEnd = r.off;
    if (parts < 2) return ER_OK;

    for (uint64_t k = 0; k < g->kvCountHdr; ++k) {
        std::string key;
        uint32_t type = 0;
        if ((st = r.string(key)) != ER_OK || (st = r.get(type)) != ER_OK) return st;
        if (type > ER_GGUF_FLOAT64) return fail(ER_ERR_INVALID_FORMAT, "Unknown GGUF metadata type: %u", type);
        Value v;
        if ((st = r.value(type, v, 0)) != ER_OK) return st;
        auto it = g->keyIndex.find(key);
        if (it != g->keyIndex.end()) {
            g->values[it->second] = std::move(v);
        } else {
            g->keyIndex.emplace(key, g->keys.size());
            g->keys.push_back(std::move(key));
            g->values.push_back(std::move(v));
        }
    }

    g->tableEnd = r.off;
    if (parts < 3) return ER_OK;
    for (uint64_t k = 0; k < g->tensorCountHdr; ++k) {
        Tensor t;
        uint32_t ndim = 0;
        if ((st = r.string(t.name)) != ER_OK || (st = r.get(ndim)) != ER_OK) return st;
        if (ndim > ER_GGUF_MAX_DIMS)
            return fail(ER_ERR_INVALID_FORMAT, "Unreasonable dimension count %u for tensor '%s'", ndim,
                        t.name.c_str());
        t.dims.resize(ndim);
        for (uint32_t d = 0; d < ndim; ++d)
            if ((st = r.get(t.dims[d])) != ER_OK) return st;
        if ((st = r.get(t.type)) != ER_OK) return st;
        if (!type_row(t.type).known) return fail(ER_ERR_UNSUPPORTED_DATA_TYPE, "unsupportedDataType(%u)", t.type);
        if ((st = r.get(t.offset)) != ER_OK) return st;
        g->tensorIndex.emplace(t.name, g->tensors.size());  // first of duplicate names wins lookups
        g->tensors.push_back(std::move(t));
    }
    g->tableEnd = r.off;

    // data section: next multiple of general.alignment (uint32 power of two)
    // when the file sets it, else of 32 as the reference
    auto al = g->keyIndex.find("general.alignment");
    if (al != g->keyIndex.end()) {
        const Value &v = g->values[al->second];
        if (v.type != ER_GGUF_UINT32 || v.u == 0 || (v.u & (v.u - 1)) != 0)
            return fail(ER_ERR_INVALID_FORMAT, "general.alignment must be a uint32 power of two");
        g->alignment = v.u;
    }
    g->dataOffset = align_up(g->tableEnd, g->alignment);
    return ER_OK;
}

// elementCount (GGUFTypes.swift:141-148) and tensorByteCount
// (GGUFLoader.swift:125-179).  Returns 0, or 1 on overflow, 2 for a type
// the reference refuses to size.
int byte_count_raw(const Tensor &t, uint64_t &elems, uint64_t &bytes) {
    elems = 1;
    bytes = 0;
    for (uint64_t d : t.dims)
        if (__builtin_mul_overflow(elems, d, &elems)) return 1;
    const TypeRow row = type_row(t.type);
    if (row.blockBytes == 0) return 2;
    const uint64_t blocks = elems / row.blockElems + (elems % row.blockElems != 0);
    if (__builtin_mul_overflow(blocks, (uint64_t)row.blockBytes, &bytes)) return 1;
    return 0;
}

er_status byte_count(const Tensor &t, uint64_t &elems, uint64_t &bytes) {
    switch (byte_count_raw(t, elems, bytes)) {
        case 0: return ER_OK;
        case 2: return fail(ER_ERR_UNSUPPORTED_DATA_TYPE, "unsupportedDataType(%u)", t.type);
        default: return fail(ER_ERR_INVALID_FORMAT, "size of tensor '%s' overflows", t.name.c_str());
    }
}

er_status check_g(const er_gguf *g) {
    return g ? ER_OK : fail(ER_ERR_INVALID_ARGUMENT, "null er_gguf");
}

}  // namespace

extern "C" {

er_status er_gguf_parse_memory(const void *data, uint64_t size, uint32_t parts, er_gguf **out) {
    if (!out) return fail(ER_ERR_INVALID_ARGUMENT, "null out");
    *out = nullptr;
    if (!data && size) return fail(ER_ERR_INVALID_ARGUMENT, "null data");
    std::unique_ptr<er_gguf> g(new (std::nothrow) er_gguf);
    if (!g) return fail(ER_ERR_ALLOCATION_FAILED, "allocationFailed");
    try {
        g->copy.assign((const uint8_t *)data, (const uint8_t *)data + size);
    } catch (...) {
        return fail(ER_ERR_ALLOCATION_FAILED, "allocationFailed(byteCount: %llu)", (unsigned long long)size);
    }
    g->base = g->copy.data();
    g->size = size;
    if (parts < 1 || parts > 3) return fail(ER_ERR_INVALID_ARGUMENT, "parts must be 1, 2 or 3");
    er_status st;
    try {
        st = parse(g.get(), parts);
    } catch (...) {
        return fail(ER_ERR_ALLOCATION_FAILED, "allocationFailed while parsing");
    }
    if (st != ER_OK) return st;
    *out = g.release();
    return ER_OK;
}

er_status er_gguf_open(const char *path, er_gguf **out) {
    if (!out || !path) return fail(ER_ERR_INVALID_ARGUMENT, "null path or out");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        if (errno == ENOENT) return fail(ER_ERR_FILE_NOT_FOUND, "fileNotFound(%s)", path);
        return fail(ER_ERR_MMAP_FAILED, "mmapFailed(errno: %d) opening %s", errno, path);
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        const int e = errno;
        ::close(fd);
        return fail(ER_ERR_MMAP_FAILED, "mmapFailed(errno: %d)", e);
    }
    std::unique_ptr<er_gguf> g(new (std::nothrow) er_gguf);
    if (!g) {
        ::close(fd);
        return fail(ER_ERR_ALLOCATION_FAILED, "allocationFailed");
    }
    g->size = (uint64_t)sb.st_size;
    if (g->size > 0) {
        void *m = mmap(nullptr, (size_t)g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            const int e = errno;
            ::close(fd);
            return fail(ER_ERR_MMAP_FAILED, "mmapFailed(errno: %d)", e);
        }
        g->map = m;
        g->base = (const uint8_t *)m;
    }
    ::close(fd);  // the mapping stays valid
    er_status st;
    try {
        st = parse(g.get());
    } catch (...) {
        return fail(ER_ERR_ALLOCATION_FAILED, "allocationFailed while parsing");
    }
    if (st != ER_OK) return st;
    // ModelConfig.from(ggufMetadata:) (GGUFMetadata.swift:119-136)
    auto arch = g->keyIndex.find("general.architecture");
    if (arch == g->keyIndex.end() || g->values[arch->second].type != ER_GGUF_STRING)
        return fail(ER_ERR_MISSING_METADATA, "missingMetadata(general.architecture)");
    for (size_t k = 0; k < g->keys.size(); ++k)
        if (g->values[k].type == ER_GGUF_UINT64 && g->values[k].u > (uint64_t)INT64_MAX)
            return fail(ER_ERR_INVALID_FORMAT, "GGUF metadata value for %s cannot be represented in ModelConfig",
                        g->keys[k].c_str());
    // load(from:) per tensor, in table order (GGUFLoader.swift:40-57)
    for (const Tensor &t : g->tensors) {
        uint64_t elems = 0, bytes = 0;
        if ((st = byte_count(t, elems, bytes)) != ER_OK) return st;
        uint64_t end = 0;
        if (__builtin_add_overflow(g->dataOffset, t.offset, &end) || __builtin_add_overflow(end, bytes, &end) ||
            end > g->size)
            return fail(ER_ERR_INVALID_FORMAT, "Tensor %s exceeds GGUF data section bounds", t.name.c_str());
    }
    *out = g.release();
    return ER_OK;
}

void er_gguf_close(er_gguf *g) { delete g; }

er_status er_gguf_header(const er_gguf *g, uint32_t *version, uint64_t *tensor_count,
                         uint64_t *metadata_kv_count) {
    er_status st = check_g(g);
    if (st != ER_OK) return st;
    if (version) *version = g->version;
    if (tensor_count) *tensor_count = g->tensorCountHdr;
    if (metadata_kv_count) *metadata_kv_count = g->kvCountHdr;
    return ER_OK;
}

uint64_t er_gguf_metadata_count(const er_gguf *g) { return g ? g->keys.size() : 0; }

er_status er_gguf_metadata_key(const er_gguf *g, uint64_t index, const char **key) {
    er_status st = check_g(g);
    if (st != ER_OK) return st;
    if (!key || index >= g->keys.size()) return fail(ER_ERR_INVALID_ARGUMENT, "metadata index %llu out of range",
                                                     (unsigned long long)index);
    *key = g->keys[index].c_str();
    return ER_OK;
}

er_status er_gguf_metadata_value(const er_gguf *g, uint64_t index, er_gguf_value *out) {
    er_status st = check_g(g);
    if (st != ER_OK) return st;
    if (!out || index >= g->values.size())
        return fail(ER_ERR_INVALID_ARGUMENT, "metadata index %llu out of range", (unsigned long long)index);
    fill_value(g->values[index], out);
    return ER_OK;
}

er_status er_gguf_find_metadata(const er_gguf *g, const char *key, uint64_t *index) {
    er_status st = check_g(g);
    if (st != ER_OK) return st;
    if (!key || !index) return fail(ER_ERR_INVALID_ARGUMENT, "null key or index");
    auto it = g->keyIndex.find(key);
    if (it == g->keyIndex.end()) return fail(ER_ERR_MISSING_METADATA, "missingMetadata(%s)", key);
    *index = it->second;
    return ER_OK;
}

er_status er_gguf_array_get(const er_gguf *g, const void *node, uint64_t j, er_gguf_value *out) {
    er_status st = check_g(g);
    if (st != ER_OK) return st;
    const Value *v = (const Value *)node;
    if (!v || !out || v->type != ER_GGUF_ARRAY || j >= v->items.size())
        return fail(ER_ERR_INVALID_ARGUMENT, "array element %llu out of range", (unsigned long long)j);
    fill_value(v->items[j], out);
    return ER_OK;
}

uint64_t er_gguf_tensor_count(const er_gguf *g) { return g ? g->tensors.size() : 0; }

er_status er_gguf_tensor_info_at(const er_gguf *g, uint64_t index, er_gguf_tensor_info *out) {
    er_status st = check_g(g);
    if (st != ER_OK) return st;
    if (!out || index >= g->tensors.size())
        return fail(ER_ERR_INVALID_ARGUMENT, "tensor index %llu out of range", (unsigned long long)index);
    const Tensor &t = g->tensors[index];
    *out = er_gguf_tensor_info{};
    out->name = t.name.c_str();
    out->ndim = (uint32_t)t.dims.size();
    out->ggml_type = t.type;
    for (size_t d = 0; d < t.dims.size(); ++d) out->dims[d] = t.dims[d];
    out->offset = t.offset;
    out->data_type = type_row(t.type).dataType;
    uint64_t elems = 0, bytes = 0;
    (void)byte_count_raw(t, elems, bytes);  // unsized or overflowing: byte_count 0
    out->element_count = elems;
    out->byte_count = bytes;
    return ER_OK;
}

er_status er_gguf_find_tensor(const er_gguf *g, const char *name, uint64_t *index) {
    er_status st = check_g(g);
    if (st != ER_OK) return st;
    if (!name || !index) return fail(ER_ERR_INVALID_ARGUMENT, "null name or index");
    auto it = g->tensorIndex.find(name);
    if (it == g->tensorIndex.end()) return fail(ER_ERR_TENSOR_NOT_FOUND, "tensorNotFound(%s)", name);
    *index = it->second;
    return ER_OK;
}

er_status er_gguf_data_section(const er_gguf *g, uint64_t *file_offset, uint64_t *bytes) {
    er_status st = check_g(g);
    if (st != ER_OK) return st;
    const uint64_t off = std::min(g->dataOffset, g->size);
    if (file_offset) *file_offset = g->dataOffset;
    if (bytes) *bytes = g->size - off;
    return ER_OK;
}

er_status er_gguf_tensor_host_data(const er_gguf *g, uint64_t index, const void **data, uint64_t *bytes) {
    er_gguf_tensor_info info;
    er_status st = er_gguf_tensor_info_at(g, index, &info);
    if (st != ER_OK) return st;
    if (info.data_type == ER_DATA_TYPE_NONE || (info.byte_count == 0 && info.element_count != 0))
        return fail(ER_ERR_UNSUPPORTED_DATA_TYPE, "unsupportedDataType(%u)", info.ggml_type);
    uint64_t end = 0;
    if (__builtin_add_overflow(g->dataOffset, info.offset, &end) ||
        __builtin_add_overflow(end, info.byte_count, &end) || end > g->size)
        return fail(ER_ERR_INVALID_FORMAT, "Tensor %s exceeds GGUF data section bounds", info.name);
    if (data) *data = g->base + g->dataOffset + info.offset;
    if (bytes) *bytes = info.byte_count;
    return ER_OK;
}

er_status er_gguf_tensor_storage(const er_gguf *g, uint64_t index, er_buffer data, er_tensor_storage *out) {
    er_gguf_tensor_info info;
    er_status st = er_gguf_tensor_info_at(g, index, &info);
    if (st != ER_OK) return st;
    if (!out) return fail(ER_ERR_INVALID_ARGUMENT, "null out");
    if (info.data_type == ER_DATA_TYPE_NONE)
        return fail(ER_ERR_UNSUPPORTED_DATA_TYPE, "unsupportedDataType(%u)", info.ggml_type);
    if (info.ndim > 4)
        return fail(ER_ERR_INVALID_ARGUMENT, "tensor %s has %u dimensions; er_tensor_storage holds 4", info.name,
                    info.ndim);
    uint64_t end = 0;
    if (__builtin_add_overflow(info.offset, info.byte_count, &end) || end > data.length)
        return fail(ER_ERR_INVALID_ARGUMENT, "tensor %s (offset %llu, %llu bytes) lies outside the %llu-byte data buffer",
                    info.name, (unsigned long long)info.offset, (unsigned long long)info.byte_count,
                    (unsigned long long)data.length);
    *out = er_tensor_storage{};
    out->buffer = data;
    out->byte_offset = info.offset;
    out->data_type = info.data_type;
    out->ndim = info.ndim;
    for (uint32_t d = 0; d < info.ndim; ++d) out->shape[d] = info.dims[d];
    return ER_OK;
}

er_status er_hip_gguf_upload(er_hip_ctx *ctx, er_stream stream, const er_gguf *g, er_buffer *out) {
    er_status st = check_g(g);
    if (st != ER_OK) return st;
    if (!ctx || !out) return fail(ER_ERR_INVALID_ARGUMENT, "null context or out");
    *out = er_buffer{nullptr, 0};
    uint64_t off = 0, bytes = 0;
    er_gguf_data_section(g, &off, &bytes);
    const uint64_t alloc = std::max<uint64_t>(bytes, 256u);
    st = er_hip_alloc(ctx, alloc, out);
    if (st != ER_OK) return st;
    out->length = bytes;
    if (bytes == 0) return ER_OK;

    const hipStream_t s = (hipStream_t)stream;
    constexpr uint64_t kChunk = 64ull << 20;
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool recorded[2] = {false, false};
    hipError_t e = hipSuccess;
    for (int k = 0; k < 2 && e == hipSuccess; ++k) {
        e = hipHostMalloc(&stage[k], (size_t)std::min(kChunk, bytes), hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&done[k], hipEventDisableTiming);
    }
    const uint8_t *src = g->base + off;
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned nthreads = std::min(8u, hw);
    for (uint64_t pos = 0, c = 0; e == hipSuccess && pos < bytes; pos += kChunk, ++c) {
        const int k = (int)(c & 1);
        const uint64_t n = std::min(kChunk, bytes - pos);
        if (recorded[k]) {
            e = hipEventSynchronize(done[k]);  // the DMA that last read this stage has finished
            if (e != hipSuccess) break;
        }
        // page copy split over host threads
        const uint64_t per = (n + nthreads - 1) / nthreads;
        std::vector<std::thread> pool;
        for (unsigned t = 1; t < nthreads && t * per < n; ++t)
            pool.emplace_back([&, t] {
                const uint64_t a = t * per, b = std::min(n, a + per);
                std::memcpy((uint8_t *)stage[k] + a, src + pos + a, (size_t)(b - a));
            });
        std::memcpy(stage[k], src + pos, (size_t)std::min(per, n));
        for (auto &th : pool) th.join();
        e = hipMemcpyAsync((uint8_t *)out->data + pos, stage[k], (size_t)n, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipEventRecord(done[k], s);
        recorded[k] = e == hipSuccess;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    for (int k = 0; k < 2; ++k) {
        if (done[k]) (void)hipEventDestroy(done[k]);
        if (stage[k]) (void)hipHostFree(stage[k]);
    }
    if (e != hipSuccess) {
        (void)er_hip_free(ctx, *out);
        *out = er_buffer{nullptr, 0};
        return fail(ER_ERR_DEVICE, "GGUF upload: %s", hipGetErrorString(e));
    }
    return ER_OK;
}

}  // extern "C"
