/*
 * er_gguf.h -- GGUF weight loading for EdgeRunnerHIP: parse a GGUF file
 * (header, typed metadata, tensor table) from a read-only memory map and
 * upload its data section into HBM, giving each tensor an er_tensor_storage
 * view that er_hip_encode_projection and the encode entry points consume.
 *
 * Replaces, for a Linux / MI355X host:
 *   - GGUFReader (Sources/EdgeRunnerIO/GGUF/GGUFParser.swift:3-205): the
 *     byte-level parser, its limits and its errors;
 *   - GGUFLoader.prepare / load / tensorByteCount
 *     (Sources/EdgeRunnerIO/GGUF/GGUFLoader.swift:35-179): data-section
 *     offset, per-tensor byte counts, bounds and data-type checks;
 *   - MemoryMappedFile / FileRegionMapper + MTLBuffer(bytesNoCopy:)
 *     (Sources/EdgeRunnerIO/MemoryMappedFile.swift:142-196): MI355X has no
 *     unified memory, so the mapped data section is copied into one HBM
 *     allocation instead, and tensors are byte-offset views into it.
 *
 * Errors are WeightLoaderError's cases (er_status 10..16, er_hip.h).  One
 * deliberate difference: the data section starts at the next multiple of
 * `general.alignment` when the file sets it (a uint32 power of two), where
 * the reference always uses 32 (GGUFLoader.swift:82); files without the key
 * behave identically.
 *
 * An er_gguf is immutable after open; it may be read from several threads.
 */
#ifndef ER_GGUF_H
#define ER_GGUF_H

#include "er_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUFMetadataValueType (GGUFTypes.swift:6-20). */
typedef enum er_gguf_value_type {
    ER_GGUF_UINT8 = 0,
    ER_GGUF_INT8 = 1,
    ER_GGUF_UINT16 = 2,
    ER_GGUF_INT16 = 3,
    ER_GGUF_UINT32 = 4,
    ER_GGUF_INT32 = 5,
    ER_GGUF_FLOAT32 = 6,
    ER_GGUF_BOOL = 7,
    ER_GGUF_STRING = 8,
    ER_GGUF_ARRAY = 9,
    ER_GGUF_UINT64 = 10,
    ER_GGUF_INT64 = 11,
    ER_GGUF_FLOAT64 = 12
} er_gguf_value_type;

#define ER_GGUF_MAGIC 0x46554747u      /* "GGUF" little-endian (GGUFTypes.swift:3) */
#define ER_GGUF_MAX_DIMS 8             /* GGUFParser.swift:55 */
#define ER_GGUF_MAX_STRING 1000000u    /* GGUFParser.swift:134 */
#define ER_GGUF_DEFAULT_ALIGNMENT 32u  /* GGUFLoader.swift:82 */
#define ER_DATA_TYPE_NONE 0xffffffffu  /* GGUF type with no TensorDataType */

typedef struct er_gguf er_gguf;

/* One metadata value (GGUFMetadataValue, GGUFMetadata.swift:3-17).  Scalars
 * fill u (unsigned and bool), i (signed) or f (float32 widened exactly, or
 * float64); strings fill str (NUL-terminated copy) and count (byte length);
 * arrays fill elem_type, count and node, a handle for er_gguf_array_get. */
typedef struct er_gguf_value {
    uint32_t type;      /* er_gguf_value_type */
    uint32_t elem_type; /* arrays only */
    uint64_t count;
    uint64_t u;
    int64_t i;
    double f;
    const char *str;
    const void *node;
} er_gguf_value;

/* GGUFTensorInfo (GGUFTypes.swift:135-149) plus what GGUFLoader.load derives. */
typedef struct er_gguf_tensor_info {
    const char *name;              /* NUL-terminated, owned by the er_gguf */
    uint32_t ndim;
    uint32_t ggml_type;            /* GGUFTensorType raw value */
    uint64_t dims[ER_GGUF_MAX_DIMS];
    uint64_t offset;               /* relative to the data section */
    uint64_t element_count;
    uint64_t byte_count;           /* GGUFLoader.tensorByteCount */
    uint32_t data_type;            /* TensorDataType raw value, or ER_DATA_TYPE_NONE */
    uint32_t reserved;
} er_gguf_tensor_info;

/* GGUFReader over bytes in memory (the parser tests' form): reads the header
 * (parts = 1), then the metadata (2), then the tensor table (3), with the
 * reader's checks and errors but none of the loader's tensor checks
 * (GGUFParser.swift:3-75).  The bytes are copied.  The data section offset
 * is set only when parts = 3. */
er_status er_gguf_parse_memory(const void *data, uint64_t size, uint32_t parts, er_gguf **out);

/* GGUFLoader(url:) + load(from:) validation: maps the file read-only, parses
 * it, requires general.architecture (missingMetadata), computes the data
 * section offset, and checks every tensor in table order as load(from:)
 * does: byte count (unsupportedDataType for types it cannot size), bounds
 * within the file (invalidFormat), a TensorDataType (unsupportedDataType). */
er_status er_gguf_open(const char *path, er_gguf **out);
void er_gguf_close(er_gguf *g);

/* GGUFHeader (GGUFTypes.swift:124-133). */
er_status er_gguf_header(const er_gguf *g, uint32_t *version, uint64_t *tensor_count,
                         uint64_t *metadata_kv_count);

/* Metadata: distinct keys in first-appearance order; a repeated key keeps
 * its first position and its last value (Swift dictionary assignment). */
uint64_t er_gguf_metadata_count(const er_gguf *g);
er_status er_gguf_metadata_key(const er_gguf *g, uint64_t index, const char **key);
er_status er_gguf_metadata_value(const er_gguf *g, uint64_t index, er_gguf_value *out);
/* Index of `key`, or ER_ERR_MISSING_METADATA. */
er_status er_gguf_find_metadata(const er_gguf *g, const char *key, uint64_t *index);
/* Element j of an array value (node from er_gguf_value.node). */
er_status er_gguf_array_get(const er_gguf *g, const void *node, uint64_t j, er_gguf_value *out);

uint64_t er_gguf_tensor_count(const er_gguf *g);
er_status er_gguf_tensor_info_at(const er_gguf *g, uint64_t index, er_gguf_tensor_info *out);
/* Index of the tensor named `name`, or ER_ERR_TENSOR_NOT_FOUND. */
er_status er_gguf_find_tensor(const er_gguf *g, const char *name, uint64_t *index);

/* Data section: file offset (aligned) and byte length up to the end of the
 * file; and a host pointer to a tensor's bytes inside the mapping. */
er_status er_gguf_data_section(const er_gguf *g, uint64_t *file_offset, uint64_t *bytes);
er_status er_gguf_tensor_host_data(const er_gguf *g, uint64_t index, const void **data,
                                   uint64_t *bytes);

/* Copies the whole data section into one new HBM allocation (*out, freed
 * with er_hip_free), streaming it through two pinned staging buffers so
 * the file-page copies overlap the DMA; synchronous on `stream`. */
er_status er_hip_gguf_upload(er_hip_ctx *ctx, er_stream stream, const er_gguf *g, er_buffer *out);

/* TensorStorage for tensor `index` as a view into the uploaded data section
 * (GGUFLoader.load building TensorStorage, GGUFLoader.swift:40-56):
 * buffer = data, byte_offset = the tensor's offset, data_type, shape.
 * Tensors of more than 4 dimensions return ER_ERR_INVALID_ARGUMENT. */
er_status er_gguf_tensor_storage(const er_gguf *g, uint64_t index, er_buffer data,
                                 er_tensor_storage *out);

#ifdef __cplusplus
}
#endif

#endif /* ER_GGUF_H */
