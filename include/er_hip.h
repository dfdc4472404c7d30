/*
 * er_hip.h -- C ABI of EdgeRunnerHIP: the MI355X (gfx950) quantized-matmul
 * backend for EdgeRunner's GGUF Q8_0 / Q4_K / Q6_K weights.
 *
 * The entry points replace the Metal kernel path behind
 * EdgeRunnerMetal.GEMVKernel (Sources/EdgeRunnerMetal/GEMVKernel.swift),
 * the Q8_0 pipelines fetched by name from KernelRegistry
 * (Sources/EdgeRunnerMetal/KernelRegistry.swift:38-49, used at
 * Sources/EdgeRunner/Models/LlamaLanguageModel.swift:260-275, 2519-2535) and
 * the Dequant*Kernel.dequantise wrappers (Sources/EdgeRunnerIO/Dequant*.swift).
 * Paths are relative to the EdgeRunner source tree.
 *
 * Conventions (mirroring the Metal protocol):
 *   - Weights are the raw GGUF blocks, row-major, each row made of K/32 (Q8_0)
 *     or K/256 (Q4_K, Q6_K) contiguous blocks; GGUF shape [K, M].
 *   - "encode" calls only enqueue work on the caller's stream (the
 *     MTLCommandBuffer analogue) and never allocate; ordering is the stream's.
 *   - A buffer is device memory plus its byte length (the MTLBuffer analogue),
 *     so the reference's buffer-length validation is reproduced exactly.
 *   - Every call returns an er_status; er_hip_last_error() gives the message of
 *     the calling thread's last failure.
 *   - A context is immutable after er_hip_create; calls on distinct streams may
 *     run concurrently from several threads.
 */
#ifndef ER_HIP_H
#define ER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ER_HIP_ABI_VERSION 1

/* Status codes.  Each maps 1:1 onto a Swift error case of the reference:
 * GEMVError (GEMVKernel.swift:1435-1441), DequantKernelError
 * (Sources/EdgeRunnerIO/DequantKernel.swift:19-25) and, for the GGUF loader,
 * WeightLoaderError. */
typedef enum er_status {
    ER_OK = 0,
    ER_ERR_LIBRARY_NOT_FOUND = 1,        /* GEMVError.libraryNotFound: code object missing/unloadable */
    ER_ERR_FUNCTION_NOT_FOUND = 2,       /* GEMVError.functionNotFound(name) */
    ER_ERR_ENCODING_FAILED = 3,          /* GEMVError.encodingFailed / DequantKernelError.encodingFailed */
    ER_ERR_INVALID_MATRIX_SHAPE = 4,     /* GEMVError.invalidMatrixShape */
    ER_ERR_INVALID_VECTOR_SHAPE = 5,     /* GEMVError.invalidVectorShape */
    ER_ERR_INVALID_BLOCK_DATA_COUNT = 6, /* DequantKernelError.invalidBlockDataCount(expected:actual:) */
    ER_ERR_ALLOCATION_FAILED = 7,        /* DequantKernelError.allocationFailed(byteCount:) */
    ER_ERR_INVALID_ARGUMENT = 8,         /* null context/pointer, misaligned device pointer */
    ER_ERR_DEVICE = 9,                   /* HIP runtime error (commandBuffer.error analogue) */
    /* WeightLoaderError (Sources/EdgeRunnerIO/WeightLoaderError.swift:3-15), GGUF loader (er_gguf.h) */
    ER_ERR_FILE_NOT_FOUND = 10,          /* fileNotFound(URL) */
    ER_ERR_INVALID_FORMAT = 11,          /* invalidFormat(String) */
    ER_ERR_UNSUPPORTED_VERSION = 12,     /* unsupportedVersion(UInt32) */
    ER_ERR_UNSUPPORTED_DATA_TYPE = 13,   /* unsupportedDataType(UInt32) */
    ER_ERR_MMAP_FAILED = 14,             /* mmapFailed(errno:) */
    ER_ERR_MISSING_METADATA = 15,        /* missingMetadata(String) */
    ER_ERR_TENSOR_NOT_FOUND = 16         /* tensorNotFound(String) */
} er_status;

/* TensorDataType raw values (Sources/EdgeRunnerIO/WeightMap.swift:69-91). */
typedef enum er_tensor_type {
    ER_TYPE_F32 = 0,
    ER_TYPE_F16 = 1,
    ER_TYPE_Q8_0 = 8,
    ER_TYPE_Q4_K = 12,
    ER_TYPE_Q6_K = 14,
    ER_TYPE_BF16 = 30
} er_tensor_type;

/* Block geometry (GGUFLoader.tensorByteCount, Sources/EdgeRunnerIO/GGUF/GGUFLoader.swift:125-179). */
#define ER_Q8_0_BLOCK_BYTES 34
#define ER_Q8_0_BLOCK_WEIGHTS 32
#define ER_Q4_K_BLOCK_BYTES 144
#define ER_Q6_K_BLOCK_BYTES 210
#define ER_K_BLOCK_WEIGHTS 256

/* Device memory plus its byte length: the MTLBuffer analogue.  The weight
 * buffer's data pointer must be 16-byte aligned (GGUF tensor data is 32-byte
 * aligned); activations and outputs must be 4-byte aligned. */
typedef struct er_buffer {
    void *data;
    uint64_t length;
} er_buffer;

/* TensorStorage (WeightMap.swift:93-127): buffer + byteOffset + dataType +
 * GGUF shape [K, M] (shape[0] = K = columns, shape[1] = M = rows). */
typedef struct er_tensor_storage {
    er_buffer buffer;
    uint64_t byte_offset;
    uint32_t data_type; /* er_tensor_type */
    uint32_t ndim;
    uint64_t shape[4];
} er_tensor_storage;

typedef struct er_hip_ctx er_hip_ctx;
typedef void *er_stream; /* hipStream_t; NULL = the device's null stream */
typedef void *er_event;  /* hipEvent_t */
typedef void *er_graph;  /* instantiated hipGraphExec_t */

typedef struct er_device_info {
    int device;
    int compute_units;
    int clock_khz;
    int memory_clock_khz;
    int memory_bus_width;
    uint64_t total_memory;
    uint64_t lds_per_workgroup; /* bytes of LDS one workgroup may allocate */
    char name[64];
    char arch[64];
} er_device_info;

/* ---- lifecycle (GEMVKernel.init: pipelines resolved once, GEMVKernel.swift:54-76) ---- */

/* Loads the embedded gfx950 code object on `device` (hipModuleLoadData) and
 * resolves every kernel by name (the KernelRegistry analogue). */
er_status er_hip_create(int device, er_hip_ctx **out_ctx);
void er_hip_destroy(er_hip_ctx *ctx);
er_status er_hip_get_device_info(const er_hip_ctx *ctx, er_device_info *out);
const char *er_hip_last_error(void);
const char *er_status_string(er_status status);
int er_hip_abi_version(void);

/* ---- memory: no unified memory on MI355X, so the mmap'd GGUF bytes are
 * uploaded once (replaces MTLBuffer(bytesNoCopy:), MemoryMappedFile.swift:142-196) ---- */
er_status er_hip_alloc(er_hip_ctx *ctx, uint64_t bytes, er_buffer *out);
er_status er_hip_free(er_hip_ctx *ctx, er_buffer buf);
er_status er_hip_upload(er_hip_ctx *ctx, er_stream stream, er_buffer dst, uint64_t dst_offset,
                        const void *src, uint64_t bytes);
er_status er_hip_download(er_hip_ctx *ctx, er_stream stream, void *dst, er_buffer src,
                          uint64_t src_offset, uint64_t bytes);
/* Device-to-device copy enqueued on `stream` (MTLBlitCommandEncoder.copy analogue). */
er_status er_hip_copy(er_hip_ctx *ctx, er_stream stream, er_buffer dst, uint64_t dst_offset,
                      er_buffer src, uint64_t src_offset, uint64_t bytes);

/* ---- streams and events (command buffer commit / completed; GPU timing as in
 * Gemma4LanguageModel.RuntimeProfiler, Gemma4LanguageModel.swift:135-200) ---- */
er_status er_hip_stream_create(er_hip_ctx *ctx, er_stream *out);
er_status er_hip_stream_destroy(er_hip_ctx *ctx, er_stream stream);
er_status er_hip_synchronize(er_hip_ctx *ctx, er_stream stream);
er_status er_hip_event_create(er_hip_ctx *ctx, er_event *out);
er_status er_hip_event_destroy(er_hip_ctx *ctx, er_event ev);
er_status er_hip_event_record(er_hip_ctx *ctx, er_event ev, er_stream stream);
er_status er_hip_event_elapsed_ms(er_hip_ctx *ctx, er_event start, er_event end, float *ms);

/* ---- recorded command sequences: the MTLCommandBuffer / indirect command
 * buffer analogue for replaying a fixed sequence of encodes (e.g. every
 * projection of a decode step, GEMVKernel.encode* calls on one command buffer,
 * Tests/EdgeRunnerMetalTests/GEMVTests.swift:662-734).  Between begin and end,
 * encode calls on `stream` are recorded instead of executed (the stream must
 * not be the null stream); the result is replayed with er_hip_graph_launch on
 * any stream.  Buffers are bound by address at record time. ---- */
er_status er_hip_graph_begin(er_hip_ctx *ctx, er_stream stream);
er_status er_hip_graph_end(er_hip_ctx *ctx, er_stream stream, er_graph *out);
er_status er_hip_graph_launch(er_hip_ctx *ctx, er_graph graph, er_stream stream);
er_status er_hip_graph_destroy(er_hip_ctx *ctx, er_graph graph);

/* ---- dequantisation to fp32 ----
 * Replace DequantQ8_0Kernel.dequantise (Sources/EdgeRunnerIO/DequantQ8_0Kernel.swift:18-78),
 * DequantQ4KMKernel.dequantise (DequantQ4KMKernel.swift:18-78) and
 * DequantQ6KKernel.dequantise (DequantQ6KKernel.swift:18-78).
 * blocks.length must be >= count * block bytes (INVALID_BLOCK_DATA_COUNT) and
 * out.length >= count * weights per block * 4 (ALLOCATION_FAILED).  Results
 * are bit-identical to the reference's CPU dequantisers. */
er_status er_hip_dequant_q8_0(er_hip_ctx *ctx, er_stream stream, er_buffer blocks,
                              uint64_t block_count, er_buffer out);
er_status er_hip_dequant_q4_k(er_hip_ctx *ctx, er_stream stream, er_buffer blocks,
                              uint64_t super_block_count, er_buffer out);
er_status er_hip_dequant_q6_k(er_hip_ctx *ctx, er_stream stream, er_buffer blocks,
                              uint64_t super_block_count, er_buffer out);

/* ---- decode GEMV: y[M] = W[M,K] . x[K], fp32 in / fp32 out ----
 * Validation as GEMVKernel.validateKQuantInputShape + encodeKQuantWeights
 * (GEMVKernel.swift:1415-1432, 1276-1300): K > 0 and K % 256 == 0 else
 * INVALID_VECTOR_SHAPE; weight.length >= M*(K/256)*blockBytes else
 * INVALID_MATRIX_SHAPE; input.length >= K*4 and output.length >= M*4 else
 * ENCODING_FAILED. */

/* GEMVKernel.encodeQ4KWeights (GEMVKernel.swift:704-722; kernel q4_k_gemv_f32). */
er_status er_hip_encode_q4k_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                    er_buffer input, er_buffer output, uint32_t M, uint32_t K);
/* GEMVKernel.encodeQ6KWeights (GEMVKernel.swift:1164-1182; kernel q6_k_gemv_f32). */
er_status er_hip_encode_q6k_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                    er_buffer input, er_buffer output, uint32_t M, uint32_t K);
/* Q8_0 GEMV: pipeline "dequant_q8_0_gemv" with ERDequantGEMVParams{rows, cols,
 * blocksPerRow} (Dequant_Q8_0.metal:86-141, DequantParams.h:11-15).  The
 * reference encodes it by hand without validation; here K > 0 and K % 32 == 0
 * (INVALID_VECTOR_SHAPE) and weight.length >= M*(K/32)*34 (INVALID_MATRIX_SHAPE). */
er_status er_hip_encode_q8_0_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                     er_buffer input, er_buffer output, uint32_t M, uint32_t K);

/* ---- fused Q4_K projections sharing one input vector (one launch, x read
 * and staged once).  Validation per weight as encodeQ4KWeights; inputs and
 * outputs too short -> ENCODING_FAILED.
 * GEMVKernel.encodeQ4KWeightsDual (GEMVKernel.swift:879-928, kernel
 * q4_k_gemv_dual_f32): yA = WA.x, yB = WB.x, both M x K. */
er_status er_hip_encode_q4k_weights_dual(er_hip_ctx *ctx, er_stream stream, er_buffer weight_a,
                                         er_buffer weight_b, er_buffer input, er_buffer output_a,
                                         er_buffer output_b, uint32_t M, uint32_t K);
/* GEMVKernel.encodeQ4KWeightsTriple (GEMVKernel.swift:978-1043, kernel
 * q4_k_gemv_three_f32): three matrices of rows_a / rows_b / rows_c rows. */
er_status er_hip_encode_q4k_weights_triple(er_hip_ctx *ctx, er_stream stream, er_buffer weight_a,
                                           er_buffer weight_b, er_buffer weight_c, er_buffer input,
                                           er_buffer output_a, er_buffer output_b,
                                           er_buffer output_c, uint32_t rows_a, uint32_t rows_b,
                                           uint32_t rows_c, uint32_t K);
/* GEMVKernel.encodeQ4KWeightsDualGeGLU (GEMVKernel.swift:930-976, kernel
 * q4_k_gemv_dual_geglu_f32): y = gelu_tanh(Wgate.x) * (Wup.x), gelu_tanh
 * saturated outside [-10, 10].  Any K % 256 == 0, as the reference: rows
 * beyond 16384 weights run an fp32 pair kernel. */
er_status er_hip_encode_q4k_weights_dual_geglu(er_hip_ctx *ctx, er_stream stream,
                                               er_buffer gate_weight, er_buffer up_weight,
                                               er_buffer input, er_buffer output, uint32_t M,
                                               uint32_t K);

/* ---- GEMVKernel's alternative encoders ----
 * The reference keeps several Metal kernels for one product and lets the
 * model pick one by flag (Gemma4RuntimeOptions, Sources/EdgeRunner/Models/
 * Gemma4/Gemma4RuntimeOptions.swift:13-24; dispatch at
 * Gemma4LanguageModel.swift:4207-4285).  They differ only in their Metal
 * lane mapping: each computes the same y = W.x with the same validation
 * (encodeKQuantWeights, GEMVKernel.swift:1276-1300).  Here each is its
 * canonical entry point under the reference's name: identical arguments,
 * validation, errors and results (bit for bit), and the kernel choice is the
 * library's (by shape) whichever name is called. */
/* encodeQ4KWeightsPacked (GEMVKernel.swift:724) = er_hip_encode_q4k_weights. */
er_status er_hip_encode_q4k_weights_packed(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                           er_buffer input, er_buffer output, uint32_t M, uint32_t K);
/* encodeQ4KWeightsPackedFourRows (GEMVKernel.swift:745) = er_hip_encode_q4k_weights. */
er_status er_hip_encode_q4k_weights_packed_four_rows(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                                     er_buffer input, er_buffer output, uint32_t M, uint32_t K);
/* encodeQ4KWeightsLlamaStyle (GEMVKernel.swift:767) = er_hip_encode_q4k_weights. */
er_status er_hip_encode_q4k_weights_llama_style(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                                er_buffer input, er_buffer output, uint32_t M, uint32_t K);
/* encodeQ4KWeightsTwoRows (GEMVKernel.swift:840) = er_hip_encode_q4k_weights. */
er_status er_hip_encode_q4k_weights_two_rows(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                             er_buffer input, er_buffer output, uint32_t M, uint32_t K);
/* encodeQ4KWeightsLlamaStyleDual (GEMVKernel.swift:789) = er_hip_encode_q4k_weights_dual. */
er_status er_hip_encode_q4k_weights_llama_style_dual(er_hip_ctx *ctx, er_stream stream, er_buffer weight_a,
                                                     er_buffer weight_b, er_buffer input, er_buffer output_a,
                                                     er_buffer output_b, uint32_t M, uint32_t K);
/* encodeQ4KWeightsTriplePacked (GEMVKernel.swift:1045) = er_hip_encode_q4k_weights_triple. */
er_status er_hip_encode_q4k_weights_triple_packed(er_hip_ctx *ctx, er_stream stream, er_buffer weight_a,
                                                  er_buffer weight_b, er_buffer weight_c, er_buffer input,
                                                  er_buffer output_a, er_buffer output_b, er_buffer output_c,
                                                  uint32_t rows_a, uint32_t rows_b, uint32_t rows_c, uint32_t K);
/* encodeQ6KWeightsPacked (GEMVKernel.swift:1184) = er_hip_encode_q6k_weights. */
er_status er_hip_encode_q6k_weights_packed(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                           er_buffer input, er_buffer output, uint32_t M, uint32_t K);

/* ---- synchronous conveniences (GEMVKernel.execute*, GEMVKernel.swift:545-627,
 * 1146-1162, 1363-1413): allocate device x and y (and the weights, for the
 * host-weight forms), encode on the device's null stream, wait, copy y to
 * the caller's host array and free.  Validation as validateKQuantInputShape
 * (GEMVKernel.swift:1415-1432): x_count == K (batched: batch_seq > 0 and
 * x_count == batch_seq * K) and K > 0, K % 256 == 0, else
 * INVALID_VECTOR_SHAPE; weight bytes >= M*(K/256)*blockBytes else
 * INVALID_MATRIX_SHAPE.  y_count (floats the caller's y holds) below M
 * (batched: batch_seq * M) or a failed allocation or copy -> ENCODING_FAILED. */
/* executeQ4KWeights / executeQ6KWeights (GEMVKernel.swift:545, 575): weights from host memory. */
er_status er_hip_execute_q4k_weights(er_hip_ctx *ctx, const void *raw_weights, uint64_t raw_bytes, const float *x,
                                     uint64_t x_count, float *y, uint64_t y_count, uint32_t M, uint32_t K);
er_status er_hip_execute_q6k_weights(er_hip_ctx *ctx, const void *raw_weights, uint64_t raw_bytes, const float *x,
                                     uint64_t x_count, float *y, uint64_t y_count, uint32_t M, uint32_t K);
/* executeQ4KWeightsWithWeightBuffer / executeQ6KWeightsWithWeightBuffer
 * (GEMVKernel.swift:605, 1146): weights already in device memory. */
er_status er_hip_execute_q4k_weights_with_weight_buffer(er_hip_ctx *ctx, er_buffer weight, const float *x,
                                                        uint64_t x_count, float *y, uint64_t y_count, uint32_t M,
                                                        uint32_t K);
er_status er_hip_execute_q6k_weights_with_weight_buffer(er_hip_ctx *ctx, er_buffer weight, const float *x,
                                                        uint64_t x_count, float *y, uint64_t y_count, uint32_t M,
                                                        uint32_t K);
/* executeBatchedQ4KWeights (GEMVKernel.swift:627): y[t*M + r] for t < batch_seq. */
er_status er_hip_execute_batched_q4k_weights(er_hip_ctx *ctx, const void *raw_weights, uint64_t raw_bytes,
                                             const float *x, uint64_t x_count, float *y, uint64_t y_count,
                                             uint32_t batch_seq, uint32_t M, uint32_t K);

/* ---- greedy top-1 over a Q6_K head ----
 * GEMVKernel.encodeQ6KWeightsPackedTop1 (GEMVKernel.swift:1205-1265; kernels
 * q6_k_gemv_packed_4row_top1_f32 + q6_k_top1_reduce, Dequant_Q6_K.metal:196-365).
 * output_index[0] = the row of the largest W.x value, lowest row on ties (the
 * reference's rule, NaN handling included).  M % 4 == 0 else
 * INVALID_MATRIX_SHAPE; K rules as er_hip_encode_q6k_weights; partial_values
 * and partial_indices of >= M/4 fp32 / uint32 entries (q6KTop1PartialCount,
 * GEMVKernel.swift:50-52) and output_index >= 4 bytes, else ENCODING_FAILED.
 * The partial buffers are scratch; their contents afterwards are unspecified.
 * Any K % 256 == 0, as the reference: the row values are those the plain
 * er_hip_encode_q6k_weights computes over the same matrix (fp32 kernels for
 * rows beyond 16384 weights). */
er_status er_hip_encode_q6k_weights_packed_top1(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                                er_buffer input, er_buffer partial_values,
                                                er_buffer partial_indices, er_buffer output_index,
                                                uint32_t M, uint32_t K);

/* ---- allocation-free greedy top-1 ----
 * No counterpart in the reference.  For callers that cannot allocate or pass
 * scratch memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc): er_hip_encode_q6k_weights_packed_top1 without the two partial
 * buffers.  The partials go to a device array inside the library's code
 * object (512 KiB, one per context, held until the context is destroyed),
 * so the call allocates nothing.  Same rules, kernels and result as
 * er_hip_encode_q6k_weights_packed_top1, plus M <= ER_HIP_TOP1_NOALLOC_MAX_ROWS
 * (else INVALID_MATRIX_SHAPE).  Every call through one context shares that
 * array: calls on one context that overlap in time (concurrent streams)
 * race on it and must be ordered by the caller. */
#define ER_HIP_TOP1_NOALLOC_MAX_ROWS 262144u
er_status er_hip_encode_q6k_weights_packed_top1_noalloc(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                                        er_buffer input, er_buffer output_index, uint32_t M,
                                                        uint32_t K);

/* ---- Q8_0 row quantizer ----
 * Kernel quantize_q8_0_rows with ERQuantizeQ8RowsParams{rowCount,
 * sourceRowStride, destinationRowBase, blocksPerRow} (Dequant_Q8_0.metal:9-49),
 * as encoded by LlamaLanguageModel.encodeQ8Rows (LlamaLanguageModel.swift:1820-1850):
 * fp32 source rows (stride in floats) -> Q8_0 blocks of destination rows
 * destination_row_base + r.  Per block: scale = maxAbs/127, d = fp16(scale),
 * q = clamp(rint(v/scale), -127, 127).  source must hold
 * ((row_count-1)*stride + blocks_per_row*32) floats and destination
 * (destination_row_base + row_count)*blocks_per_row*34 bytes, else
 * ENCODING_FAILED; source 4-byte and destination 2-byte aligned. */
er_status er_hip_quantize_q8_0_rows(er_hip_ctx *ctx, er_stream stream, er_buffer source,
                                    er_buffer destination, uint32_t row_count,
                                    uint32_t source_row_stride, uint32_t destination_row_base,
                                    uint32_t blocks_per_row);

/* ---- fused Q8_0 projections (the pipelines LlamaLanguageModel fetches by
 * name, LlamaLanguageModel.swift:260-275; kernels Dequant_Q8_0.metal:199-586).
 * RMSNorm as the reference: n = x * (1/sqrt(sum(x^2)/cols + eps)) * norm_weight,
 * per token.  The reference encodes these without checks; here weights must
 * hold rows*(cols/32)*34 bytes (INVALID_MATRIX_SHAPE), inputs, outputs, norm
 * weight and residual their implied sizes (ENCODING_FAILED), and cols must be
 * a positive multiple of 32 (INVALID_VECTOR_SHAPE); any block count is taken,
 * as the reference's kernels take any blocksPerRow (rows of an odd block
 * count or beyond 16384 weights run fp32 kernels). ---- */

/* dequant_q8_0_fused_qkv (ERFusedQKVParams{qRows, kvRows, cols, blocksPerRow,
 * tokenCount, rmsEps}, Dequant_Q8_0.metal:199-314): per token t, q = Wq.n,
 * k = Wk.n (fp32), v = Wv.n written as fp16 (the KV-cache form). */
er_status er_hip_q8_0_fused_qkv(er_hip_ctx *ctx, er_stream stream, er_buffer wq, er_buffer wk, er_buffer wv,
                                er_buffer input, er_buffer out_q, er_buffer out_k, er_buffer out_v_f16,
                                er_buffer norm_weight, uint32_t q_rows, uint32_t kv_rows, uint32_t cols,
                                uint32_t token_count, float rms_eps);
/* dequant_q8_0_fused_qkv_turbo (Dequant_Q8_0.metal:835-933): as
 * er_hip_q8_0_fused_qkv with v kept in fp32 (out_v holds token_count*kv_rows
 * floats).  dequant_q8_0_fused_qkv_turbo_hybrid_v (:935-1031) writes v as fp16
 * and is er_hip_q8_0_fused_qkv itself. */
er_status er_hip_q8_0_fused_qkv_turbo(er_hip_ctx *ctx, er_stream stream, er_buffer wq, er_buffer wk,
                                      er_buffer wv, er_buffer input, er_buffer out_q, er_buffer out_k,
                                      er_buffer out_v, er_buffer norm_weight, uint32_t q_rows,
                                      uint32_t kv_rows, uint32_t cols, uint32_t token_count, float rms_eps);
/* dequant_q8_0_fused_gate_up_silu (ERFusedGateUpSiluParams{rows, cols,
 * blocksPerRow, tokenCount, rmsEps}, Dequant_Q8_0.metal:316-330, 399-483):
 * activated[t*rows + i] = silu(gate_i . n) * (up_i . n), silu(v) = v / (1 + exp(-v)). */
er_status er_hip_q8_0_fused_gate_up_silu(er_hip_ctx *ctx, er_stream stream, er_buffer w_gate,
                                         er_buffer w_up, er_buffer input, er_buffer activated,
                                         er_buffer norm_weight, uint32_t rows, uint32_t cols,
                                         uint32_t token_count, float rms_eps);
/* dequant_q8_0_fused_final_norm_gemv (Dequant_Q8_0.metal:332-397): y = W.n, one token. */
er_status er_hip_q8_0_fused_final_norm_gemv(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                            er_buffer input, er_buffer output, er_buffer norm_weight,
                                            uint32_t rows, uint32_t cols, float rms_eps);
/* dequant_q8_0_gemv_f16out (Dequant_Q8_0.metal:485-534): y = W.x stored as fp16. */
er_status er_hip_q8_0_gemv_f16out(er_hip_ctx *ctx, er_stream stream, er_buffer weight, er_buffer input,
                                  er_buffer output_f16, uint32_t rows, uint32_t cols);
/* dequant_q8_0_gemv_add (Dequant_Q8_0.metal:536-586): y = W.x + residual. */
er_status er_hip_q8_0_gemv_add(er_hip_ctx *ctx, er_stream stream, er_buffer weight, er_buffer input,
                               er_buffer residual, er_buffer output, uint32_t rows, uint32_t cols);

/* ---- batched (token-axis) GEMV: y[t*M + r] = W[r,:] . x[t*K : (t+1)*K] ----
 * GEMVKernel.encodeBatchedQ4KWeights (GEMVKernel.swift:682-702, validation
 * :1319-1361: batchSeq > 0, input >= batchSeq*K*4, output >= batchSeq*M*4 else
 * ENCODING_FAILED) and dequant_q8_0_gemv_batched (Dequant_Q8_0.metal:143-197).
 * The Q6_K variant has no reference counterpart but follows the same contract. */
er_status er_hip_encode_batched_q4k_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                            er_buffer input, er_buffer output, uint32_t batch_seq,
                                            uint32_t M, uint32_t K);
er_status er_hip_encode_batched_q6k_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                            er_buffer input, er_buffer output, uint32_t batch_seq,
                                            uint32_t M, uint32_t K);
er_status er_hip_encode_batched_q8_0_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                             er_buffer input, er_buffer output, uint32_t batch_seq,
                                             uint32_t M, uint32_t K);

/* ---- prefill GEMM on the matrix cores: Y[t][n] = sum_k X[t][k] * W[n][k] ----
 * X is bf16 [tokens][K] (16-byte aligned), W the raw Q4_K / Q8_0 rows of an
 * [K, N] tensor, Y fp32 [tokens][N].  The reference has no quantised GEMM: its
 * prefill is the token-batched GEMV (dequant_q8_0_gemv_batched,
 * Dequant_Q8_0.metal:143-197; per-token GEMV loop, LlamaLanguageModel.swift:2552-2617)
 * and these entry points compute the same product with the weights
 * dequantised to bf16 tiles and multiplied with fp32 accumulation.
 * Validation: tokens >= 1; Q4_K K % 256 == 0, Q8_0 K % 64 == 0, else
 * INVALID_VECTOR_SHAPE; weight too short -> INVALID_MATRIX_SHAPE; x shorter
 * than tokens*K*2 or y shorter than tokens*N*4 -> ENCODING_FAILED. */
er_status er_hip_gemm_q4_k(er_hip_ctx *ctx, er_stream stream, er_buffer weight, er_buffer x_bf16,
                           er_buffer y, uint32_t tokens, uint32_t N, uint32_t K);
er_status er_hip_gemm_q8_0(er_hip_ctx *ctx, er_stream stream, er_buffer weight, er_buffer x_bf16,
                           er_buffer y, uint32_t tokens, uint32_t N, uint32_t K);

/* ---- projection by tensor descriptor (Gemma4LanguageModel.encodeProjection,
 * Sources/EdgeRunner/Models/Gemma4LanguageModel.swift:4207-4285): dispatches on
 * tensor->data_type (Q8_0, Q4_K, Q6_K); shape = [K, M]; tokens >= 1 selects the
 * batched form.  Other data types return INVALID_ARGUMENT. ---- */
er_status er_hip_encode_projection(er_hip_ctx *ctx, er_stream stream,
                                   const er_tensor_storage *tensor, er_buffer input,
                                   er_buffer output, uint32_t tokens);

#ifdef __cplusplus
}
#endif

#endif /* ER_HIP_H */
