"""GEMVKernel / Dequant*Kernel: the reference's Swift dispatch protocol on HIP.

Method names and argument meaning follow
Sources/EdgeRunnerMetal/GEMVKernel.swift (encode* append to the caller's
stream and never allocate; execute* allocate, run, wait and copy out) and
Sources/EdgeRunnerIO/Dequant{Q8_0,Q4KM,Q6K}Kernel.swift (dequantise).
Validation errors are raised as the same Swift error cases.
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from . import _ffi
from .runtime import (Buffer, Context, InvalidBlockDataCount, InvalidVectorShape, Stream, check,
                      default_context)

Q8_0_BLOCK_BYTES = 34
Q4_K_BLOCK_BYTES = 144
Q6_K_BLOCK_BYTES = 210

TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q6_K = 14


def _sh(stream: Optional[Stream]):
    return stream.handle if stream is not None else None


def _u8(raw) -> np.ndarray:
    if isinstance(raw, (bytes, bytearray, memoryview)):
        return np.frombuffer(raw, dtype=np.uint8)
    return np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)


class GEMVKernel:
    """Quantized GEMV dispatch (GEMVKernel.swift:6-1433, K-quant + Q8_0 part)."""

    def __init__(self, ctx: Optional[Context] = None):
        self.ctx = ctx or default_context()
        self.lib = self.ctx.lib

    # ---------------------------------------------------------------- encode
    def encodeQ4KWeights(self, stream: Optional[Stream], weightBuffer: Buffer, inputBuffer: Buffer,
                         outputBuffer: Buffer, M: int, K: int) -> None:
        check(self.lib.er_hip_encode_q4k_weights(self.ctx.handle, _sh(stream), weightBuffer.raw,
                                                 inputBuffer.raw, outputBuffer.raw, M, K))

    def encodeQ6KWeights(self, stream: Optional[Stream], weightBuffer: Buffer, inputBuffer: Buffer,
                         outputBuffer: Buffer, M: int, K: int) -> None:
        check(self.lib.er_hip_encode_q6k_weights(self.ctx.handle, _sh(stream), weightBuffer.raw,
                                                 inputBuffer.raw, outputBuffer.raw, M, K))

    def encodeQ8_0Weights(self, stream: Optional[Stream], weightBuffer: Buffer,
                          inputBuffer: Buffer, outputBuffer: Buffer, M: int, K: int) -> None:
        check(self.lib.er_hip_encode_q8_0_weights(self.ctx.handle, _sh(stream), weightBuffer.raw,
                                                  inputBuffer.raw, outputBuffer.raw, M, K))

    # The reference's alternative encoders (GEMVKernel.swift:724-877, 1045,
    # 1184): other Metal lane mappings of the same product.  Each is its
    # canonical entry point under the reference's name (same validation and
    # bit-identical results).
    def _encode_alias(self, entry: str, stream, weightBuffer, inputBuffer, outputBuffer, M, K) -> None:
        check(getattr(self.lib, entry)(self.ctx.handle, _sh(stream), weightBuffer.raw, inputBuffer.raw,
                                       outputBuffer.raw, M, K))

    def encodeQ4KWeightsPacked(self, stream, weightBuffer, inputBuffer, outputBuffer, M, K) -> None:
        self._encode_alias("er_hip_encode_q4k_weights_packed", stream, weightBuffer, inputBuffer, outputBuffer, M, K)

    def encodeQ4KWeightsPackedFourRows(self, stream, weightBuffer, inputBuffer, outputBuffer, M, K) -> None:
        self._encode_alias("er_hip_encode_q4k_weights_packed_four_rows", stream, weightBuffer, inputBuffer,
                           outputBuffer, M, K)

    def encodeQ4KWeightsLlamaStyle(self, stream, weightBuffer, inputBuffer, outputBuffer, M, K) -> None:
        self._encode_alias("er_hip_encode_q4k_weights_llama_style", stream, weightBuffer, inputBuffer,
                           outputBuffer, M, K)

    def encodeQ4KWeightsTwoRows(self, stream, weightBuffer, inputBuffer, outputBuffer, M, K) -> None:
        self._encode_alias("er_hip_encode_q4k_weights_two_rows", stream, weightBuffer, inputBuffer, outputBuffer,
                           M, K)

    def encodeQ6KWeightsPacked(self, stream, weightBuffer, inputBuffer, outputBuffer, M, K) -> None:
        self._encode_alias("er_hip_encode_q6k_weights_packed", stream, weightBuffer, inputBuffer, outputBuffer, M, K)

    def encodeQ4KWeightsLlamaStyleDual(self, stream, weightBufferA, weightBufferB, inputBuffer, outputBufferA,
                                       outputBufferB, M, K) -> None:
        check(self.lib.er_hip_encode_q4k_weights_llama_style_dual(
            self.ctx.handle, _sh(stream), weightBufferA.raw, weightBufferB.raw, inputBuffer.raw,
            outputBufferA.raw, outputBufferB.raw, M, K))

    def encodeQ4KWeightsTriplePacked(self, stream, weightBufferA, weightBufferB, weightBufferC, inputBuffer,
                                     outputBufferA, outputBufferB, outputBufferC, rowsA, rowsB, rowsC, K) -> None:
        check(self.lib.er_hip_encode_q4k_weights_triple_packed(
            self.ctx.handle, _sh(stream), weightBufferA.raw, weightBufferB.raw, weightBufferC.raw,
            inputBuffer.raw, outputBufferA.raw, outputBufferB.raw, outputBufferC.raw, rowsA, rowsB, rowsC, K))

    def executeQ4KWeightsWithWeightBuffer(self, weightBuffer: Buffer, x, M: int, K: int) -> np.ndarray:
        """GEMVKernel.executeQ4KWeightsWithWeightBuffer (GEMVKernel.swift:605): the C
        convenience er_hip_execute_q4k_weights_with_weight_buffer (allocates x and y, waits)."""
        return self._execute_c("er_hip_execute_q4k_weights_with_weight_buffer", weightBuffer.raw, x, M, M, K)

    def executeQ6KWeightsWithWeightBuffer(self, weightBuffer: Buffer, x, M: int, K: int) -> np.ndarray:
        """GEMVKernel.executeQ6KWeightsWithWeightBuffer (GEMVKernel.swift:1146)."""
        return self._execute_c("er_hip_execute_q6k_weights_with_weight_buffer", weightBuffer.raw, x, M, M, K)

    def _execute_c(self, entry: str, weight, x, yCount: int, *shape) -> np.ndarray:
        xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        y = np.empty(max(yCount, 1), dtype=np.float32)
        check(getattr(self.lib, entry)(self.ctx.handle, weight, xv.ctypes.data, xv.size, y.ctypes.data, yCount,
                                       *shape))
        return y[:yCount]

    def encodeBatchedQ4KWeights(self, stream: Optional[Stream], weightBuffer: Buffer,
                                inputBuffer: Buffer, outputBuffer: Buffer, batchSeq: int, M: int,
                                K: int) -> None:
        check(self.lib.er_hip_encode_batched_q4k_weights(
            self.ctx.handle, _sh(stream), weightBuffer.raw, inputBuffer.raw, outputBuffer.raw,
            batchSeq, M, K))

    def encodeBatchedQ6KWeights(self, stream: Optional[Stream], weightBuffer: Buffer,
                                inputBuffer: Buffer, outputBuffer: Buffer, batchSeq: int, M: int,
                                K: int) -> None:
        check(self.lib.er_hip_encode_batched_q6k_weights(
            self.ctx.handle, _sh(stream), weightBuffer.raw, inputBuffer.raw, outputBuffer.raw,
            batchSeq, M, K))

    def encodeBatchedQ8_0Weights(self, stream: Optional[Stream], weightBuffer: Buffer,
                                 inputBuffer: Buffer, outputBuffer: Buffer, batchSeq: int, M: int,
                                 K: int) -> None:
        check(self.lib.er_hip_encode_batched_q8_0_weights(
            self.ctx.handle, _sh(stream), weightBuffer.raw, inputBuffer.raw, outputBuffer.raw,
            batchSeq, M, K))

    def encodeQ4KWeightsDual(self, stream: Optional[Stream], weightBufferA: Buffer,
                             weightBufferB: Buffer, inputBuffer: Buffer, outputBufferA: Buffer,
                             outputBufferB: Buffer, M: int, K: int) -> None:
        """GEMVKernel.encodeQ4KWeightsDual (GEMVKernel.swift:879-928)."""
        check(self.lib.er_hip_encode_q4k_weights_dual(
            self.ctx.handle, _sh(stream), weightBufferA.raw, weightBufferB.raw, inputBuffer.raw,
            outputBufferA.raw, outputBufferB.raw, M, K))

    def encodeQ4KWeightsTriple(self, stream: Optional[Stream], weightBufferA: Buffer,
                               weightBufferB: Buffer, weightBufferC: Buffer, inputBuffer: Buffer,
                               outputBufferA: Buffer, outputBufferB: Buffer, outputBufferC: Buffer,
                               rowsA: int, rowsB: int, rowsC: int, K: int) -> None:
        """GEMVKernel.encodeQ4KWeightsTriple (GEMVKernel.swift:978-1043)."""
        check(self.lib.er_hip_encode_q4k_weights_triple(
            self.ctx.handle, _sh(stream), weightBufferA.raw, weightBufferB.raw, weightBufferC.raw,
            inputBuffer.raw, outputBufferA.raw, outputBufferB.raw, outputBufferC.raw, rowsA, rowsB,
            rowsC, K))

    def encodeQ4KWeightsDualGeGLU(self, stream: Optional[Stream], gateWeightBuffer: Buffer,
                                  upWeightBuffer: Buffer, inputBuffer: Buffer, outputBuffer: Buffer,
                                  M: int, K: int) -> None:
        """GEMVKernel.encodeQ4KWeightsDualGeGLU (GEMVKernel.swift:930-976)."""
        check(self.lib.er_hip_encode_q4k_weights_dual_geglu(
            self.ctx.handle, _sh(stream), gateWeightBuffer.raw, upWeightBuffer.raw,
            inputBuffer.raw, outputBuffer.raw, M, K))

    @staticmethod
    def q6KTop1PartialCount(rows: int) -> int:
        """Entries each partial buffer of the top-1 head needs
        (GEMVKernel.q6KTop1PartialCount, GEMVKernel.swift:50-52)."""
        return (rows + 3) // 4

    def encodeQ6KWeightsPackedTop1(self, stream: Optional[Stream], weightBuffer: Buffer,
                                   inputBuffer: Buffer, partialValuesBuffer: Buffer,
                                   partialIndicesBuffer: Buffer, outputIndexBuffer: Buffer,
                                   M: int, K: int) -> None:
        """GEMVKernel.encodeQ6KWeightsPackedTop1 (GEMVKernel.swift:1205-1265):
        outputIndexBuffer[0] (uint32) = the row of the largest W.x value,
        lowest row on ties."""
        check(self.lib.er_hip_encode_q6k_weights_packed_top1(
            self.ctx.handle, _sh(stream), weightBuffer.raw, inputBuffer.raw,
            partialValuesBuffer.raw, partialIndicesBuffer.raw, outputIndexBuffer.raw, M, K))

    def executeQ6KWeightsTop1(self, rawWeights, x, M: int, K: int) -> int:
        """Uploads W and x, runs the top-1 head and returns the row index."""
        xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        if xv.size != K:
            raise InvalidVectorShape(f"x.count {xv.size} != K {K}")
        ctx = self.ctx
        n = self.q6KTop1PartialCount(M)
        wb, xb = ctx.upload(_u8(rawWeights)), ctx.upload(xv)
        pv, pi, ob = ctx.alloc(max(4, 4 * n)), ctx.alloc(max(4, 4 * n)), ctx.alloc(4)
        try:
            self.encodeQ6KWeightsPackedTop1(None, wb, xb, pv, pi, ob, M, K)
            ctx.synchronize()
            return int(ob.download(np.uint32, 1)[0])
        finally:
            for b in (wb, xb, pv, pi, ob):
                b.free()

    def executeQ4KWeightsMulti(self, rawWeights: list, x, rows: list, K: int, geglu: bool = False):
        """Uploads 2 or 3 Q4_K matrices sharing x and runs the dual / triple
        (or, with geglu=True and two equal-height matrices, the fused GeGLU)
        projection; returns the list of outputs (one array for GeGLU)."""
        ctx = self.ctx
        xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        wbs = [ctx.upload(_u8(w)) for w in rawWeights]
        xb = ctx.upload(xv)
        try:
            if geglu:
                yb = ctx.alloc(rows[0] * 4)
                self.encodeQ4KWeightsDualGeGLU(None, wbs[0], wbs[1], xb, yb, rows[0], K)
                ctx.synchronize()
                out = yb.download(np.float32, rows[0])
                yb.free()
                return out
            ybs = [ctx.alloc(m * 4) for m in rows]
            if len(rawWeights) == 2:
                self.encodeQ4KWeightsDual(None, wbs[0], wbs[1], xb, ybs[0], ybs[1], rows[0], K)
            else:
                self.encodeQ4KWeightsTriple(None, wbs[0], wbs[1], wbs[2], xb, ybs[0], ybs[1], ybs[2],
                                            rows[0], rows[1], rows[2], K)
            ctx.synchronize()
            outs = [b.download(np.float32, m) for b, m in zip(ybs, rows)]
            for b in ybs:
                b.free()
            return outs
        finally:
            for b in wbs:
                b.free()
            xb.free()

    def encodeTensor(self, stream: Optional[Stream], tensor, inputBuffer: Buffer,
                     outputBuffer: Buffer, tokens: int = 1) -> None:
        """encodeProjection on a loaded TensorStorage (edgerunner_amd.gguf):
        its data type and GGUF shape [K, M] pick the kernel
        (Gemma4LanguageModel.swift:4207-4285)."""
        import ctypes as C
        check(self.lib.er_hip_encode_projection(self.ctx.handle, _sh(stream), C.byref(tensor.storage),
                                                inputBuffer.raw, outputBuffer.raw, tokens))

    def encodeProjection(self, stream: Optional[Stream], weightBuffer: Buffer, dataType: int,
                         inputBuffer: Buffer, outputBuffer: Buffer, M: int, K: int,
                         tokens: int = 1, byteOffset: int = 0) -> None:
        """Gemma4LanguageModel.encodeProjection (Gemma4LanguageModel.swift:4207-4285)."""
        t = _ffi.er_tensor_storage()
        t.buffer = weightBuffer.raw
        t.byte_offset = byteOffset
        t.data_type = dataType
        t.ndim = 2
        t.shape[0] = K
        t.shape[1] = M
        import ctypes as C
        check(self.lib.er_hip_encode_projection(self.ctx.handle, _sh(stream), C.byref(t),
                                                inputBuffer.raw, outputBuffer.raw, tokens))

    # ---------------------------------------------------------------- execute
    def _execute(self, encode, block_bytes: int, rawWeights, x, M: int, K: int,
                 batchSeq: Optional[int] = None) -> np.ndarray:
        w = _u8(rawWeights)
        xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        per = 32 if block_bytes == Q8_0_BLOCK_BYTES else 256
        tokens = 1 if batchSeq is None else batchSeq
        # validateKQuantInputShape(vectorCount: x.count) (GEMVKernel.swift:1415-1432)
        if batchSeq is None and xv.size != K:
            raise InvalidVectorShape(f"x.count {xv.size} != K {K}")
        if batchSeq is not None and (batchSeq <= 0 or xv.size != batchSeq * K):
            raise InvalidVectorShape(f"x.count {xv.size} != batchSeq*K {tokens * K}")
        if K <= 0 or K % per != 0:
            raise InvalidVectorShape(f"K={K} must be a positive multiple of {per}")
        ctx = self.ctx
        wb = ctx.upload(w) if w.size else ctx.alloc(0)
        xb = ctx.upload(xv)
        yb = ctx.alloc(tokens * M * 4)
        try:
            if batchSeq is None:
                encode(None, wb, xb, yb, M, K)
            else:
                encode(None, wb, xb, yb, batchSeq, M, K)
            ctx.synchronize()
            return yb.download(np.float32, tokens * M)
        finally:
            wb.free()
            xb.free()
            yb.free()

    def executeQ4KWeights(self, rawWeights, x, M: int, K: int) -> np.ndarray:
        return self._execute(self.encodeQ4KWeights, Q4_K_BLOCK_BYTES, rawWeights, x, M, K)

    def executeQ6KWeights(self, rawWeights, x, M: int, K: int) -> np.ndarray:
        return self._execute(self.encodeQ6KWeights, Q6_K_BLOCK_BYTES, rawWeights, x, M, K)

    def executeQ8_0Weights(self, rawWeights, x, M: int, K: int) -> np.ndarray:
        return self._execute(self.encodeQ8_0Weights, Q8_0_BLOCK_BYTES, rawWeights, x, M, K)

    def executeBatchedQ4KWeights(self, rawWeights, x, batchSeq: int, M: int, K: int) -> np.ndarray:
        return self._execute(self.encodeBatchedQ4KWeights, Q4_K_BLOCK_BYTES, rawWeights, x, M, K,
                             batchSeq)

    def executeBatchedQ6KWeights(self, rawWeights, x, batchSeq: int, M: int, K: int) -> np.ndarray:
        return self._execute(self.encodeBatchedQ6KWeights, Q6_K_BLOCK_BYTES, rawWeights, x, M, K,
                             batchSeq)

    def executeBatchedQ8_0Weights(self, rawWeights, x, batchSeq: int, M: int,
                                  K: int) -> np.ndarray:
        return self._execute(self.encodeBatchedQ8_0Weights, Q8_0_BLOCK_BYTES, rawWeights, x, M, K,
                             batchSeq)


class _DequantKernel:
    block_bytes = 0
    weights_per_block = 0
    entry = ""

    def __init__(self, ctx: Optional[Context] = None):
        self.ctx = ctx or default_context()

    def encode(self, stream: Optional[Stream], blocks: Buffer, count: int, out: Buffer) -> None:
        check(getattr(self.ctx.lib, self.entry)(self.ctx.handle, _sh(stream), blocks.raw, count,
                                                out.raw))

    def dequantise(self, blockData, count: int) -> np.ndarray:
        """dequantise(blockData:blockCount:) -- exact byte count required
        (DequantQ8_0Kernel.swift:23-29)."""
        data = _u8(blockData)
        expected = count * self.block_bytes
        if data.size != expected:
            raise InvalidBlockDataCount(
                f"invalidBlockDataCount(expected: {expected}, actual: {data.size})",
                expected=expected, actual=int(data.size))
        ctx = self.ctx
        if count == 0:
            return np.zeros(0, dtype=np.float32)
        ib = ctx.upload(data)
        ob = ctx.alloc(count * self.weights_per_block * 4)
        try:
            self.encode(None, ib, count, ob)
            ctx.synchronize()
            return ob.download(np.float32, count * self.weights_per_block)
        finally:
            ib.free()
            ob.free()


class DequantQ8_0Kernel(_DequantKernel):
    """Sources/EdgeRunnerIO/DequantQ8_0Kernel.swift:18-78."""
    block_bytes = Q8_0_BLOCK_BYTES
    weights_per_block = 32
    entry = "er_hip_dequant_q8_0"


class DequantQ4KMKernel(_DequantKernel):
    """Sources/EdgeRunnerIO/DequantQ4KMKernel.swift:18-78."""
    block_bytes = Q4_K_BLOCK_BYTES
    weights_per_block = 256
    entry = "er_hip_dequant_q4_k"


class DequantQ6KKernel(_DequantKernel):
    """Sources/EdgeRunnerIO/DequantQ6KKernel.swift:18-78."""
    block_bytes = Q6_K_BLOCK_BYTES
    weights_per_block = 256
    entry = "er_hip_dequant_q6_k"


class QuantGEMMKernel:
    """Prefill GEMM over raw Q4_K / Q8_0 weights on the matrix cores.

    The reference has no quantised GEMM (its prefill is the token-batched
    GEMV, Dequant_Q8_0.metal:143-197); this class keeps the GEMVKernel style:
    encode* appends to a stream, execute* allocates, runs, waits and copies out.
    X is bf16 bits (uint16) [tokens][K]; Y is fp32 [tokens][N]."""

    def __init__(self, ctx: Optional[Context] = None):
        self.ctx = ctx or default_context()
        self.lib = self.ctx.lib

    def encodeQ4K(self, stream: Optional[Stream], weightBuffer: Buffer, inputBuffer: Buffer,
                  outputBuffer: Buffer, tokens: int, N: int, K: int) -> None:
        check(self.lib.er_hip_gemm_q4_k(self.ctx.handle, _sh(stream), weightBuffer.raw,
                                        inputBuffer.raw, outputBuffer.raw, tokens, N, K))

    def encodeQ8_0(self, stream: Optional[Stream], weightBuffer: Buffer, inputBuffer: Buffer,
                   outputBuffer: Buffer, tokens: int, N: int, K: int) -> None:
        check(self.lib.er_hip_gemm_q8_0(self.ctx.handle, _sh(stream), weightBuffer.raw,
                                        inputBuffer.raw, outputBuffer.raw, tokens, N, K))

    def execute(self, fmt: str, rawWeights, X_bf16, tokens: int, N: int, K: int) -> np.ndarray:
        enc = {"q4_k": self.encodeQ4K, "q8_0": self.encodeQ8_0}[fmt]
        w = _u8(rawWeights)
        x = np.ascontiguousarray(X_bf16, dtype=np.uint16).reshape(-1)
        if x.size != tokens * K:
            raise InvalidVectorShape(f"X holds {x.size} values, tokens*K = {tokens * K}")
        ctx = self.ctx
        wb = ctx.upload(w) if w.size else ctx.alloc(0)
        xb = ctx.upload(x)
        yb = ctx.alloc(tokens * N * 4)
        try:
            enc(None, wb, xb, yb, tokens, N, K)
            ctx.synchronize()
            return yb.download(np.float32, tokens * N).reshape(tokens, N)
        finally:
            wb.free()
            xb.free()
            yb.free()


class QuantizeQ8RowsKernel:
    """Q8_0 row quantizer: the reference's `quantize_q8_0_rows` pipeline as
    LlamaLanguageModel.encodeQ8Rows encodes it (LlamaLanguageModel.swift:1820-1850,
    kernel Dequant_Q8_0.metal:19-49).  encode appends to a stream;
    execute allocates, runs, waits and returns the destination bytes."""

    def __init__(self, ctx: Optional[Context] = None):
        self.ctx = ctx or default_context()
        self.lib = self.ctx.lib

    def encode(self, stream: Optional[Stream], sourceBuffer: Buffer, destinationBuffer: Buffer,
               rowCount: int, sourceRowStride: int, destinationRowBase: int,
               blocksPerRow: int) -> None:
        check(self.lib.er_hip_quantize_q8_0_rows(self.ctx.handle, _sh(stream), sourceBuffer.raw,
                                                 destinationBuffer.raw, rowCount, sourceRowStride,
                                                 destinationRowBase, blocksPerRow))

    def execute(self, source, rowCount: int, sourceRowStride: int, destinationRowBase: int,
                blocksPerRow: int, destination=None) -> np.ndarray:
        """source: fp32 values; destination: optional existing Q8_0 bytes whose
        rows outside [destinationRowBase, +rowCount) are kept."""
        src = np.ascontiguousarray(source, dtype=np.float32).reshape(-1)
        nbytes = (destinationRowBase + rowCount) * blocksPerRow * Q8_0_BLOCK_BYTES
        dst = (np.zeros(nbytes, np.uint8) if destination is None
               else np.ascontiguousarray(destination, dtype=np.uint8).reshape(-1))
        ctx = self.ctx
        sb = ctx.upload(src) if src.size else ctx.alloc(4)
        db = ctx.upload(dst) if dst.size else ctx.alloc(2)
        try:
            self.encode(None, sb, db, rowCount, sourceRowStride, destinationRowBase, blocksPerRow)
            ctx.synchronize()
            return db.download(np.uint8, dst.size) if dst.size else dst
        finally:
            sb.free()
            db.free()


class FusedQ8Kernel:
    """Fused Q8_0 projections: the pipelines LlamaLanguageModel fetches by name
    (LlamaLanguageModel.swift:260-275; kernels Dequant_Q8_0.metal:199-586).
    encode* append to a stream; the RMSNorm-fused ones normalise each token's
    x with norm weight and eps as RMSNorm does (x * rmsScale * w)."""

    def __init__(self, ctx: Optional[Context] = None):
        self.ctx = ctx or default_context()
        self.lib = self.ctx.lib

    def encodeFusedQKV(self, stream: Optional[Stream], wq: Buffer, wk: Buffer, wv: Buffer,
                       inputBuffer: Buffer, outQ: Buffer, outK: Buffer, outVHalf: Buffer,
                       normWeight: Buffer, qRows: int, kvRows: int, cols: int, tokenCount: int,
                       rmsEps: float) -> None:
        """dequant_q8_0_fused_qkv: q, k fp32; v fp16."""
        check(self.lib.er_hip_q8_0_fused_qkv(self.ctx.handle, _sh(stream), wq.raw, wk.raw, wv.raw,
                                             inputBuffer.raw, outQ.raw, outK.raw, outVHalf.raw,
                                             normWeight.raw, qRows, kvRows, cols, tokenCount, rmsEps))

    def encodeFusedQKVTurbo(self, stream: Optional[Stream], wq: Buffer, wk: Buffer, wv: Buffer,
                            inputBuffer: Buffer, outQ: Buffer, outK: Buffer, outV: Buffer,
                            normWeight: Buffer, qRows: int, kvRows: int, cols: int, tokenCount: int,
                            rmsEps: float) -> None:
        """dequant_q8_0_fused_qkv_turbo: as encodeFusedQKV with v in fp32."""
        check(self.lib.er_hip_q8_0_fused_qkv_turbo(self.ctx.handle, _sh(stream), wq.raw, wk.raw, wv.raw,
                                                   inputBuffer.raw, outQ.raw, outK.raw, outV.raw,
                                                   normWeight.raw, qRows, kvRows, cols, tokenCount, rmsEps))

    def encodeFusedGateUpSilu(self, stream: Optional[Stream], wGate: Buffer, wUp: Buffer,
                              inputBuffer: Buffer, activated: Buffer, normWeight: Buffer, rows: int,
                              cols: int, tokenCount: int, rmsEps: float) -> None:
        """dequant_q8_0_fused_gate_up_silu: silu(gate . n) * (up . n)."""
        check(self.lib.er_hip_q8_0_fused_gate_up_silu(self.ctx.handle, _sh(stream), wGate.raw, wUp.raw,
                                                      inputBuffer.raw, activated.raw, normWeight.raw,
                                                      rows, cols, tokenCount, rmsEps))

    def encodeFusedFinalNormGEMV(self, stream: Optional[Stream], weight: Buffer, inputBuffer: Buffer,
                                 outputBuffer: Buffer, normWeight: Buffer, rows: int, cols: int,
                                 rmsEps: float) -> None:
        """dequant_q8_0_fused_final_norm_gemv: y = W . RMSNorm(x)."""
        check(self.lib.er_hip_q8_0_fused_final_norm_gemv(self.ctx.handle, _sh(stream), weight.raw,
                                                         inputBuffer.raw, outputBuffer.raw,
                                                         normWeight.raw, rows, cols, rmsEps))

    def encodeGEMVF16Out(self, stream: Optional[Stream], weight: Buffer, inputBuffer: Buffer,
                         outputHalf: Buffer, rows: int, cols: int) -> None:
        """dequant_q8_0_gemv_f16out: y = W . x stored as fp16."""
        check(self.lib.er_hip_q8_0_gemv_f16out(self.ctx.handle, _sh(stream), weight.raw,
                                               inputBuffer.raw, outputHalf.raw, rows, cols))

    def encodeGEMVAdd(self, stream: Optional[Stream], weight: Buffer, inputBuffer: Buffer,
                      residual: Buffer, outputBuffer: Buffer, rows: int, cols: int) -> None:
        """dequant_q8_0_gemv_add: y = W . x + residual."""
        check(self.lib.er_hip_q8_0_gemv_add(self.ctx.handle, _sh(stream), weight.raw,
                                            inputBuffer.raw, residual.raw, outputBuffer.raw, rows, cols))
