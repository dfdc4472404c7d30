"""EdgeRunnerHIP: MI355X (gfx950) quantized-matmul backend for EdgeRunner.

GGUF Q8_0 / Q4_K / Q6_K dequantisation, decode GEMV and prefill GEMM as
hand-written HIP kernels behind the C ABI in include/er_hip.h.  This Python
package is the host-side mirror of the reference's Swift dispatch protocol
(GEMVKernel, Dequant*Kernel) used by the tests and the benchmark.
"""
from .runtime import (AllocationFailed, Buffer, Capture, Context, Graph, DequantKernelError, DeviceError,  # noqa: F401
                      EdgeRunnerHIPError, EncodingFailed, Event, FunctionNotFound, GEMVError,
                      InvalidArgument, InvalidBlockDataCount, InvalidMatrixShape,
                      InvalidVectorShape, LibraryNotFound, Stream, default_context,
                      WeightLoaderError, FileNotFound, InvalidFormat, UnsupportedVersion,
                      UnsupportedDataType, MmapFailed, MissingMetadata, TensorNotFound)
from .gemv import (DequantQ4KMKernel, DequantQ6KKernel, DequantQ8_0Kernel,  # noqa: F401
                   FusedQ8Kernel, GEMVKernel, QuantGEMMKernel, QuantizeQ8RowsKernel, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0)

__all__ = [
    "Context", "Buffer", "Stream", "Event", "Graph", "Capture", "default_context",
    "GEMVKernel", "FusedQ8Kernel", "QuantGEMMKernel", "QuantizeQ8RowsKernel", "DequantQ8_0Kernel", "DequantQ4KMKernel", "DequantQ6KKernel",
    "GEMVError", "DequantKernelError", "EdgeRunnerHIPError", "WeightLoaderError",
    "TYPE_Q8_0", "TYPE_Q4_K", "TYPE_Q6_K",
]
