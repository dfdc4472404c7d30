/*
 * er_hip_probe.h -- measurement entry points of EdgeRunnerHIP.
 *
 * Not part of the drop-in interface (no reference counterpart) and not in
 * the product library: libedgerunner_probe.so, the measurement build of the
 * same sources (-DER_WITH_PROBES), exports them beside every er_hip.h entry
 * point.  Kernels whose timings are the ceilings the GEMV and decode-chain
 * designs are measured against (bench.py's "ceilings" leg) and a
 * clock-stamped copy of the prefill GEMM, launched through a context of that
 * library on the same streams and graphs as the product entry points.
 */
#ifndef ER_HIP_PROBE_H
#define ER_HIP_PROBE_H

#include "er_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Reads bytes (a multiple of 16, src 16-byte aligned) of src with
 * non-temporal 16-byte loads, `workgroups` x 256 lanes, grid-stride; sink
 * must hold workgroups * 256 uint32 (written only in a case that does not
 * occur with real data, so the loads cannot be removed). */
er_status er_hip_probe_stream_read(er_hip_ctx *ctx, er_stream stream, er_buffer src, uint64_t bytes,
                                   uint32_t workgroups, er_buffer sink);
/* The prefill GEMM (er_hip_gemm_q4_k / _q8_0 for type ER_TYPE_Q4_K /
 * ER_TYPE_Q8_0, same arguments and result) where its loader-specialised
 * kernel takes the shape (ER_ERR_INVALID_ARGUMENT otherwise), with clock
 * stamps: *items receives the number of work items and stamps (8-byte
 * aligned, at least 32 bytes per item) four uint64 per item: the 100 MHz
 * real-time counter and the shader-clock counter at the start of its
 * workgroup and after its epilogue.  The clock a workgroup ran at is
 * (s[3] - s[2]) / (s[1] - s[0]) x 100 MHz. */
er_status er_hip_probe_gemm_clock(er_hip_ctx *ctx, er_stream stream, er_tensor_type type, er_buffer weight,
                                  er_buffer x_bf16, er_buffer y, uint32_t tokens, uint32_t N, uint32_t K,
                                  er_buffer stamps, uint32_t *items);
/* One launch of an empty 64-thread kernel. */
er_status er_hip_probe_empty(er_hip_ctx *ctx, er_stream stream);
/* `rounds` grid-wide barriers across `workgroups` single-wave workgroups
 * (1 <= workgroups <= the CU count, so all are resident).  counter (16
 * bytes, 16-byte aligned) is cleared by a fill kernel first; every wait is
 * bounded by spin_limit polls; the launch adds its total polls to out[0] and
 * the number of waits that ran out to out[1] (uint32 each, 16 bytes, 16-byte
 * aligned), so out sums over the launches since the caller last cleared it. */
er_status er_hip_probe_grid_barrier(er_hip_ctx *ctx, er_stream stream, uint32_t workgroups, uint32_t rounds,
                                    uint32_t spin_limit, er_buffer counter, er_buffer out);

/* LDS read rate: one workgroup of `waves` (4, 8 or 16) waves per CU, each
 * wave `iters` x 8 independent 16-byte-per-lane LDS reads in the prefill
 * GEMM's A-fragment layout; sink holds CU count * 1024 uint32. */
er_status er_hip_probe_lds_read(er_hip_ctx *ctx, er_stream stream, uint32_t waves, uint32_t iters, er_buffer sink);
/* Matrix-core / vector-ALU overlap: one 8-wave workgroup per CU, `iters`
 * iterations of 8 bf16 MFMAs and/or 64 fp32 FMAs per wave; mode 0 MFMA
 * alone, 1 FMAs alone, 2 both from different waves of each SIMD, 3 both
 * interleaved in one wave; 4 and 5: 8 int8 MFMAs (32x32x32) per iteration
 * on waves 0-3, alone (4) or each followed by the per-block rescale of its 16
 * int32 sums per lane (5: convert, scale product, fused multiply-add);
 * sink holds CU count * 512 uint32. */
er_status er_hip_probe_mfma_valu(er_hip_ctx *ctx, er_stream stream, uint32_t mode, uint32_t iters, er_buffer sink);

#ifdef __cplusplus
}
#endif

#endif /* ER_HIP_PROBE_H */
