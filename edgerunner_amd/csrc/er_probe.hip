// er_probe.hip -- measurement kernels behind er_hip_probe.h (built only into
// the measurement library, -DER_WITH_PROBES): the
// ceilings the GEMV and decode-chain designs are judged against, measured
// with the same launch machinery as the product kernels.
//
//   er_probe_stream_read : a coalesced non-temporal 16-byte-per-lane read of a
//                          buffer (grid-stride), the attainable HBM read rate
//                          of one launch of that size;
//   er_probe_empty       : a kernel that does nothing, the floor cost of one
//                          launch (inside a graph, its per-node cost);
//   er_probe_grid_barrier: `rounds` grid-wide barriers across the workgroups
//                          of one launch (one agent-scope counter, bounded
//                          waits), the cost a persistent kernel would pay per
//                          stage boundary instead of a launch boundary.
#include "er_common.h"

// XOR of every dword read; stored only when it equals `never` (the caller
// passes a value the data cannot produce in practice), so the loads stay.
extern "C" __global__ void __launch_bounds__(256)
    er_probe_stream_read(const u32x4 *__restrict__ src, uint64_t n16, uint32_t never, uint32_t *__restrict__ sink) {
    uint32_t acc = 0;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(src + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == never) sink[(uint64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

extern "C" __global__ void __launch_bounds__(64) er_probe_empty() {}

// One workgroup per CU at most (the host checks gridDim.x <= CU count, and a
// 64-thread workgroup with no LDS always fits beside the others, so every
// workgroup is resident).  Barrier r waits until the counter reaches
// (r + 1) * gridDim.x; each wait is bounded by `spin_limit` polls, after
// which the workgroup records a timeout in out[1] and carries on, so every
// wave reaches the end.  counter must be zero at launch; out[0] collects the
// polls (for checking), out[1] the timeouts.
extern "C" __global__ void __launch_bounds__(64)
    er_probe_grid_barrier(uint32_t *__restrict__ counter, uint32_t rounds, uint32_t spin_limit,
                          uint32_t *__restrict__ out) {
    if (threadIdx.x != 0) return;
    uint32_t polls = 0, timeouts = 0;
    for (uint32_t r = 0; r < rounds; ++r) {
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t target = (r + 1u) * gridDim.x;
        uint32_t n = 0;
        while (__hip_atomic_load(counter, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (++n >= spin_limit) {
                ++timeouts;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        polls += n;
    }
    __hip_atomic_fetch_add(out, polls, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(out + 1, timeouts, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Per-CU rates the prefill GEMM design rests on.  Both run one workgroup per
// CU (the host asks for 96 KB of LDS, so no second workgroup fits beside it)
// and keep their results alive through a store that real data never takes.
// ---------------------------------------------------------------------------
typedef __bf16 pb_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pb_f32x16 __attribute__((ext_vector_type(16)));
typedef int pb_i32x4 __attribute__((ext_vector_type(4)));
typedef int pb_i32x16 __attribute__((ext_vector_type(16)));

// LDS read rate: every wave issues, per iteration, 8 independent 16-byte-per-
// lane reads laid out like the GEMM's A fragments (lane l: row l % 32 of a
// 144-byte pitch, column 16 (l / 32)), and XORs them into its result.
extern "C" __global__ void __launch_bounds__(1024)
    er_probe_lds_read(uint32_t iters, uint32_t never, uint32_t *__restrict__ sink) {
    extern __shared__ __attribute__((aligned(16))) uint8_t plds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    for (uint32_t i = tid; i < 16384u; i += blockDim.x) ((uint32_t *)plds)[i] = i * 2654435761u;
    __syncthreads();
    u32x4 x = {0u, 0u, 0u, 0u};
    const uint32_t base = (lane & 31u) * 144u + 16u * (lane >> 5);
    uint32_t off = (wave * 1024u) & 32767u;
    for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
        for (uint32_t u = 0; u < 8u; ++u) x ^= *(const u32x4 *)(plds + ((base + ((off + 4608u * u) & 16383u)) & ~15u));
        off += 64u;
        asm volatile("" : "+v"(off));
    }
    const uint32_t v = x.x ^ x.y ^ x.z ^ x.w;
    if (v == never) sink[blockIdx.x * blockDim.x + tid] = v;
}

// Matrix-core / vector-ALU overlap, 8 waves (2 per SIMD: waves w and w + 4).
// Per iteration a wave of role MFMA issues 8 v_mfma_f32_32x32x16_bf16 on
// independent accumulators, a wave of role VALU 64 independent fp32 FMAs, and
// a wave of role BOTH the two interleaved (one matrix instruction, then 8
// FMAs).  mode: 0 waves 0-3 MFMA, 4-7 idle; 1 waves 0-3 VALU; 2 waves 0-3
// MFMA and 4-7 VALU (the two on each SIMD from different waves); 3 waves 0-3
// BOTH (from one wave).
//
// Modes 4 and 5 price an int8 path for the Q8_0 prefill GEMM: waves 0-3 issue
// 8 v_mfma_i32_32x32x32_i8 per iteration (one MFMA spans exactly one 32-wide
// Q8_0 block of K).  Mode 4 runs them alone.  Mode 5 gives each one the
// per-block rescale such a kernel cannot avoid: the block's int32 sums differ
// in scale per output (weight row n, token t), so each of a lane's 16 sums
// takes a convert, the product of the two block scales and a fused
// multiply-add into an fp32 accumulator (48 vector instructions per MFMA).
extern "C" __global__ void __launch_bounds__(512)
    er_probe_mfma_valu(uint32_t mode, uint32_t iters, uint32_t never, uint32_t *__restrict__ sink) {
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t role = wave < 4u ? (mode == 1u ? 2u : mode == 3u ? 3u : mode >= 4u ? mode : 1u)
                                    : (mode == 2u ? 2u : 0u);
    // every role keeps its accumulators inside its own branch, so no role
    // holds another's registers
    float y[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = (float)(tid + k);
    const float m = 1.0001f, c = 0.5f;
    float s = 0.0f;
    if (role == 1u || role == 3u) {
        pb_f32x16 acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[j][q] = 0.0f;
        pb_bf16x8 a, b;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            a[q] = (__bf16)(float)(tid + q);
            b[q] = (__bf16)(float)(3 * q);
        }
        if (role == 1u) {
            for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
        } else {
            for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
#pragma unroll
                    for (int k = 0; k < 8; ++k) y[k] = __builtin_fmaf(y[k], m, c);
                }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) s += acc[j][q];
    } else if (role == 2u) {
        for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
            for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int k = 0; k < 8; ++k) y[k] = __builtin_fmaf(y[k], m, c);
    } else if (role >= 4u) {
        const pb_i32x4 ia = {(int)(tid * 0x01030507u), (int)(tid ^ 0x7f3a1c05u), 0x05f3a1c7, (int)tid};
        const pb_i32x4 ib = {0x11223344, (int)(tid * 0x9e3779b1u), 0x7c0d5a13, 0x2468ace0};
        if (role == 4u) {
            pb_i32x16 iacc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) iacc[j][q] = 0;
            for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
                for (int j = 0; j < 8; ++j) iacc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ia, ib, iacc[j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) s += (float)iacc[j][q];
        } else {
            // per-token block scales in registers (a kernel would read them
            // from LDS); one weight-block scale per accumulator, changing
            // every iteration like the block index does
            pb_f32x16 acc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[j][q] = 0.0f;
            float sx[16], sw[8];
#pragma unroll
            for (int q = 0; q < 16; ++q) sx[q] = 1.0f + (float)(tid + q) * 1e-6f;
#pragma unroll
            for (int j = 0; j < 8; ++j) sw[j] = 1.0f + (float)(tid * 8u + j) * 1e-7f;
            const pb_i32x16 zero = {};
            pb_i32x4 ja = ia;
            // software-pipelined as a kernel would run it: the next block's
            // MFMA is issued before the previous block's sums are rescaled,
            // into other registers, so the two overlap
            pb_i32x16 r = __builtin_amdgcn_mfma_i32_32x32x32_i8(ja, ib, zero, 0, 0, 0);
            for (uint32_t it = 0; it < iters; ++it)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    // an opaque operand, so each product is issued (not one
                    // hoisted out of the loop for all)
                    asm volatile("" : "+v"(ja));
                    const pb_i32x16 rn = __builtin_amdgcn_mfma_i32_32x32x32_i8(ja, ib, zero, 0, 0, 0);
                    sw[j] *= m;
#pragma unroll
                    for (int q = 0; q < 16; ++q) acc[j][q] = __builtin_fmaf((float)r[q], sw[j] * sx[q], acc[j][q]);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 49, 0);
                    r = rn;
                }
#pragma unroll
            for (int q = 0; q < 16; ++q) s += (float)r[q];
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) s += acc[j][q];
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) s += y[k];
    const uint32_t v = __builtin_bit_cast(uint32_t, s);
    if (v == never) sink[blockIdx.x * 512u + tid] = v;
}
