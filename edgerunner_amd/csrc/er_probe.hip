// er_probe.hip -- measurement kernels behind include/er_hip_probe.h: the
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
