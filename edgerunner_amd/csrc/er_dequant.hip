// er_dequant.hip -- raw GGUF blocks -> fp32 (load-time dequantisation).
//
// Replaces the Metal kernels dequant_q8_0 (Dequant_Q8_0.metal:51-64),
// dequant_q4_k_m (Dequant_Q4_K_M.metal:28-68) and dequant_q6_k
// (Dequant_Q6_K.metal:20-58).  The reference runs one thread per block with
// byte loads; here each thread owns 4 (Q8_0) or 8 (Q4_K, Q6_K) output
// positions so that every store is a coalesced 16-byte float4 and the grid
// has enough waves to cover 256 CUs.
//
// Every dequantised value is exact in fp32 (Q8_0 d*q <= 18 significant bits,
// Q6_K (d*sc)*q <= 23, Q4_K (d*sc)*q <= 21 and dmin*m <= 17 with a single
// rounding in the subtraction), so the results are bit-identical to the CPU
// reference regardless of FMA contraction.
#include "er_common.h"

// One thread per (block, 4 consecutive weights).
extern "C" __global__ void __launch_bounds__(256)
er_dequant_q8_0(const uint8_t *__restrict__ blocks, float *__restrict__ out, uint64_t nblocks) {
    const uint64_t total = nblocks * 8u;
    for (uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; gid < total;
         gid += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t b = gid >> 3;
        const uint32_t k = (uint32_t)gid & 7u;
        const uint8_t *p = blocks + b * 34u;
        const float d = f16_to_f32(ld2(p));
        const uint32_t q = ld4_a2(p + 2 + 4 * k);
        float4 o;
        o.x = d * sb(q, 0);
        o.y = d * sb(q, 1);
        o.z = d * sb(q, 2);
        o.w = d * sb(q, 3);
        *(float4 *)(out + b * 32u + 4u * k) = o;
    }
}

// One thread per (super-block, qs dword t): the dword's low nibbles are
// weights 64p+l0..+3 of sub-block 2p, the high nibbles weights 64p+32+l0..+3
// of sub-block 2p+1 (p = t/8, l0 = 4*(t%8)).
extern "C" __global__ void __launch_bounds__(256)
er_dequant_q4_k(const uint8_t *__restrict__ blocks, float *__restrict__ out, uint64_t nblocks) {
    const uint64_t total = nblocks * 32u;
    for (uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; gid < total;
         gid += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t b = gid >> 5;
        const uint32_t t = (uint32_t)gid & 31u;
        const uint32_t p = t >> 3, l0 = (t & 7u) << 2;
        const uint8_t *blk = blocks + b * 144u;
        const u32x4 hdr = ld16_a16(blk);
        const uint32_t q = ld4_a4(blk + 16 + 4 * t);
        const float d = f16_to_f32(hdr.x & 0xffffu);
        const float dmin = f16_to_f32(hdr.x >> 16);
        uint32_t sc2, m2;
        q4k_scales_pair(hdr.y, hdr.z, hdr.w, p, &sc2, &m2);
        const float scA = d * ub0(sc2), mnA = dmin * ub0(m2);
        const float scB = d * ub1(sc2), mnB = dmin * ub1(m2);
        const uint32_t lo = q & 0x0f0f0f0fu, hi = (q >> 4) & 0x0f0f0f0fu;
        float4 a, c;
        a.x = scA * ub0(lo) - mnA;
        a.y = scA * ub1(lo) - mnA;
        a.z = scA * ub2(lo) - mnA;
        a.w = scA * ub3(lo) - mnA;
        c.x = scB * ub0(hi) - mnB;
        c.y = scB * ub1(hi) - mnB;
        c.z = scB * ub2(hi) - mnB;
        c.w = scB * ub3(hi) - mnB;
        float *o = out + b * 256u + 64u * p + l0;
        *(float4 *)o = a;
        *(float4 *)(o + 32) = c;
    }
}

// One thread per (super-block, half h, lanes l0..l0+3), l0 = 4*(t%8):
// q1..q4 land at 128h + {0,32,64,96} + l0.
extern "C" __global__ void __launch_bounds__(256)
er_dequant_q6_k(const uint8_t *__restrict__ blocks, float *__restrict__ out, uint64_t nblocks) {
    const uint64_t total = nblocks * 16u;
    for (uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; gid < total;
         gid += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t b = gid >> 4;
        const uint32_t t = (uint32_t)gid & 15u;
        const uint32_t h = t >> 3, l0 = (t & 7u) << 2;
        const uint8_t *blk = blocks + b * 210u;
        const uint32_t A = ld4_a2(blk + 64 * h + l0);
        const uint32_t B = ld4_a2(blk + 64 * h + 32 + l0);
        const uint32_t H = ld4_a2(blk + 128 + 32 * h + l0);
        const uint32_t is = l0 >> 4;
        const uint8_t *scp = blk + 192 + 8 * h + is;
        const float d = f16_to_f32(ld2(blk + 208));
        const float s1 = d * (float)(int8_t)scp[0];
        const float s2 = d * (float)(int8_t)scp[2];
        const float s3 = d * (float)(int8_t)scp[4];
        const float s4 = d * (float)(int8_t)scp[6];
        const uint32_t q1 = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
        const uint32_t q2 = (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
        const uint32_t q3 = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
        const uint32_t q4 = ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
        float *o = out + b * 256u + 128u * h + l0;
        float4 v;
        v.x = s1 * (ub0(q1) - 32.0f);
        v.y = s1 * (ub1(q1) - 32.0f);
        v.z = s1 * (ub2(q1) - 32.0f);
        v.w = s1 * (ub3(q1) - 32.0f);
        *(float4 *)o = v;
        v.x = s2 * (ub0(q2) - 32.0f);
        v.y = s2 * (ub1(q2) - 32.0f);
        v.z = s2 * (ub2(q2) - 32.0f);
        v.w = s2 * (ub3(q2) - 32.0f);
        *(float4 *)(o + 32) = v;
        v.x = s3 * (ub0(q3) - 32.0f);
        v.y = s3 * (ub1(q3) - 32.0f);
        v.z = s3 * (ub2(q3) - 32.0f);
        v.w = s3 * (ub3(q3) - 32.0f);
        *(float4 *)(o + 64) = v;
        v.x = s4 * (ub0(q4) - 32.0f);
        v.y = s4 * (ub1(q4) - 32.0f);
        v.z = s4 * (ub2(q4) - 32.0f);
        v.w = s4 * (ub3(q4) - 32.0f);
        *(float4 *)(o + 96) = v;
    }
}
