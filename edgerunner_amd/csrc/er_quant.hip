// er_quant.hip -- Q8_0 row quantizer (the reference's quantize_q8_0_rows,
// Dequant_Q8_0.metal:19-49: the activation quantizer of the int8 path and the
// Q8_0 KV-cache writer, LlamaLanguageModel.swift:1820-1850).
//
// Row r of `rowCount` reads source[r * sourceRowStride + 32 b + i] and writes
// Q8_0 block b of destination row destinationRowBase + r:
//   scale = maxAbs > 0 ? maxAbs / 127 : 0          (fp32, IEEE division)
//   d     = fp16(scale), round to nearest even      (bytes 0..1)
//   q[i]  = scale == 0 ? 0 : clamp(rint(v / scale), -127, 127)   (bytes 2..33)
// The quotient uses the fp32 scale, not its fp16 rounding, as the reference.
//
// Mapping: 8 lanes per block, 4 values per lane (a 16-byte load when the
// source rows are 16-byte aligned, else 4 scalar loads); the block maximum is
// 3 DPP steps inside the 8-lane group.  A block is 34 bytes, so
// destination blocks are only 2-byte aligned: each lane stores its 4 q bytes
// as one 2-byte-aligned dword and lane 0 of the group stores d.  HBM-bound: 128
// bytes read and 34 written per block.
#include "er_common.h"

#define ER_QUANT_THREADS 256

// One Q8_0 block from 8 lanes holding 4 values each (this lane: values
// 4 sub .. 4 sub + 3); writes the block at blk.
ER_DEV void quantize_block(const float v[4], uint32_t sub, uint8_t *__restrict__ blk) {
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    // maximum over the 8 lanes of the block: DPP quad swaps, then the half-row mirror
    m = dpp_max<ER_DPP_QUAD_XOR1>(m);
    m = dpp_max<ER_DPP_QUAD_XOR2>(m);
    m = dpp_max<ER_DPP_ROW_HALF_MIRROR>(m);
    const float scale = m > 0.0f ? m / 127.0f : 0.0f;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int q = 0;
        if (scale != 0.0f) {
            const float t = rintf(v[i] / scale);
            q = (int)fminf(fmaxf(t, -127.0f), 127.0f);
        }
        packed |= ((uint32_t)q & 0xffu) << (8 * i);
    }
    // one 2-byte-aligned dword store (the global memory path's unaligned access mode)
    typedef uint32_t u32_a2 __attribute__((aligned(2)));
    *(u32_a2 *)(blk + 2u + 4u * sub) = packed;
    if (sub == 0) *(uint16_t *)blk = __builtin_bit_cast(uint16_t, (_Float16)scale);
}

// Grid-stride over blocks, one block per 8-lane group per pass; block
// indices are 32-bit (the host rejects 2^32 or more blocks).
template <bool VEC>
ER_DEV void quantize_q8_0_rows_impl(const float *__restrict__ src, uint8_t *__restrict__ dst,
                                    uint32_t rowCount, uint32_t srcStride, uint32_t dstRowBase,
                                    uint32_t blocksPerRow) {
    const uint32_t total = rowCount * blocksPerRow;
    const uint32_t sub = threadIdx.x & 7u;
    const uint32_t groups = gridDim.x * (ER_QUANT_THREADS / 8u);
    for (uint32_t g = blockIdx.x * (ER_QUANT_THREADS / 8u) + (threadIdx.x >> 3); g < total; g += groups) {
        const uint32_t r = g / blocksPerRow, b = g - r * blocksPerRow;
        const float *s = src + (size_t)r * srcStride + (size_t)b * 32u + 4u * sub;
        float v[4];
        if constexpr (VEC) {
            const float4 t = *(const float4 *)s;
            v[0] = t.x;
            v[1] = t.y;
            v[2] = t.z;
            v[3] = t.w;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = s[i];
        }
        quantize_block(v, sub, dst + (((size_t)dstRowBase + r) * blocksPerRow + b) * 34u);
    }
}

extern "C" __global__ void __launch_bounds__(ER_QUANT_THREADS)
    er_quantize_q8_0_rows_v(const float *__restrict__ src, uint8_t *__restrict__ dst, uint32_t rowCount,
                            uint32_t srcStride, uint32_t dstRowBase, uint32_t blocksPerRow) {
    quantize_q8_0_rows_impl<true>(src, dst, rowCount, srcStride, dstRowBase, blocksPerRow);
}

extern "C" __global__ void __launch_bounds__(ER_QUANT_THREADS)
    er_quantize_q8_0_rows_s(const float *__restrict__ src, uint8_t *__restrict__ dst, uint32_t rowCount,
                            uint32_t srcStride, uint32_t dstRowBase, uint32_t blocksPerRow) {
    quantize_q8_0_rows_impl<false>(src, dst, rowCount, srcStride, dstRowBase, blocksPerRow);
}
