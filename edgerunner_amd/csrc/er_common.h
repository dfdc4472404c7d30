// er_common.h -- device helpers shared by the gfx950 kernels.
//
// Raw GGUF block layouts handled here (byte offsets inside one block):
//   Q8_0  34 B / 32 w : [0,2) d fp16, [2,34) q int8
//   Q4_K 144 B / 256 w: [0,2) d, [2,4) dmin, [4,16) 12 packed 6-bit scales/mins,
//                       [16,144) qs (byte 32*(j/2)+l holds sub-block j, low nibble
//                       for even j, high nibble for odd j)
//   Q6_K 210 B / 256 w: [0,128) ql, [128,192) qh, [192,208) int8 scales, [208,210) d
// Q8_0 and Q6_K blocks are only 2-byte aligned inside a row, so their fields
// are fetched with dword loads from the enclosing 4-byte-aligned window and
// realigned with v_alignbyte_b32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// Same vectors with only dword alignment guaranteed: gfx950 global loads of
// 2/4 dwords need 4-byte alignment only.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

#define ER_DEV static __device__ __forceinline__

ER_DEV float f16_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// s_waitcnt immediate for vmcnt(n), n < 64, with the other counters unconstrained.
constexpr uint16_t vmcnt_imm(int n) { return (uint16_t)((n & 15) | ((n >> 4) << 14) | 0x0070 | 0x0f00); }

// Lane index within the wave, computed afresh from the exec-mask counters
// (no register has to stay live to provide it).
ER_DEV uint32_t lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// A constant materialised in a VGPR that the compiler treats as opaque, so
// that masks reach VOP3 forms from a register instead of being split into
// literal-carrying VOP2 pairs.
ER_DEV uint32_t vreg_const(uint32_t c) {
    uint32_t r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
    return r;
}

// Byte n of a dword, widened exactly (v_cvt_f32_ubyte{0..3}).
ER_DEV float ub0(uint32_t v) { return (float)(v & 0xffu); }
ER_DEV float ub1(uint32_t v) { return (float)((v >> 8) & 0xffu); }
ER_DEV float ub2(uint32_t v) { return (float)((v >> 16) & 0xffu); }
ER_DEV float ub3(uint32_t v) { return (float)(v >> 24); }

ER_DEV float sb(uint32_t v, uint32_t n) { return (float)(int8_t)((v >> (8u * n)) & 0xffu); }

ER_DEV uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t sh) {
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}

ER_DEV u32x4 ld16_a16(const uint8_t *p) { return *(const u32x4 *)p; }
ER_DEV u32x4 ld16_a4(const uint8_t *p) {
    u32x4_a4 v = *(const u32x4_a4 *)p;
    return u32x4{v.x, v.y, v.z, v.w};
}
ER_DEV uint32_t ld4_a4(const uint8_t *p) { return *(const uint32_t *)p; }
ER_DEV uint32_t ld2(const uint8_t *p) { return (uint32_t)(*(const uint16_t *)p); }

// 16 bytes at a 2-byte-aligned address p inside a 4-byte-aligned buffer.
// Reads the window [p & ~3, p + 18) when p % 4 == 2 and exactly [p, p + 16)
// when p % 4 == 0, so callers keep p + 18 inside the buffer for the former.
ER_DEV u32x4 ld16_a2(const uint8_t *p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3u);
    const uint32_t *q = (const uint32_t *)((uintptr_t)p & ~(uintptr_t)3);
    u32x4_a4 v = *(const u32x4_a4 *)q;
    const uint32_t v4 = q[sh ? 4 : 3];
    return u32x4{alignbyte(v.y, v.x, sh), alignbyte(v.z, v.y, sh), alignbyte(v.w, v.z, sh),
                 alignbyte(v4, v.w, sh)};
}

// 8 bytes at a 2-byte-aligned address, same window rule as ld16_a2.
ER_DEV u32x2 ld8_a2(const uint8_t *p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3u);
    const uint32_t *q = (const uint32_t *)((uintptr_t)p & ~(uintptr_t)3);
    u32x2_a4 v = *(const u32x2_a4 *)q;
    const uint32_t v2 = q[sh ? 2 : 1];
    return u32x2{alignbyte(v.y, v.x, sh), alignbyte(v2, v.y, sh)};
}

// 16 / 8 bytes at a 2-byte-aligned address as one vector load (the global
// memory path's unaligned access mode, which the compiler itself relies on
// for under-aligned vector loads).  Reads exactly [p, p + 16) / [p, p + 8).
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32x2_a2 __attribute__((ext_vector_type(2), aligned(2)));
ER_DEV u32x4 ld16_u2(const uint8_t *p) { return *(const u32x4_a2 *)p; }
ER_DEV u32x2 ld8_u2(const uint8_t *p) { return *(const u32x2_a2 *)p; }

// 4 bytes at a 2-byte-aligned address (two 16-bit loads, never over-reads).
ER_DEV uint32_t ld4_a2(const uint8_t *p) { return ld2(p) | (ld2(p + 2) << 16); }

// a . b (4 int8 products) + 0 in one VOP3P v_dot4_i32_i8.  The compiler
// forms every sdot4 as v_dot4c_i32_i8, which accumulates into its destination,
// so each chain started from 0 cost a v_mov of 0 (6 to 12 per slot dot).
ER_DEV int sdot4_0(int a, int b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// sdot4 accumulating into c, or starting a chain (first: c is not read)
ER_DEV int sdot4_acc(int a, int b, int c, bool first) {
    return first ? sdot4_0(a, b) : __builtin_amdgcn_sdot4(a, b, c, false);
}

// DPP lane moves (GFX9 encodings): quad permutations, row (16-lane) mirrors
// and the row broadcasts of lane 15 / lane 31 into the next rows.
#define ER_DPP_QUAD_XOR1 0xb1   // quad_perm [1,0,3,2]
#define ER_DPP_QUAD_XOR2 0x4e   // quad_perm [2,3,0,1]
#define ER_DPP_ROW_MIRROR 0x140
#define ER_DPP_ROW_HALF_MIRROR 0x141
#define ER_DPP_ROW_BCAST15 0x142
#define ER_DPP_ROW_BCAST31 0x143

// v + (v of the lane that `ctrl` selects), on the rows of `rowMask` (other
// rows keep v).
template <int CTRL, int ROWMASK = 0xf>
ER_DEV float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xf, false));
}
template <int CTRL>
ER_DEV float dpp_max(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false)));
}
// dpp_max for v >= 0 that is never NaN (a maximum of magnitudes formed with
// fmaxf): such floats order as their bit patterns, so an unsigned maximum
// gives fmaxf's result in one DPP instruction (no NaN canonicalisation).
template <int CTRL>
ER_DEV float dpp_max_nonneg(float v) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b, CTRL, 0xf, 0xf, false);
    return __uint_as_float(b > o ? b : o);
}

// Sum over the lanes of an aligned group of W lanes (W in {1, 2, 4, 8, 16,
// 32, 64}); every lane of the group gets the sum.  Within a 16-lane row the
// steps are DPP moves fused into the adds (quad swaps, then the half-row and
// row mirrors, which pair each lane with one of the other half); rows are
// joined by the lane-15 / lane-31 broadcasts and the total is read back from
// the group's last lane.
template <int W>
ER_DEV float group_sum(float v) {
    static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
    if constexpr (W >= 2) v = dpp_add<ER_DPP_QUAD_XOR1>(v);
    if constexpr (W >= 4) v = dpp_add<ER_DPP_QUAD_XOR2>(v);
    if constexpr (W >= 8) v = dpp_add<ER_DPP_ROW_HALF_MIRROR>(v);
    if constexpr (W >= 16) v = dpp_add<ER_DPP_ROW_MIRROR>(v);
    if constexpr (W == 32) {
        v = dpp_add<ER_DPP_ROW_BCAST15, 0xa>(v);  // rows 1 and 3 hold the two group sums
        const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
        const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
        v = (threadIdx.x & 32u) ? hi : lo;
    }
    if constexpr (W == 64) {
        v = dpp_add<ER_DPP_ROW_BCAST15, 0xa>(v);
        v = dpp_add<ER_DPP_ROW_BCAST31, 0xc>(v);  // row 3 holds the total
        v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    }
    return v;
}

// Q4_K 6-bit scale/min unpack for the two sub-blocks j = 2p and 2p+1 that
// share qs bytes [32p, 32p+32).  hy, hz, hw are the block's bytes [4,8),
// [8,12), [12,16).  Returns scales in bytes 0/1 of *sc2 and mins in bytes
// 0/1 of *m2 (sub-block 2p in byte 0).
//   j < 4 : sc = s[j] & 63,                  m = s[j+4] & 63
//   j >= 4: sc = (s[j+4] & 15) | (s[j-4]>>6)<<4, m = (s[j+4]>>4) | (s[j]>>6)<<4
ER_DEV void q4k_scales_pair(uint32_t hy, uint32_t hz, uint32_t hw, uint32_t p, uint32_t *sc2,
                            uint32_t *m2) {
    const uint32_t sh = (p & 1u) << 4;
    const uint32_t A = (hy >> sh) & 0xffffu;  // s[q], s[q+1]
    const uint32_t B = (hz >> sh) & 0xffffu;  // s[q+4], s[q+5]
    const uint32_t C = (hw >> sh) & 0xffffu;  // s[q+8], s[q+9]
    const uint32_t scLo = A & 0x3f3fu;
    const uint32_t mLo = B & 0x3f3fu;
    const uint32_t scHi = (C & 0x0f0fu) | ((A >> 2) & 0x3030u);
    const uint32_t mHi = ((C >> 4) & 0x0f0fu) | ((B >> 2) & 0x3030u);
    *sc2 = p < 2 ? scLo : scHi;
    *m2 = p < 2 ? mLo : mHi;
}
