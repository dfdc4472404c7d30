// er_xlimbs.h -- activation staging for the integer-dot GEMV kernels.
//
// A workgroup converts the fp32 activation vector x[0..K) once into LDS as
// three signed int8 "limbs" per value, so that the weight x activation
// products can be formed with v_dot4_i32_i8 (4 MACs per instruction, exact
// int32 accumulation) instead of per-weight float conversions.
//
// Representation, per 64-value group g (positions [64g, 64g+64)):
//   s_g  = smallest power of two with max|x| / s_g <= 4161407 = 2^23 - C - 1
//          (0 for an all-zero group), C = 64*2^16 + 128*2^8 + 128
//   xi   = rint(x / s_g)                   exact scaling (s_g = 2^e)
//   u    = xi + C                          in [0, 2^23): base-256 digits d0 d1 d2
//   l0   = d0 - 64  in [-64, 63],  l1 = d1 - 128,  l2 = d2 - 128  in [-128, 127]
//   x   ~= s_g * (65536 * l0 + 256 * l1 + l2),   |error| <= s_g / 2 <= max|x_g| / 2^22
// so every activation carries at least 22 significant bits relative to its
// group maximum (fp32-class), and a one-hot x is represented exactly.
// u comes out of one FMA: x * (1/s_g) + (2^23 + C) lies in [2^23, 2^24), where
// the fp32 spacing is 1, so the FMA's single rounding is rint and the low 23
// bits of the result are u; its bytes are the digits (v_perm gathers them).
//
// Conditioning: a group whose maximum dwarfs its other values leaves those
// values few bits (an outlier 10^5 times its neighbours' size leaves them
// about 5), and a row whose weight at the outlier is zero sums exactly those
// neighbours.  Each group's rounding error has energy ~ 64 s_g^2 / 12; the
// launch compares their total with the energy R of the values the limbs
// carry well (per group, the squares in the lanes not holding its maximum):
//   f * sum over groups (64 / 12) s_g^2  >  2^-24 * R
// (f = 1 for Q8_0; 4 for Q4_K and Q6_K, whose unsigned nibbles weigh the
// error against a smaller signed weight), i.e. when the limbs' error would
// exceed ~2^-12 of a row built from the well-carried values, the launch
// evaluates its rows in fp32 from the raw weights instead (the non-finite
// path of er_nonfinite.h with every term).  A few outlier channels of 10^3
// or 10^4 among thousands of ordinary ones stay on the integer path; many
// groups with 10^4 outliers, or any at 10^5, do not.
//
// LDS layout (K a multiple of 64):
//   [0, 3K)        planes 0..2: limb bytes l0, l1, l2; 16-byte granules swizzled by xl_gswz
//   [3K, 3K+K/4)   x16[K/16]  fp32 sums of each 16-value chunk (exact fp32 x),
//                  summed as (x0 + .. + x7) + (x8 + .. + x15), each half in order
//   then           sg64[K/64] the group scales s_g
//   then           rest64[K/64] each group's energy outside its maximum's lanes (xl_rest_energy)
#pragma once

#include "er_common.h"

#define ER_XL_QMAX 4161407.0f
#define ER_XL_MAGIC 12615808.0f  // 2^23 + C, C = 4227200
#define ER_XL_PLANES 3

// 16-byte granule swizzle: the 8 lanes that one ds_read_b128 cycle serves read
// granules 4s+m (s = 8 consecutive slots, m fixed); XOR-ing bits 3-4 into bits
// 0-1 spreads them over all 8 four-bank groups.
ER_DEV uint32_t xl_gswz(uint32_t G) { return G ^ ((G >> 3) & 3u); }

ER_DEV uint32_t xl_lds_bytes(uint32_t K) { return ER_XL_PLANES * K + (K / 16u) * 4u + (K / 64u) * 8u; }

// 2^-24: the launch takes the fp32 path when its limbs' error energy exceeds
// this fraction of the energy they carry well (xl_ill_rule)
#define ER_XL_EPS2 5.9604645e-08f

struct XLimbs {
    const uint8_t *planes;
    const float *x16;
    const float *sg64;
    const float *rest64;
    uint32_t K;
};

ER_DEV XLimbs xl_view(const uint32_t *lds, uint32_t K) {
    XLimbs v;
    v.planes = (const uint8_t *)lds;
    v.x16 = (const float *)(lds + (ER_XL_PLANES * K) / 4u);
    v.sg64 = v.x16 + (K >> 4);
    v.rest64 = v.sg64 + (K >> 6);
    v.K = K;
    return v;
}

// The conditioning rule on its two sums: e adds s_g^2 over the groups that
// carry energy outside their maximum's lanes, r adds that energy.
ER_DEV bool xl_ill_rule(float e, float r, float f) { return f * (64.0f / 12.0f) * e > ER_XL_EPS2 * r; }

// The launch's end-of-launch checks, gathered while x is converted: each lane
// adds, over the chunks it converts, the conditioning sums of xl_ill_rule
// (e: s_g^2 of each group with energy outside its maximum's lanes, r: that
// energy; a group counts once, at its first chunk) and whether a chunk sum is
// non-finite.  xl_check_share reduces a wave's lanes; xl_check_decide adds the
// waves' shares in wave order.  Every workgroup of a launch converts the same
// chunks in the same lanes, so all reach the same decisions.
struct XlCheck {
    float e = 0.0f, r = 0.0f;
    bool nf = false;
};

// Wave-uniform: this wave's share {e, r, 1 if a chunk sum was non-finite, 0}.
ER_DEV float4 xl_check_share(const XlCheck &c) {
    return float4{group_sum<64>(c.e), group_sum<64>(c.r), __builtin_amdgcn_ballot_w64(c.nf) != 0 ? 1.0f : 0.0f,
                  0.0f};
}

// The decisions from n wave shares (f: the format's factor of xl_ill_rule):
// ill -- the fp32 path for every row; nf -- the non-finite path (only when
// not ill).
ER_DEV void xl_check_decide(const float4 *share, int n, float f, bool &ill, bool &nf) {
    float e = 0.0f, r = 0.0f, bad = 0.0f;
    for (int w = 0; w < n; ++w) {
        const float4 c = share[w];
        e += c.x;
        r += c.y;
        bad += c.z;
    }
    ill = xl_ill_rule(e, r, f);
    nf = !ill && bad > 0.0f;
}

// The group's energy outside its maximum's lanes, from this lane's values
// v[0..N), this lane's maximum lmx and the group maximum mx: each lane sums
// its squares (one FMA per value), the lane(s) holding mx contribute nothing,
// and the group sums over its lanes with the DPP steps `reduce` applies, so
// 48 (or 56) of the 63 other values count.  Leaving a whole lane out, rather
// than subtracting max^2 from a sum holding it, keeps the value free of
// cancellation (the square of the maximum has an ulp far above it).  0 for
// an all-zero or non-finite group; squares past ~1.8e19 overflow to infinity,
// which keeps the launch on the integer path (its error is then negligible).
template <int N, class Reduce>
ER_DEV float xl_rest_energy(const float (&v)[N], float lmx, float mx, Reduce reduce) {
    float s2 = 0.0f;
#pragma unroll
    for (int q = 0; q < N; ++q) s2 = __builtin_fmaf(v[q], v[q], s2);
    const float rest = reduce(lmx == mx ? 0.0f : s2);
    return mx > 0.0f && mx < __builtin_inff() ? rest : 0.0f;
}

// Sums over the 4 lanes (16-value chunks) or 8 lanes (8-value halves) that
// hold one 64-group.
ER_DEV float xl_group_sum4(float r) {
    r = dpp_add<ER_DPP_QUAD_XOR1>(r);
    return dpp_add<ER_DPP_QUAD_XOR2>(r);
}
ER_DEV float xl_group_sum8(float r) {
    r = dpp_add<ER_DPP_QUAD_XOR1>(r);
    r = dpp_add<ER_DPP_QUAD_XOR2>(r);
    return dpp_add<ER_DPP_ROW_HALF_MIRROR>(r);  // quads 2k and 2k+1 of each 8 lanes
}


// Loads of chunk c (16 values) of x for thread `tid`; XG chunks per thread.
// Out-of-range chunks reload the last chunk (always in bounds, never stored).
template <int XG, int NT>
ER_DEV void xl_load(const float *__restrict__ x, uint32_t K, float4 (&xr)[XG][4]) {
    const uint32_t C16 = K >> 4;
#pragma unroll
    for (int c = 0; c < XG; ++c) {
        const uint32_t t = min(threadIdx.x + (uint32_t)NT * c, C16 - 1u);
#pragma unroll
        for (int q = 0; q < 4; ++q) xr[c][q] = ((const float4 *)(x + 16u * t))[q];
    }
}

// Power-of-two group scale for a group maximum mx >= 0: the smallest 2^e with
// mx / 2^e <= ER_XL_QMAX (0 when mx == 0); inv = 1 / scale exactly.  A group
// holding an infinity (mx = inf) gets scale 0 like an all-zero one: its limbs
// carry nothing, and the kernels evaluate non-finite activations apart
// (er_nonfinite.h).
ER_DEV void xl_scale(float mx, float *sg, float *inv) {
    const float v = mx * (1.0f / ER_XL_QMAX);
    uint32_t b = __float_as_uint(v);
    b = (b + 0x007fffffu) & 0xff800000u;  // round up to a power of two (v >= 0)
    if (mx > 0.0f && b == 0u) b = 0x00800000u;  // keep the scale normal
    const bool live = mx > 0.0f && mx < __builtin_inff();
    *sg = live ? __uint_as_float(b) : 0.0f;
    // 1/2^e = 2^-e: exponent field 254 - e_field (exact for normal scales)
    *inv = live ? __uint_as_float((254u - (b >> 23)) << 23) : 0.0f;
}

// Converts one 16-value chunk (index tRaw, values in xr) into LDS.  The 4
// chunks of a 64-group are held by 4 consecutive lanes, which exchange their
// maxima; every lane of the wave must call this together.
ER_DEV void xl_store_chunk(uint32_t *lds, uint32_t K, const float4 (&xr)[4], uint32_t tRaw, XlCheck *ck = nullptr) {
    const uint32_t C16 = K >> 4;
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        v[4 * q + 0] = xr[q].x;
        v[4 * q + 1] = xr[q].y;
        v[4 * q + 2] = xr[q].z;
        v[4 * q + 3] = xr[q].w;
    }
    float mx = 0.0f, sa = 0.0f, sb = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        mx = fmaxf(mx, fabsf(v[q]));
        sa += v[q];
    }
#pragma unroll
    for (int q = 8; q < 16; ++q) {
        mx = fmaxf(mx, fabsf(v[q]));
        sb += v[q];
    }
    const float sm = sa + sb;
    const float lmx = mx;
    mx = dpp_max_nonneg<ER_DPP_QUAD_XOR1>(mx);
    mx = dpp_max_nonneg<ER_DPP_QUAD_XOR2>(mx);
    float sg, inv;
    xl_scale(mx, &sg, &inv);
    const float rest = xl_rest_energy(v, lmx, mx, xl_group_sum4);
    // digits of u = xi + C are bytes 0..2 of fma(v, 1/s_g, 2^23 + C)
    uint32_t u[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) u[q] = __float_as_uint(__builtin_fmaf(v[q], inv, ER_XL_MAGIC));
    uint32_t lb[ER_XL_PLANES][4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t a = u[4 * d], b = u[4 * d + 1], c = u[4 * d + 2], e = u[4 * d + 3];
        // byte k of the result = byte `sel` of values a, b, c, e
        const uint32_t d0 = __builtin_amdgcn_perm(__builtin_amdgcn_perm(e, c, 0x0c0c0602u),
                                                  __builtin_amdgcn_perm(b, a, 0x0c0c0602u), 0x05040100u);
        const uint32_t d1 = __builtin_amdgcn_perm(__builtin_amdgcn_perm(e, c, 0x0c0c0501u),
                                                  __builtin_amdgcn_perm(b, a, 0x0c0c0501u), 0x05040100u);
        const uint32_t d2 = __builtin_amdgcn_perm(__builtin_amdgcn_perm(e, c, 0x0c0c0400u),
                                                  __builtin_amdgcn_perm(b, a, 0x0c0c0400u), 0x05040100u);
        // d - 128 as int8 is d ^ 0x80; d0 - 64 (d0 < 128) is d0 ^ 0x40 with bit 7
        // set where bit 6 of d0 ^ 0x40 is set (sign extension of a 7-bit value)
        const uint32_t t = d0 ^ 0x40404040u;
        lb[0][d] = t ^ ((t & 0x40404040u) << 1);
        lb[1][d] = d1 ^ 0x80808080u;
        lb[2][d] = d2 ^ 0x80808080u;
    }
    if (ck) {
        const bool st = tRaw < C16, first = st && (tRaw & 3u) == 0;
        ck->e = __builtin_fmaf(first && rest > 0.0f ? sg : 0.0f, sg, ck->e);
        ck->r += first ? rest : 0.0f;
        ck->nf |= st && !__builtin_isfinite(sm);
    }
    // chunks past the end are clamped copies with a different group max: never stored
    if (tRaw < C16) {
        uint8_t *planes = (uint8_t *)lds;
        float *x16 = (float *)(lds + (ER_XL_PLANES * K) / 4u);
        float *sg64 = x16 + C16;
        const uint32_t G = xl_gswz(tRaw);
#pragma unroll
        for (int l = 0; l < ER_XL_PLANES; ++l)
            *(u32x4 *)__builtin_assume_aligned(planes + (size_t)l * K + 16u * G, 16) =
                u32x4{lb[l][0], lb[l][1], lb[l][2], lb[l][3]};
        x16[tRaw] = sm;
        if ((tRaw & 3u) == 0) {
            sg64[tRaw >> 2] = sg;
            sg64[C16 / 4u + (tRaw >> 2)] = rest;
        }
    }
}

// Converts one 8-value half-chunk (index hRaw: values 8 hRaw .. 8 hRaw + 7,
// in xr) into LDS, giving the same bytes, chunk sums and scales as
// xl_store_chunk.  The 8 half-chunks of a 64-group are held by 8 consecutive
// lanes, which exchange their maxima (and pairs their half sums); every lane
// of the wave must call this together.
ER_DEV void xl_store_half(uint32_t *lds, uint32_t K, const float4 (&xr)[2], uint32_t hRaw, XlCheck *ck = nullptr) {
    const uint32_t C8 = K >> 3;
    const float v[8] = {xr[0].x, xr[0].y, xr[0].z, xr[0].w, xr[1].x, xr[1].y, xr[1].z, xr[1].w};
    float mx = 0.0f, sh = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        mx = fmaxf(mx, fabsf(v[q]));
        sh += v[q];
    }
    const float sm = dpp_add<ER_DPP_QUAD_XOR1>(sh);  // even lane: own half + the odd lane's
    const float lmx = mx;
    mx = dpp_max_nonneg<ER_DPP_QUAD_XOR1>(mx);
    mx = dpp_max_nonneg<ER_DPP_QUAD_XOR2>(mx);
    mx = dpp_max_nonneg<ER_DPP_ROW_HALF_MIRROR>(mx);  // quads 2k and 2k+1 of each 8 lanes
    float sg, inv;
    xl_scale(mx, &sg, &inv);
    const float rest = xl_rest_energy(v, lmx, mx, xl_group_sum8);
    uint32_t u[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) u[q] = __float_as_uint(__builtin_fmaf(v[q], inv, ER_XL_MAGIC));
    uint32_t lb[ER_XL_PLANES][2];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const uint32_t a = u[4 * d], b = u[4 * d + 1], c = u[4 * d + 2], e = u[4 * d + 3];
        const uint32_t d0 = __builtin_amdgcn_perm(__builtin_amdgcn_perm(e, c, 0x0c0c0602u),
                                                  __builtin_amdgcn_perm(b, a, 0x0c0c0602u), 0x05040100u);
        const uint32_t d1 = __builtin_amdgcn_perm(__builtin_amdgcn_perm(e, c, 0x0c0c0501u),
                                                  __builtin_amdgcn_perm(b, a, 0x0c0c0501u), 0x05040100u);
        const uint32_t d2 = __builtin_amdgcn_perm(__builtin_amdgcn_perm(e, c, 0x0c0c0400u),
                                                  __builtin_amdgcn_perm(b, a, 0x0c0c0400u), 0x05040100u);
        const uint32_t t = d0 ^ 0x40404040u;
        lb[0][d] = t ^ ((t & 0x40404040u) << 1);
        lb[1][d] = d1 ^ 0x80808080u;
        lb[2][d] = d2 ^ 0x80808080u;
    }
    if (ck) {
        const bool st = hRaw < C8, first = st && (hRaw & 7u) == 0;
        ck->e = __builtin_fmaf(first && rest > 0.0f ? sg : 0.0f, sg, ck->e);
        ck->r += first ? rest : 0.0f;
        ck->nf |= st && (hRaw & 1u) == 0 && !__builtin_isfinite(sm);
    }
    if (hRaw < C8) {
        uint8_t *planes = (uint8_t *)lds;
        float *x16 = (float *)(lds + (ER_XL_PLANES * K) / 4u);
        float *sg64 = x16 + (K >> 4);
        const uint32_t off = 16u * xl_gswz(hRaw >> 1) + 8u * (hRaw & 1u);
#pragma unroll
        for (int l = 0; l < ER_XL_PLANES; ++l)
            *(u32x2 *)__builtin_assume_aligned(planes + (size_t)l * K + off, 8) = u32x2{lb[l][0], lb[l][1]};
        if ((hRaw & 1u) == 0) x16[hRaw >> 1] = sm;
        if ((hRaw & 7u) == 0) {
            sg64[hRaw >> 3] = sg;
            sg64[(K >> 6) + (hRaw >> 3)] = rest;
        }
    }
}

// Stores the XG register-held chunks of this thread.
template <int XG, int NT>
ER_DEV void xl_store(uint32_t *lds, uint32_t K, const float4 (&xr)[XG][4], XlCheck *ck = nullptr) {
#pragma unroll
    for (int c = 0; c < XG; ++c) xl_store_chunk(lds, K, xr[c], threadIdx.x + (uint32_t)NT * c, ck);
}

// Chunks with index >= XG*NT (K beyond the register-staged part): loaded and
// stored after the weight loads are in flight.
template <int XG, int NT>
ER_DEV void xl_store_tail(const float *__restrict__ x, uint32_t *lds, uint32_t K, XlCheck *ck = nullptr) {
    const uint32_t C16 = K >> 4;
    for (uint32_t base = (uint32_t)NT * XG; base < C16; base += NT) {
        float4 xr[4];
        const uint32_t t = min(base + threadIdx.x, C16 - 1u);
#pragma unroll
        for (int q = 0; q < 4; ++q) xr[q] = ((const float4 *)(x + 16u * t))[q];
        xl_store_chunk(lds, K, xr, base + threadIdx.x, ck);
    }
}

// The 4 granules (64 positions) of 64-group `grp` from every plane.
ER_DEV void xl_read_group(const XLimbs &X, uint32_t grp, u32x4 (&xv)[ER_XL_PLANES][4]) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t off = 16u * xl_gswz(4u * grp + (uint32_t)m);
#pragma unroll
        for (int l = 0; l < ER_XL_PLANES; ++l)
            xv[l][m] = *(const u32x4 *)__builtin_assume_aligned(X.planes + (size_t)l * X.K + off, 16);
    }
}

// Limb partial sums (each an exact int32 dot product) recombined into the
// value of sum(q * xi): c0 * 2^16 + c1 * 2^8 + c2.  c1 * 2^8 + c2 is exact in
// int32 for every slot size used (|c1| <= 64 * 128 * 128); the result is
// rounded to fp32 twice at most.
ER_DEV float xl_combine(int c0, int c1, int c2) {
    return __builtin_fmaf((float)c0, 65536.0f, (float)((c1 << 8) + c2));
}
