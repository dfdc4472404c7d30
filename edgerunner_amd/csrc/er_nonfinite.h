// er_nonfinite.h -- non-finite activations in the GEMV kernels.
//
// The reference's CPU loops add w[r][k] * x[k] term by term in fp32
// (GEMVTests.swift:61-134, FusedKernelTests.swift:60-83).  When x holds
// non-finite values, a row's sum is decided by the terms at those positions
// alone: a finite partial sum cannot cancel an infinite term, so
//   y[r] = IEEE sum over {k : x[k] not finite} of w[r][k] * x[k]
// which is NaN if any such x[k] is NaN, if a weight at an infinite x[k] is
// zero (0 * inf), or if infinite terms of both signs meet, and otherwise an
// infinity of their common sign.  (Finite terms are assumed not to overflow
// on their own, and weights to be finite.)
//
// The integer-dot kernels cannot carry this through their limb form of x (a
// non-finite value has no limbs), so after its rows are computed each kernel
// checks whether its x held a non-finite value and, only then, replaces every
// row value by the sum above, evaluated from the raw weight bytes with the
// reference's dequantisation.  The check looks at the fp32 chunk sums (a sum
// of 16 values is non-finite exactly when one of them is, or when finite
// values overflow it; the slow path finds the values themselves, so an
// overflow alone changes nothing): the x conversion notes a non-finite chunk
// sum as it forms each one (XlCheck, er_xlimbs.h), so the decision at the end
// of the launch reads one share per wave instead of scanning x again.
#pragma once

#include "er_common.h"

// Weight k of a row as the reference's CPU loops form it (each product below
// is exact in fp32, so only the Q4_K subtraction rounds, as there).
// Q8_0: Float(q) * scale (FusedKernelTests.swift:76-77).
ER_DEV float q8_0_weight_at(const uint8_t *row, uint32_t k) {
    const uint8_t *b = row + (size_t)(k >> 5) * 34u;
    return (float)(int8_t)b[2u + (k & 31u)] * f16_to_f32(ld2(b));
}
// Q4_K: (d * sc) * nibble - dmin * m (GEMVTests.swift:71-94).
ER_DEV float q4k_weight_at(const uint8_t *row, uint32_t k) {
    const uint8_t *b = row + (size_t)(k >> 8) * 144u;
    const uint32_t j = (k >> 5) & 7u, l = k & 31u;
    const uint32_t s = b[4u + (j & 3u)], m = b[8u + (j & 3u)], h = b[12u + (j & 3u)];
    const uint32_t sc = j < 4u ? (s & 63u) : ((h & 15u) | ((s >> 6) << 4));
    const uint32_t mn = j < 4u ? (m & 63u) : ((h >> 4) | ((m >> 6) << 4));
    const uint32_t qb = b[16u + 32u * (j >> 1) + l];
    const uint32_t q = (j & 1u) ? (qb >> 4) : (qb & 15u);
    const float scale = f16_to_f32(ld2(b)) * (float)sc;
    const float minv = f16_to_f32(ld2(b + 2)) * (float)mn;
    return scale * (float)q - minv;
}
// Q6_K: d * sc * (q6 - 32) (GEMVTests.swift:111-130): position 128h + 32m + l
// of a block takes ql[64h + 32(m & 1) + l] (low nibble for m < 2), bits 2m of
// qh[32h + l] and scale sc[8h + l/16 + 2m].
ER_DEV float q6k_weight_at(const uint8_t *row, uint32_t k) {
    const uint8_t *b = row + (size_t)(k >> 8) * 210u;
    const uint32_t p = k & 255u, h = p >> 7, m = (p >> 5) & 3u, l = p & 31u;
    const uint32_t qlb = b[64u * h + 32u * (m & 1u) + l];
    const uint32_t lo = m >= 2u ? (qlb >> 4) : (qlb & 15u);
    const uint32_t hi = (b[128u + 32u * h + l] >> (2u * m)) & 3u;
    const float sc = (float)(int8_t)b[192u + 8u * h + (l >> 4) + 2u * m];
    return f16_to_f32(ld2(b + 208)) * sc * (float)((int)(lo | (hi << 4)) - 32);
}

#define ER_FMT_Q8_0 0
#define ER_FMT_Q4_K 1
#define ER_FMT_Q6_K 2

template <int FMT>
ER_DEV float weight_at(const uint8_t *row, uint32_t k) {
    if constexpr (FMT == ER_FMT_Q8_0) return q8_0_weight_at(row, k);
    else if constexpr (FMT == ER_FMT_Q4_K) return q4k_weight_at(row, k);
    else return q6k_weight_at(row, k);
}

// Wave-uniform: does any of the K values (K % 4 == 0, 16-byte aligned) hold a
// non-finite value?  For kernels that keep no chunk sums.
ER_DEV bool nf_any_value(const float *v, uint32_t K) {
    bool f = false;
#pragma unroll 1
    for (uint32_t i = lane_id(); i < (K >> 2); i += 64u) {
        const float4 q = ((const float4 *)v)[i];
        f |= !(__builtin_isfinite(q.x) && __builtin_isfinite(q.y) && __builtin_isfinite(q.z) &&
               __builtin_isfinite(q.w));
    }
    return __builtin_amdgcn_ballot_w64(f) != 0;
}

// For NR rows: adds to sp[r] the terms weight(r, k) * v(k) of the non-finite
// values v(k) of the 16-value chunks c0, c0 + cs, ... below C16 (only those
// whose sum x16[c] is non-finite when x16 is given), and counts those values
// in hits.  A NaN value's term is NaN whatever the weight, so no weight is
// read for it; the scan ends once every sp[r] is NaN.
// all: every term of those chunks, finite or not (the fp32 evaluation of
// rows whose x the limbs do not carry precisely enough, er_xlimbs.h; with
// non-finite values present its IEEE sum is the one above, since finite
// terms cannot cancel an infinite one).
template <int NR, class WAt, class VAt>
ER_DEV void nf_terms(WAt weight, VAt v, const float *x16, uint32_t C16, uint32_t c0, uint32_t cs,
                     float (&sp)[NR], float &hits, bool all = false) {
#pragma unroll 1
    for (uint32_t c = c0; c < C16; c += cs) {
        if (!all && x16 && __builtin_isfinite(x16[c])) continue;
#pragma unroll 1
        for (uint32_t i = 0; i < 16u; ++i) {
            const uint32_t k = 16u * c + i;
            const float xv = v(k);
            if (!all && __builtin_isfinite(xv)) continue;
            hits += 1.0f;
#pragma unroll
            for (int r = 0; r < NR; ++r) sp[r] += __builtin_isnan(xv) ? xv : weight(r, k) * xv;
        }
        bool done = true;
#pragma unroll
        for (int r = 0; r < NR; ++r) done = done && __builtin_isnan(sp[r]);
        if (done) break;
    }
}
