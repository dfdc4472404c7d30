/*
 * er_oracle.c -- CPU oracle for the quantized-matmul path (TEST INFRASTRUCTURE).
 *
 * This file is a plain-C restatement of EdgeRunner's own Swift CPU reference
 * for GGUF Q8_0 / Q4_K / Q6_K dequantisation and dequant+dot GEMV.  It is the
 * checker that the HIP kernels are compared against.  Only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load it;
 * the product library (edgerunner_amd) never links or calls it.
 *
 * Build: `make -C oracle` (gcc -O2 -ffp-contract=off, no fast-math) so that
 * every fp32 operation rounds exactly where the Swift source rounds.
 *
 * Paths in citations are relative to the EdgeRunner source tree.
 *
 * Pinning (what checks each function, see tests/test_oracle_*.py):
 *   - dequant_*: hand-derived known answers on the reference's formula
 *     fillers, an independent numpy statement (bit-exact), single-bit brute
 *     force, pack->dequant round trips, zero blocks.
 *   - gemv_*: float64 accumulation of independently dequantised weights,
 *     one-hot x extracts a column exactly, linearity, batched == per token.
 *   - quantize_q8_0_rows: closed-form checks (max |v| maps to +-127, rint
 *     ties-to-even, zero rows) and round-trip error bound.
 *   - argmax: brute force with lowest-index ties.
 *   - rmsnorm: unit RMS of the output for w = 1, scale invariance, a
 *     constant vector's closed form; silu: silu(0) = 0, silu(v) - silu(-v) = v,
 *     the sigmoid limits.
 *   - top1: equals argmax on finite values (brute force); hand-derived
 *     answers for NaN candidates and all -inf inputs.
 *   - xoshiro256** / splitmix64: published reference outputs.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define Q8_0_BYTES 34
#define Q4_K_BYTES 144
#define Q6_K_BYTES 210

/* ------------------------------------------------------------------------ */
/* IEEE binary16 <-> binary32                                                */
/* ------------------------------------------------------------------------ */

/* Exact widening, as Swift's Float(Float16(bitPattern:)) used by readF16
 * (Tests/EdgeRunnerMetalTests/GEMVTests.swift:56-59). */
float er_ref_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t expo = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (expo == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: mant * 2^-24, exact in binary32 */
            float v = (float)mant * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (expo == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((expo + 112u) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* Round-to-nearest-even narrowing, as Swift's Float16(Float) used by the
 * reference's block packers (e.g. DequantQ4KMTests.swift:34-35). */
uint16_t er_ref_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) {                       /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
    }
    if (absx >= 0x477ff000u) {                       /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (absx < 0x38800000u) {                        /* result subnormal or zero */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 -> +-0 */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7fffffu) | 0x800000u;
        /* value = m * 2^(e-150); in units of 2^-24 that is m >> (126-e) */
        uint32_t shift = 126u - e;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112u;
    uint32_t m = absx & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

/* bfloat16 -> float (exact). */
float er_ref_bf16_to_f32(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* float -> bfloat16, round to nearest even (NaN kept quiet). */
uint16_t er_ref_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

static inline float rd16(const uint8_t *p) {
    return er_ref_f16_to_f32((uint16_t)(p[0] | ((uint16_t)p[1] << 8)));
}

/* ------------------------------------------------------------------------ */
/* Dequantisation (one block -> fp32)                                        */
/* ------------------------------------------------------------------------ */

/* Q8_0: Tests/EdgeRunnerIOTests/DequantQ8_0Tests.swift:25-34
 * (w[i] = scale * Float(Int8(q[i])); same as Dequant_Q8_0.metal:57-63). */
void er_ref_dequant_q8_0(const uint8_t *blocks, uint64_t nblocks, float *out) {
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = blocks + b * Q8_0_BYTES;
        float scale = rd16(blk);
        for (int i = 0; i < 32; ++i) {
            out[b * 32 + i] = scale * (float)(int8_t)blk[2 + i];
        }
    }
}

/* Q4_K: Tests/EdgeRunnerIOTests/DequantQ4KMTests.swift:84-119
 * (scales/mins unpack :92-101, value (scale*nibble) - min :103-116;
 *  cross-checked with Dequant_Q4_K_M.metal:38-67 and
 *  LlamaLanguageModel.swift:5475-5510). */
void er_ref_dequant_q4_k(const uint8_t *blocks, uint64_t nblocks, float *out) {
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = blocks + b * Q4_K_BYTES;
        float d = rd16(blk);
        float dmin = rd16(blk + 2);
        uint8_t scales[8], mins[8];
        for (int sb = 0; sb < 4; ++sb) {
            scales[sb] = blk[4 + sb] & 0x3f;
            scales[sb + 4] = (uint8_t)((blk[12 + sb] & 0x0f) | ((blk[4 + sb] >> 6) << 4));
            mins[sb] = blk[8 + sb] & 0x3f;
            mins[sb + 4] = (uint8_t)(((blk[12 + sb] >> 4) & 0x0f) | ((blk[8 + sb] >> 6) << 4));
        }
        for (int sb = 0; sb < 8; ++sb) {
            float scale = d * (float)scales[sb];
            float minv = dmin * (float)mins[sb];
            for (int i = 0; i < 32; ++i) {
                uint8_t byte = blk[16 + (sb / 2) * 32 + i];
                uint8_t nib = (sb % 2 == 0) ? (byte & 0x0f) : ((byte >> 4) & 0x0f);
                out[b * 256 + sb * 32 + i] = (scale * (float)nib) - minv;
            }
        }
    }
}

/* Q6_K: Tests/EdgeRunnerIOTests/DequantQ6KTests.swift:80-113
 * (half-block / lane walk, w = d * Float(scale) * Float(q); cross-checked with
 *  Dequant_Q6_K.metal:20-35 and LlamaLanguageModel.swift:5536-5565). */
void er_ref_dequant_q6_k(const uint8_t *blocks, uint64_t nblocks, float *out) {
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t *blk = blocks + b * Q6_K_BYTES;
        float d = rd16(blk + 208);
        const int8_t *sc = (const int8_t *)(blk + 192);
        float *o = out + b * 256;
        for (int h = 0; h < 2; ++h) {
            const uint8_t *ql = blk + h * 64;
            const uint8_t *qh = blk + 128 + h * 32;
            const int8_t *s = sc + h * 8;
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[32 + l] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[32 + l] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                o[h * 128 + l] = d * (float)s[is + 0] * (float)q1;
                o[h * 128 + 32 + l] = d * (float)s[is + 2] * (float)q2;
                o[h * 128 + 64 + l] = d * (float)s[is + 4] * (float)q3;
                o[h * 128 + 96 + l] = d * (float)s[is + 6] * (float)q4;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GEMV, reference loop and fp32 operation order.  y[M] = W[M,K] . x[K]      */
/* ------------------------------------------------------------------------ */

/* Q8_0 row: Tests/EdgeRunnerMetalTests/FusedKernelTests.swift:60-83
 * (sum += Float(quant) * scale * x[block*32+i]). */
static float gemv_q8_0_row(const uint8_t *row, const float *x, int K) {
    int nb = K / 32;
    float sum = 0.0f;
    for (int blk = 0; blk < nb; ++blk) {
        const uint8_t *p = row + (size_t)blk * Q8_0_BYTES;
        float scale = rd16(p);
        for (int i = 0; i < 32; ++i) {
            float q = (float)(int8_t)p[2 + i];
            sum += q * scale * x[blk * 32 + i];
        }
    }
    return sum;
}

/* Q4_K row: Tests/EdgeRunnerMetalTests/GEMVTests.swift:61-97
 * (sub-block major; sum += (scale * nibble - minValue) * x[col]). */
static float gemv_q4_k_row(const uint8_t *row, const float *x, int K) {
    int nb = K / 256;
    float sum = 0.0f;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t *blk = row + (size_t)bi * Q4_K_BYTES;
        float d = rd16(blk);
        float dmin = rd16(blk + 2);
        for (int sb = 0; sb < 8; ++sb) {
            uint8_t scaleByte = blk[4 + (sb & 3)];
            uint8_t minByte = blk[8 + (sb & 3)];
            uint8_t highBits = blk[12 + (sb & 3)];
            float scale, minv;
            if (sb < 4) {
                scale = d * (float)(scaleByte & 0x3f);
                minv = dmin * (float)(minByte & 0x3f);
            } else {
                scale = d * (float)((highBits & 0x0f) | (((scaleByte >> 6) & 3) << 4));
                minv = dmin * (float)(((highBits >> 4) & 0x0f) | (((minByte >> 6) & 3) << 4));
            }
            for (int i = 0; i < 32; ++i) {
                uint8_t packed = blk[16 + (sb / 2) * 32 + i];
                uint8_t nib = (sb % 2 == 0) ? (packed & 0x0f) : ((packed >> 4) & 0x0f);
                int col = bi * 256 + sb * 32 + i;
                sum += (scale * (float)nib - minv) * x[col];
            }
        }
    }
    return sum;
}

/* Q6_K row: Tests/EdgeRunnerMetalTests/GEMVTests.swift:99-134
 * (half -> lane -> q1..q4; sum += d * Float(s) * Float(q) * x). */
static float gemv_q6_k_row(const uint8_t *row, const float *x, int K) {
    int nb = K / 256;
    float sum = 0.0f;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t *blk = row + (size_t)bi * Q6_K_BYTES;
        float d = rd16(blk + 208);
        for (int h = 0; h < 2; ++h) {
            int outBase = h * 128;
            const uint8_t *ql = blk + h * 64;
            const uint8_t *qh = blk + 128 + h * 32;
            const uint8_t *sc = blk + 192 + h * 8;
            for (int l = 0; l < 32; ++l) {
                int so = l / 16;
                int q1 = (int)((ql[l] & 0x0f) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[32 + l] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[32 + l] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                float s1 = (float)(int8_t)sc[so + 0];
                float s2 = (float)(int8_t)sc[so + 2];
                float s3 = (float)(int8_t)sc[so + 4];
                float s4 = (float)(int8_t)sc[so + 6];
                const float *xb = x + bi * 256 + outBase;
                sum += d * s1 * (float)q1 * xb[l];
                sum += d * s2 * (float)q2 * xb[32 + l];
                sum += d * s3 * (float)q3 * xb[64 + l];
                sum += d * s4 * (float)q4 * xb[96 + l];
            }
        }
    }
    return sum;
}

typedef float (*row_fn)(const uint8_t *, const float *, int);

static void gemv_rows(row_fn fn, size_t rowBytes, const uint8_t *W, const float *x, float *y,
                      int M, int K, int threads) {
#ifdef _OPENMP
    if (threads > 1) {
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int r = 0; r < M; ++r) y[r] = fn(W + (size_t)r * rowBytes, x, K);
        return;
    }
#else
    (void)threads;
#endif
    for (int r = 0; r < M; ++r) y[r] = fn(W + (size_t)r * rowBytes, x, K);
}

/* Batched GEMV: token t uses x[t*K..] and writes y[t*M..]; the reference's
 * batched kernels are defined as the per-token GEMV
 * (GEMVTests.swift:480-514, Dequant_Q8_0.metal:143-197). */
void er_ref_gemv_q8_0(const uint8_t *W, const float *x, float *y, int M, int K, int tokens,
                      int threads) {
    size_t rb = (size_t)(K / 32) * Q8_0_BYTES;
    for (int t = 0; t < tokens; ++t)
        gemv_rows(gemv_q8_0_row, rb, W, x + (size_t)t * K, y + (size_t)t * M, M, K, threads);
}

void er_ref_gemv_q4_k(const uint8_t *W, const float *x, float *y, int M, int K, int tokens,
                      int threads) {
    size_t rb = (size_t)(K / 256) * Q4_K_BYTES;
    for (int t = 0; t < tokens; ++t)
        gemv_rows(gemv_q4_k_row, rb, W, x + (size_t)t * K, y + (size_t)t * M, M, K, threads);
}

void er_ref_gemv_q6_k(const uint8_t *W, const float *x, float *y, int M, int K, int tokens,
                      int threads) {
    size_t rb = (size_t)(K / 256) * Q6_K_BYTES;
    for (int t = 0; t < tokens; ++t)
        gemv_rows(gemv_q6_k_row, rb, W, x + (size_t)t * K, y + (size_t)t * M, M, K, threads);
}

/* Prefill GEMM oracle: Y[t][n] = sum_k W[n][k] * X[t][k] with X given in
 * bfloat16.  The reference has no quantised GEMM; its prefill is the
 * token-batched GEMV (LlamaLanguageModel.swift:2515-2535, 2552-2617), so the
 * oracle is the per-token GEMV above applied to X widened to fp32. */
int er_ref_gemm(int fmt, const uint8_t *W, const uint16_t *Xbf16, float *Y, int T, int N, int K,
                int threads) {
    float *xf = (float *)malloc((size_t)T * K * sizeof(float));
    if (!xf) return -1;
    for (size_t i = 0; i < (size_t)T * K; ++i) xf[i] = er_ref_bf16_to_f32(Xbf16[i]);
    if (fmt == 8) er_ref_gemv_q8_0(W, xf, Y, N, K, T, threads);
    else if (fmt == 12) er_ref_gemv_q4_k(W, xf, Y, N, K, T, threads);
    else if (fmt == 14) er_ref_gemv_q6_k(W, xf, Y, N, K, T, threads);
    free(xf);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Q8_0 row quantiser: Sources/EdgeRunnerMetal/Shaders/Dequant_Q8_0.metal:19-49
 * (scale = maxAbs/127 stored as fp16; q = clamp(rint(v/scale), -127, 127),
 *  where the division uses the fp32 scale, not the fp16-rounded one). */
void er_ref_quantize_q8_0_rows(const float *src, uint8_t *dst, uint32_t rowCount,
                               uint32_t srcRowStride, uint32_t dstRowBase, uint32_t blocksPerRow) {
    for (uint32_t r = 0; r < rowCount; ++r) {
        const float *srow = src + (size_t)r * srcRowStride;
        uint8_t *drow = dst + (size_t)(dstRowBase + r) * blocksPerRow * Q8_0_BYTES;
        for (uint32_t b = 0; b < blocksPerRow; ++b) {
            const float *v = srow + b * 32;
            uint8_t *o = drow + (size_t)b * Q8_0_BYTES;
            float maxAbs = 0.0f;
            for (int i = 0; i < 32; ++i) maxAbs = fmaxf(maxAbs, fabsf(v[i]));
            float scale = maxAbs > 0.0f ? maxAbs / 127.0f : 0.0f;
            uint16_t h = er_ref_f32_to_f16(scale);
            o[0] = (uint8_t)(h & 0xff);
            o[1] = (uint8_t)(h >> 8);
            for (int i = 0; i < 32; ++i) {
                int q = 0;
                if (scale != 0.0f) {
                    float r0 = rintf(v[i] / scale);
                    q = (int)r0;
                    if (q < -127) q = -127;
                    if (q > 127) q = 127;
                }
                o[2 + i] = (uint8_t)(int8_t)q;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Block packers used by the reference's tests to build fixtures.            */
/* Swift's round() is ties-away-from-zero == C roundf().                      */
/* ------------------------------------------------------------------------ */

/* DequantQ8_0Tests.swift:5-23 (clamp to [-128,127]). */
void er_ref_pack_q8_0_block(const float *v, uint8_t *out) {
    float absMax = 0.0f;
    for (int i = 0; i < 32; ++i) absMax = fmaxf(absMax, fabsf(v[i]));
    float scale = absMax == 0.0f ? 0.0f : absMax / 127.0f;
    uint16_t h = er_ref_f32_to_f16(scale);
    out[0] = (uint8_t)(h & 0xff);
    out[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; ++i) {
        int q = 0;
        if (scale != 0.0f) {
            q = (int)roundf(v[i] / scale);
            if (q < -128) q = -128;
            if (q > 127) q = 127;
        }
        out[2 + i] = (uint8_t)(int8_t)q;
    }
}

/* DequantQ4KMTests.swift:8-82. */
void er_ref_pack_q4_k_block(const float *values, uint8_t *block) {
    float subScales[8], subMins[8];
    memset(block, 0, Q4_K_BYTES);
    for (int sb = 0; sb < 8; ++sb) {
        const float *sv = values + sb * 32;
        float mx = sv[0], mn = sv[0];
        for (int i = 1; i < 32; ++i) {
            mx = fmaxf(mx, sv[i]);
            mn = fminf(mn, sv[i]);
        }
        subScales[sb] = (mx - mn > 0.0f) ? (mx - mn) / 15.0f : 0.0f;
        subMins[sb] = fmaxf(0.0f, -mn);
    }
    float maxScale = subScales[0], maxMin = subMins[0];
    for (int sb = 1; sb < 8; ++sb) {
        maxScale = fmaxf(maxScale, subScales[sb]);
        maxMin = fmaxf(maxMin, subMins[sb]);
    }
    float d = maxScale > 0.0f ? maxScale / 63.0f : 0.0f;
    float dmin = maxMin > 0.0f ? maxMin / 63.0f : 0.0f;
    uint16_t dBits = er_ref_f32_to_f16(d), dminBits = er_ref_f32_to_f16(dmin);
    block[0] = (uint8_t)(dBits & 0xff);
    block[1] = (uint8_t)(dBits >> 8);
    block[2] = (uint8_t)(dminBits & 0xff);
    block[3] = (uint8_t)(dminBits >> 8);
    uint8_t qs[8], qm[8];
    for (int sb = 0; sb < 8; ++sb) {
        qs[sb] = d > 0.0f ? (uint8_t)fminf(63.0f, roundf(subScales[sb] / d)) : 0;
        qm[sb] = dmin > 0.0f ? (uint8_t)fminf(63.0f, roundf(subMins[sb] / dmin)) : 0;
    }
    for (int sb = 0; sb < 4; ++sb) {
        block[4 + sb] = (uint8_t)((qs[sb] & 0x3f) | (((qs[sb + 4] >> 4) & 3) << 6));
        block[8 + sb] = (uint8_t)((qm[sb] & 0x3f) | (((qm[sb + 4] >> 4) & 3) << 6));
        block[12 + sb] = (uint8_t)((qs[sb + 4] & 0x0f) | ((qm[sb + 4] & 0x0f) << 4));
    }
    float dF = er_ref_f16_to_f32(dBits), dminF = er_ref_f16_to_f32(dminBits);
    for (int sb = 0; sb < 8; ++sb) {
        float scale = dF * (float)qs[sb];
        float minv = dminF * (float)qm[sb];
        for (int i = 0; i < 32; ++i) {
            int q = 0;
            if (scale > 0.0f) {
                q = (int)roundf((values[sb * 32 + i] + minv) / scale);
                if (q < 0) q = 0;
                if (q > 15) q = 15;
            }
            int bi = 16 + (sb / 2) * 32 + i;
            if (sb % 2 == 0) block[bi] = (uint8_t)((block[bi] & 0xf0) | (q & 0x0f));
            else block[bi] = (uint8_t)((block[bi] & 0x0f) | ((q & 0x0f) << 4));
        }
    }
}

/* DequantQ6KTests.swift:8-78. */
void er_ref_pack_q6_k_block(const float *values, uint8_t *block) {
    memset(block, 0, Q6_K_BYTES);
    float absMax = 0.0f;
    for (int i = 0; i < 256; ++i) absMax = fmaxf(absMax, fabsf(values[i]));
    float d = absMax > 0.0f ? absMax / (63.0f * 31.0f) : 0.0f;
    uint16_t dBits = er_ref_f32_to_f16(d);
    float dF = er_ref_f16_to_f32(dBits);
    int quant[256];
    int8_t sc[16];
    for (int sub = 0; sub < 16; ++sub) {
        const float *sv = values + sub * 16;
        float sm = 0.0f;
        for (int i = 0; i < 16; ++i) sm = fmaxf(sm, fabsf(sv[i]));
        if (dF > 0.0f && sm > 0.0f) {
            float ideal = sm / (dF * 31.0f);
            int c = (int)roundf(ideal);
            if (c > 127) c = 127;
            if (c < -128) c = -128;
            sc[sub] = (int8_t)c;
        } else {
            sc[sub] = 0;
        }
        float sf = dF * (float)sc[sub];
        for (int i = 0; i < 16; ++i) {
            if (fabsf(sf) > 0.0f) {
                int raw = (int)roundf(sv[i] / sf) + 32;
                quant[sub * 16 + i] = raw < 0 ? 0 : (raw > 63 ? 63 : raw);
            } else {
                quant[sub * 16 + i] = 32;
            }
        }
    }
    for (int h = 0; h < 2; ++h) {
        int ob = h * 128, qlb = h * 64, qhb = 128 + h * 32;
        for (int l = 0; l < 32; ++l) {
            uint8_t q1 = (uint8_t)quant[ob + l], q2 = (uint8_t)quant[ob + 32 + l];
            uint8_t q3 = (uint8_t)quant[ob + 64 + l], q4 = (uint8_t)quant[ob + 96 + l];
            block[qlb + l] = (uint8_t)((q1 & 0x0f) | ((q3 & 0x0f) << 4));
            block[qlb + 32 + l] = (uint8_t)((q2 & 0x0f) | ((q4 & 0x0f) << 4));
            block[qhb + l] = (uint8_t)(((q1 >> 4) & 3) | (((q2 >> 4) & 3) << 2) |
                                       (((q3 >> 4) & 3) << 4) | (((q4 >> 4) & 3) << 6));
        }
    }
    for (int sub = 0; sub < 16; ++sub) block[192 + sub] = (uint8_t)sc[sub];
    block[208] = (uint8_t)(dBits & 0xff);
    block[209] = (uint8_t)(dBits >> 8);
}

/* Deterministic formula fillers: GEMVTests.swift:136-151 (Q4_K) and
 * :153-170 (Q6_K). */
void er_ref_make_q4k_weights(int rows, int cols, uint8_t *bytes) {
    int blocks = rows * cols / 256;
    for (int b = 0; b < blocks; ++b) {
        uint8_t *p = bytes + (size_t)b * Q4_K_BYTES;
        uint16_t d = er_ref_f32_to_f16(0.03125f + (float)(b % 3) * 0.0078125f);
        uint16_t dm = er_ref_f32_to_f16(0.00390625f);
        p[0] = (uint8_t)(d & 0xff);
        p[1] = (uint8_t)(d >> 8);
        p[2] = (uint8_t)(dm & 0xff);
        p[3] = (uint8_t)(dm >> 8);
        for (int i = 0; i < 12; ++i) p[4 + i] = (uint8_t)((b * 17 + i * 13) & 0xff);
        for (int i = 0; i < 128; ++i) p[16 + i] = (uint8_t)((b * 31 + i * 7) & 0xff);
    }
}

void er_ref_make_q6k_weights(int rows, int cols, uint8_t *bytes) {
    int blocks = rows * cols / 256;
    for (int b = 0; b < blocks; ++b) {
        uint8_t *p = bytes + (size_t)b * Q6_K_BYTES;
        for (int i = 0; i < 128; ++i) p[i] = (uint8_t)((b * 11 + i * 5) & 0xff);
        for (int i = 0; i < 64; ++i) p[128 + i] = (uint8_t)((b * 19 + i * 3) & 0xff);
        for (int i = 0; i < 16; ++i) p[192 + i] = (uint8_t)(int8_t)((i % 7) - 3);
        uint16_t d = er_ref_f32_to_f16(0.015625f + (float)(b % 5) * 0.001953125f);
        p[208] = (uint8_t)(d & 0xff);
        p[209] = (uint8_t)(d >> 8);
    }
}

/* ------------------------------------------------------------------------ */
/* GELU, tanh approximation, saturated outside [-10, 10]: cpuGeluTanh,
 * Tests/EdgeRunnerMetalTests/GEMVTests.swift:38-47 (fp32 evaluation order of
 * the Swift expression: c * (v + 0.044715 * v * v * v), v * 0.5 * (1 + tanh)). */
float er_ref_gelu_tanh(float v) {
    if (v > 10.0f) return v;
    if (v < -10.0f) return 0.0f;
    const float c = 0.7978845608028654f;
    float inner = c * (v + 0.044715f * v * v * v);
    return v * 0.5f * (1.0f + tanhf(inner));
}

/* RMSNorm as FusedKernelTests.cpuRMSNorm (FusedKernelTests.swift:53-57):
 * sequential fp32 sum of squares, scale = 1 / sqrt(sum / n + eps),
 * out[i] = x[i] * scale * w[i] (left to right). */
void er_ref_rmsnorm(const float *x, const float *w, uint32_t n, float eps, float *out) {
    float sumSq = 0.0f;
    for (uint32_t i = 0; i < n; ++i) sumSq = sumSq + x[i] * x[i];
    const float scale = 1.0f / sqrtf(sumSq / (float)n + eps);
    for (uint32_t i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

/* FusedKernelTests.silu (FusedKernelTests.swift:85-87): x / (1 + exp(-x)). */
float er_ref_silu(float v) { return v / (1.0f + expf(-v)); }

/* ------------------------------------------------------------------------ */
/* Greedy top-1 over logits: lowest index wins ties, as the reference's
 * Swift max(by:) in GEMVTests.swift:629 and Dequant_Q6_K.metal:327,338.      */
/* ------------------------------------------------------------------------ */
uint32_t er_ref_argmax(const float *v, uint32_t n) {
    uint32_t best = 0;
    for (uint32_t i = 1; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

/* Greedy top-1 as q6_k_gemv_packed_4row_top1_f32 + q6_k_top1_reduce
 * (Dequant_Q6_K.metal:196-365): per 4-row quad, start from row 4t and take a
 * later row only when strictly larger (Dequant_Q6_K.metal:298-311); then a
 * serial merge of the quad candidates from (-inf, 0), a candidate winning
 * when larger or equal with a lower index (:327, :338).  n % 4 == 0. */
uint32_t er_ref_top1(const float *v, uint32_t n) {
    float best = -INFINITY;
    uint32_t bestIdx = 0;
    for (uint32_t t = 0; t + 3 < n; t += 4) {
        float cv = v[t];
        uint32_t ci = t;
        for (uint32_t k = 1; k < 4; ++k)
            if (v[t + k] > cv) {
                cv = v[t + k];
                ci = t + k;
            }
        if (cv > best || (cv == best && ci < bestIdx)) {
            best = cv;
            bestIdx = ci;
        }
    }
    return bestIdx;
}

int er_ref_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
