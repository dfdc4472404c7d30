/*
 * er_synth.c -- seeded synthetic GGUF weight blocks and activations for the
 * benchmark configurations (host only, no GPU).
 *
 * RNG: xoshiro256** seeded by four splitmix64 outputs, the generator of
 * EdgeRunner's SeededRandomSource (Sources/EdgeRunnerCore/Sampling/
 * SeededRandomSource.swift:3-30).  Draw conventions:
 *   - random bytes come from next() least-significant byte first, 8 per call;
 *   - an integer uniform on n < 256 values rejects bytes >= 256 - 256 % n;
 *   - a normal is Box-Muller on two 53-bit uniforms (one output per pair);
 *   - fp16 / bf16 narrowing rounds to nearest even.
 * Per-block draw order:
 *   Q8_0: d = f16(|N|*dscale); 32 x q ~ U{-127..127}.
 *   Q4_K: d = f16(|N|*dscale), dmin = f16(|N|*dminscale); 8 scales then 8 mins
 *         ~ U{0..63}, packed as DequantQ4KMTests.swift:51-58; 128 qs bytes ~ U{0..255}.
 *   Q6_K: d = f16(|N|*dscale); 16 scales ~ U{-32..31}; 256 x q ~ U{0..63} in
 *         output order, packed as DequantQ6KTests.swift:46-63.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

typedef struct {
    uint64_t s[4];
    uint64_t bytes;
    int nbytes;
} er_rng;

static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void er_synth_rng_seed(er_rng *r, uint64_t seed) {
    uint64_t s = seed;
    for (int i = 0; i < 4; ++i) {
        s += 0x9e3779b97f4a7c15ULL;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
        r->s[i] = z ^ (z >> 31);
    }
    r->bytes = 0;
    r->nbytes = 0;
}

uint64_t er_synth_rng_next(er_rng *r) {
    uint64_t *s = r->s;
    uint64_t result = rotl(s[1] * 5, 7) * 9;
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return result;
}

/* First `n` outputs of the generator for `seed` (used to pin the RNG). */
void er_synth_rng_outputs(uint64_t seed, uint64_t *out, uint32_t n) {
    er_rng r;
    er_synth_rng_seed(&r, seed);
    for (uint32_t i = 0; i < n; ++i) out[i] = er_synth_rng_next(&r);
}

static uint32_t next_byte(er_rng *r) {
    if (r->nbytes == 0) {
        r->bytes = er_synth_rng_next(r);
        r->nbytes = 8;
    }
    uint32_t b = (uint32_t)(r->bytes & 0xffu);
    r->bytes >>= 8;
    r->nbytes -= 1;
    return b;
}

/* uniform integer in [0, n), 1 <= n <= 256 */
static uint32_t uniform_small(er_rng *r, uint32_t n) {
    uint32_t limit = 256u - (256u % n);
    for (;;) {
        uint32_t b = next_byte(r);
        if (b < limit) return b % n;
    }
}

static double uniform53(er_rng *r) { return (double)(er_synth_rng_next(r) >> 11) * 0x1.0p-53; }

static double normal(er_rng *r) {
    double u1 = 1.0 - uniform53(r); /* (0, 1] */
    double u2 = uniform53(r);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return (uint16_t)sign;
        uint32_t e = a >> 23, m = (a & 0x7fffffu) | 0x800000u, sh = 126u - e;
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t h = (((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13);
    uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

static uint16_t f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

static void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xff);
    p[1] = (uint8_t)(v >> 8);
}

/* Q8_0 matrix M x K (K % 32 == 0) -> M*(K/32)*34 bytes. */
int er_synth_q8_0(uint64_t seed, uint32_t M, uint32_t K, float dscale, uint8_t *out) {
    if (K == 0 || K % 32 != 0) return -1;
    er_rng r;
    er_synth_rng_seed(&r, seed);
    uint64_t nblk = (uint64_t)M * (K / 32);
    for (uint64_t b = 0; b < nblk; ++b) {
        uint8_t *p = out + b * 34;
        put16(p, f32_to_f16((float)(fabs(normal(&r)) * dscale)));
        for (int i = 0; i < 32; ++i) p[2 + i] = (uint8_t)(int8_t)((int)uniform_small(&r, 255) - 127);
    }
    return 0;
}

/* Q4_K matrix M x K (K % 256 == 0) -> M*(K/256)*144 bytes. */
int er_synth_q4_k(uint64_t seed, uint32_t M, uint32_t K, float dscale, float dminscale,
                  uint8_t *out) {
    if (K == 0 || K % 256 != 0) return -1;
    er_rng r;
    er_synth_rng_seed(&r, seed);
    uint64_t nblk = (uint64_t)M * (K / 256);
    for (uint64_t b = 0; b < nblk; ++b) {
        uint8_t *p = out + b * 144;
        put16(p, f32_to_f16((float)(fabs(normal(&r)) * dscale)));
        put16(p + 2, f32_to_f16((float)(fabs(normal(&r)) * dminscale)));
        uint8_t sc[8], mn[8];
        for (int i = 0; i < 8; ++i) sc[i] = (uint8_t)uniform_small(&r, 64);
        for (int i = 0; i < 8; ++i) mn[i] = (uint8_t)uniform_small(&r, 64);
        for (int j = 0; j < 4; ++j) {
            p[4 + j] = (uint8_t)((sc[j] & 0x3f) | (((sc[j + 4] >> 4) & 3) << 6));
            p[8 + j] = (uint8_t)((mn[j] & 0x3f) | (((mn[j + 4] >> 4) & 3) << 6));
            p[12 + j] = (uint8_t)((sc[j + 4] & 0x0f) | ((mn[j + 4] & 0x0f) << 4));
        }
        for (int i = 0; i < 128; ++i) p[16 + i] = (uint8_t)next_byte(&r);
    }
    return 0;
}

/* Q6_K matrix M x K (K % 256 == 0) -> M*(K/256)*210 bytes. */
int er_synth_q6_k(uint64_t seed, uint32_t M, uint32_t K, float dscale, uint8_t *out) {
    if (K == 0 || K % 256 != 0) return -1;
    er_rng r;
    er_synth_rng_seed(&r, seed);
    uint64_t nblk = (uint64_t)M * (K / 256);
    uint8_t q[256];
    for (uint64_t b = 0; b < nblk; ++b) {
        uint8_t *p = out + b * 210;
        uint16_t d = f32_to_f16((float)(fabs(normal(&r)) * dscale));
        for (int i = 0; i < 16; ++i) p[192 + i] = (uint8_t)(int8_t)((int)uniform_small(&r, 64) - 32);
        for (int i = 0; i < 256; ++i) q[i] = (uint8_t)uniform_small(&r, 64);
        for (int h = 0; h < 2; ++h) {
            const uint8_t *qq = q + 128 * h;
            uint8_t *ql = p + 64 * h;
            uint8_t *qh = p + 128 + 32 * h;
            for (int l = 0; l < 32; ++l) {
                uint8_t q1 = qq[l], q2 = qq[32 + l], q3 = qq[64 + l], q4 = qq[96 + l];
                ql[l] = (uint8_t)((q1 & 0x0f) | ((q3 & 0x0f) << 4));
                ql[32 + l] = (uint8_t)((q2 & 0x0f) | ((q4 & 0x0f) << 4));
                qh[l] = (uint8_t)(((q1 >> 4) & 3) | (((q2 >> 4) & 3) << 2) | (((q3 >> 4) & 3) << 4) |
                                  (((q4 >> 4) & 3) << 6));
            }
        }
        put16(p + 208, d);
    }
    return 0;
}

void er_synth_normal_f32(uint64_t seed, uint64_t n, float *out) {
    er_rng r;
    er_synth_rng_seed(&r, seed);
    for (uint64_t i = 0; i < n; ++i) out[i] = (float)normal(&r);
}

void er_synth_normal_bf16(uint64_t seed, uint64_t n, uint16_t *out) {
    er_rng r;
    er_synth_rng_seed(&r, seed);
    for (uint64_t i = 0; i < n; ++i) out[i] = f32_to_bf16((float)normal(&r));
}
