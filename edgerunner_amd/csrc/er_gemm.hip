// er_gemm.hip -- prefill GEMM over raw GGUF weights on the matrix cores.
//
//   Y[t][n] = sum_k X[t][k] * W[n][k]      X bf16 [T][K], W Q4_K or Q8_0 rows, Y fp32 [T][N]
//
// The reference has no quantised GEMM: its prefill runs the token-batched
// GEMV (Dequant_Q8_0.metal:143-197, 214-314; LlamaLanguageModel.swift:2515-2617),
// re-reading W once per token.  Here each workgroup dequantises a K-chunk of
// its W tile once into LDS as bf16 and multiplies it against a bf16 X tile
// with v_mfma_f32_32x32x16_bf16 (fp32 accumulation), so W is read from HBM
// about T/TT times instead of T times.
//
// Tiling: a workgroup of 4 waves computes a TT x 128 tile of Y (TT tokens x
// 128 weight rows).  Wave w owns rows [ (w/2)*TT/2, +TT/2 ) x columns
// [ (w%2)*64, +64 ) as (TT/64) x 2 blocks of 32x32 MFMA accumulators.  The K
// loop advances in chunks of 64 (one Q4_K sub-block pair, two Q8_0 blocks):
// global loads of chunk c+1 are issued before the MFMAs of chunk c.
//
// MFMA 32x32x16 bf16 operand layout (lane l, 8 bf16 per operand register):
//   A: row i = l % 32, k = 8 * (l / 32) + 0..7
//   B: col j = l % 32, k = 8 * (l / 32) + 0..7
//   D: 16 fp32 per lane, col j = l % 32, row i = 8 * (r / 4) + 4 * (l / 32) + r % 4
//
// Dequantised weights are rounded to bf16 (round to nearest even) before the
// products; X is bf16 on input.  Products and sums are fp32.
#include "er_common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define ER_GEMM_TN 128         // weight rows per workgroup
#define ER_GEMM_KC 64          // K per chunk
#define ER_GEMM_PITCH 72       // bf16 per LDS row: 64 + 8 padding (16 B) spreads rows over banks

ER_DEV uint32_t pack_bf16x2(float a, float b) {
    bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// Raw bytes one thread fetches for its share of a W chunk, per format.
// Q4_K: thread (row n = t/2, half h = t%2) -> super-block header (16 B) and
//       qs bytes [32p + 16h, +16) of pair p = chunk % 4.
// Q8_0: thread (row n = t/2, half h = t%2) -> block 2*chunk + h (34 B) fetched
//       as the 4-byte-aligned 36-byte window around it.
struct WRaw {
    u32x4 a;      // Q4_K header / Q8_0 window dwords 0-3
    u32x4 b;      // Q4_K qs / Q8_0 window dwords 4-7
    uint32_t c;   // Q8_0 window dword 8
};

template <bool Q4K>
ER_DEV void load_w(const uint8_t *__restrict__ W, size_t rowBytes, uint32_t row, uint32_t chunk,
                   uint32_t h, WRaw &r) {
    const uint8_t *rp = W + (size_t)row * rowBytes;
    if (Q4K) {
        const uint8_t *bp = rp + (size_t)(chunk >> 2) * 144u;
        r.a = ld16_a16(bp);
        r.b = ld16_a16(bp + 16u + 32u * (chunk & 3u) + 16u * h);
        r.c = 0;
    } else {
        // block 2*chunk + h starts at 68*chunk + 34*h; the aligned window starts at 68*chunk + 32*h
        const uint8_t *wp = rp + (size_t)chunk * 68u + 32u * h;
        r.a = ld16_a4(wp);
        r.b = ld16_a4(wp + 16);
        r.c = ld4_a4(wp + 32);
    }
}

// Loads at a uniform base plus a 32-bit per-lane byte offset: the compiler
// forms them as SGPR-base + VGPR-offset loads, so the per-chunk address update
// is scalar instead of 64-bit vector arithmetic per load.
ER_DEV u32x4 ld16_off(const void *base, uint32_t off) { return *(const u32x4 *)((const uint8_t *)base + off); }
ER_DEV u32x4 ld16_off_a4(const void *base, uint32_t off) {
    const u32x4_a4 v = *(const u32x4_a4 *)((const uint8_t *)base + off);
    return u32x4{v.x, v.y, v.z, v.w};
}
ER_DEV uint32_t ld4_off(const void *base, uint32_t off) { return *(const uint32_t *)((const uint8_t *)base + off); }

// load_w with the row's byte offset from W precomputed (rowOff < 2^32, checked
// by the host): the chunk's part of the offset is wave-uniform.
template <bool Q4K>
ER_DEV void load_w_off(const uint8_t *__restrict__ W, uint32_t rowOff, uint32_t chunk, uint32_t h, WRaw &r) {
    if (Q4K) {
        const uint32_t bp = rowOff + (chunk >> 2) * 144u;
        r.a = ld16_off(W, bp);
        r.b = ld16_off(W, bp + 16u + 32u * (chunk & 3u) + 16u * h);
        r.c = 0;
    } else {
        const uint32_t wp = rowOff + chunk * 68u + 32u * h;
        r.a = ld16_off_a4(W, wp);
        r.b = ld16_off_a4(W, wp + 16u);
        r.c = ld4_off(W, wp + 32u);
    }
}

// Dequantises a thread's 32 weights into 16 packed bf16 pairs: out[0..7] are
// chunk positions [16h, 16h+16), out[8..15] positions [32 + 16h, 32 + 16h + 16)
// for Q4_K; for Q8_0 out[0..15] are positions [32h, 32h + 32).
template <bool Q4K>
ER_DEV void dequant_w(const WRaw &r, uint32_t chunk, uint32_t h, uint32_t (&out)[16]) {
    if (Q4K) {
        const float d = f16_to_f32(r.a.x & 0xffffu), dmin = f16_to_f32(r.a.x >> 16);
        uint32_t sc2, m2;
        q4k_scales_pair(r.a.y, r.a.z, r.a.w, chunk & 3u, &sc2, &m2);
        const float sL = d * ub0(sc2), mL = dmin * ub0(m2);
        const float sH = d * ub1(sc2), mH = dmin * ub1(m2);
        const uint32_t qw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        // the nibble mask lives in a register so each masked byte converts with
        // one v_cvt_f32_ubyteN instead of a bit-field extract and a convert
        const uint32_t M0F = vreg_const(0x0f0f0f0fu);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = qw[k] & M0F, hi = (qw[k] >> 4) & M0F;
            out[2 * k + 0] = pack_bf16x2(__builtin_fmaf(sL, ub0(lo), -mL), __builtin_fmaf(sL, ub1(lo), -mL));
            out[2 * k + 1] = pack_bf16x2(__builtin_fmaf(sL, ub2(lo), -mL), __builtin_fmaf(sL, ub3(lo), -mL));
            out[8 + 2 * k + 0] = pack_bf16x2(__builtin_fmaf(sH, ub0(hi), -mH), __builtin_fmaf(sH, ub1(hi), -mH));
            out[8 + 2 * k + 1] = pack_bf16x2(__builtin_fmaf(sH, ub2(hi), -mH), __builtin_fmaf(sH, ub3(hi), -mH));
        }
    } else {
        (void)chunk;
        const uint32_t v[9] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c};
        // h = 0: block at window byte 0 (d = bytes 0-1, qs = bytes 2..33)
        // h = 1: block at window byte 2 (d = bytes 2-3, qs = bytes 4..35)
        const uint32_t sh = h ? 0u : 2u;  // qs dword k = alignbyte(v[k+1], v[k], 2) for h = 0, v[k+1] for h = 1
        const float d = f16_to_f32(h ? (v[0] >> 16) : (v[0] & 0xffffu));
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t q = sh ? alignbyte(v[k + 1], v[k], 2) : v[k + 1];
            out[2 * k + 0] = pack_bf16x2(d * sb(q, 0), d * sb(q, 1));
            out[2 * k + 1] = pack_bf16x2(d * sb(q, 2), d * sb(q, 3));
        }
    }
}

template <bool Q4K, int TT>
ER_DEV void gemm_q(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X,
                   float *__restrict__ Y, uint32_t T, uint32_t N, uint32_t K) {
    constexpr int WT = TT / 2;       // tokens per wave
    constexpr int AI = WT / 32;      // 32-row MFMA blocks per wave along tokens
    constexpr int XLOADS = TT * ER_GEMM_KC * 2 / 16 / 256;  // 16-byte X loads per thread per chunk
    __shared__ __attribute__((aligned(16))) uint16_t As[TT * ER_GEMM_PITCH];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[ER_GEMM_TN * ER_GEMM_PITCH];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n0 = blockIdx.x * ER_GEMM_TN, t0 = blockIdx.y * TT;
    const size_t rowBytes = Q4K ? (size_t)(K >> 8) * 144u : (size_t)(K >> 6) * 68u;
    const uint32_t NC = K / ER_GEMM_KC;

    // W share: row n0 + tid/2 (clamped), half tid%2
    const uint32_t wRow = min(n0 + (tid >> 1), N - 1u), wh = tid & 1u;
    // X share: XLOADS 16-byte pieces; piece q of thread tid covers X tile row
    // (tid + 256 q) / 8 and k offset 8 * ((tid + 256 q) % 8)
    auto load_x = [&](uint32_t chunk, u32x4 (&xr)[XLOADS]) {
#pragma unroll
        for (int q = 0; q < XLOADS; ++q) {
            const uint32_t p = tid + 256u * q;
            const uint32_t row = min(t0 + (p >> 3), T - 1u);
            xr[q] = *(const u32x4 *)(X + (size_t)row * K + chunk * ER_GEMM_KC + 8u * (p & 7u));
        }
    };

    f32x16 acc[AI][2];
#pragma unroll
    for (int i = 0; i < AI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    WRaw wr;
    u32x4 xr[XLOADS];
    load_w<Q4K>(W, rowBytes, wRow, 0, wh, wr);
    load_x(0, xr);

    const uint32_t wt = wave >> 1, wn = wave & 1u;
    for (uint32_t c = 0; c < NC; ++c) {
        uint32_t wd[16];
        dequant_w<Q4K>(wr, c, wh, wd);
        __syncthreads();  // the previous chunk's MFMAs are done with As/Bs
        {
            uint16_t *brow = Bs + (tid >> 1) * ER_GEMM_PITCH;
            if (Q4K) {
                *(u32x4 *)(brow + 16u * wh) = u32x4{wd[0], wd[1], wd[2], wd[3]};
                *(u32x4 *)(brow + 16u * wh + 8u) = u32x4{wd[4], wd[5], wd[6], wd[7]};
                *(u32x4 *)(brow + 32u + 16u * wh) = u32x4{wd[8], wd[9], wd[10], wd[11]};
                *(u32x4 *)(brow + 32u + 16u * wh + 8u) = u32x4{wd[12], wd[13], wd[14], wd[15]};
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *(u32x4 *)(brow + 32u * wh + 8u * q) =
                        u32x4{wd[4 * q], wd[4 * q + 1], wd[4 * q + 2], wd[4 * q + 3]};
            }
#pragma unroll
            for (int q = 0; q < XLOADS; ++q) {
                const uint32_t p = tid + 256u * q;
                *(u32x4 *)(As + (p >> 3) * ER_GEMM_PITCH + 8u * (p & 7u)) = xr[q];
            }
        }
        __syncthreads();
        if (c + 1 < NC) {
            load_w<Q4K>(W, rowBytes, wRow, c + 1, wh, wr);
            load_x(c + 1, xr);
        }
#pragma unroll
        for (int ks = 0; ks < ER_GEMM_KC / 16; ++ks) {
            const uint32_t kof = 16u * ks + 8u * (lane >> 5);
            bf16x8 a[AI], b[2];
#pragma unroll
            for (int i = 0; i < AI; ++i)
                a[i] = *(const bf16x8 *)(As + (wt * WT + 32u * i + (lane & 31u)) * ER_GEMM_PITCH + kof);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *(const bf16x8 *)(Bs + (wn * 64u + 32u * j + (lane & 31u)) * ER_GEMM_PITCH + kof);
#pragma unroll
            for (int i = 0; i < AI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
    // D layout: col j = lane % 32, row i = 8 * (r / 4) + 4 * (lane / 32) + r % 4
#pragma unroll
    for (int i = 0; i < AI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n0 + wn * 64u + 32u * j + (lane & 31u);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t t = t0 + wt * WT + 32u * i + 8u * (r >> 2) + 4u * (lane >> 5) + (r & 3);
                if (t < T && n < N) Y[(size_t)t * N + n] = acc[i][j][r];
            }
        }
}

#define ER_GEMM_ENTRY(fmt, q4k, tt)                                                              \
    extern "C" __global__ void __launch_bounds__(256)                                          \
        er_gemm_##fmt##_t##tt(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X,   \
                              float *__restrict__ Y, uint32_t T, uint32_t N, uint32_t K) {      \
        gemm_q<q4k, tt>(W, X, Y, T, N, K);                                                      \
    }

ER_GEMM_ENTRY(q4k, true, 128)
ER_GEMM_ENTRY(q4k, true, 256)
ER_GEMM_ENTRY(q8_0, false, 128)
ER_GEMM_ENTRY(q8_0, false, 256)

// ---------------------------------------------------------------------------
// Pipelined variant: two LDS stages and one register stage, so the global
// loads of chunk c+2 are in flight while the MFMAs of chunk c run; one
// barrier per chunk.  Tiles are walked XCD-major: workgroup L runs on XCD
// L % 8 (round-robin dispatch) and takes tile (L % 8) * per + L / 8 of the
// (N-tile major, token-tile minor) order, so each XCD's L2 keeps a contiguous
// slice of W while it sweeps the token tiles.
// ---------------------------------------------------------------------------
template <bool Q4K, int TT>
ER_DEV void gemm_q_pipe(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X,
                        float *__restrict__ Y, uint32_t T, uint32_t N, uint32_t K, uint32_t SK) {
    constexpr int WT = TT / 2;
    constexpr int AI = WT / 32;
    constexpr int XLOADS = TT * ER_GEMM_KC * 2 / 16 / 256;
    constexpr int ASZ = TT * ER_GEMM_PITCH, BSZ = ER_GEMM_TN * ER_GEMM_PITCH;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];  // 2 x (A stage + B stage)

    const uint32_t nT = (T + TT - 1) / TT, nN = (N + ER_GEMM_TN - 1) / ER_GEMM_TN;
    const uint32_t total = nT * nN * SK, per = (total + 7u) / 8u;
    const uint32_t L = blockIdx.x;
    const uint32_t item = (L % 8u) * per + L / 8u;  // (N tile, K split, token tile), token tile fastest
    if (item >= total) return;
    const uint32_t tt = item % nT, rest = item / nT;
    const uint32_t ks0 = rest % SK, nt = rest / SK;
    const uint32_t n0 = nt * ER_GEMM_TN, t0 = tt * TT;

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const size_t rowBytes = Q4K ? (size_t)(K >> 8) * 144u : (size_t)(K >> 6) * 68u;
    const uint32_t NCall = K / ER_GEMM_KC;
    const uint32_t cBeg = (uint32_t)(((uint64_t)NCall * ks0) / SK);
    const uint32_t NC = (uint32_t)(((uint64_t)NCall * (ks0 + 1u)) / SK) - cBeg;
    const uint32_t wRow = min(n0 + (tid >> 1), N - 1u), wh = tid & 1u;
    const uint32_t wRowOff = wRow * (uint32_t)rowBytes;  // < 2^32 (host check)
    // byte offsets of this thread's X pieces in chunk 0 (< 2^32, host check)
    uint32_t xOff[XLOADS];
#pragma unroll
    for (int q = 0; q < XLOADS; ++q) {
        const uint32_t p = tid + 256u * q;
        xOff[q] = (min(t0 + (p >> 3), T - 1u) * K + 8u * (p & 7u)) * 2u;
    }
    auto load_x = [&](uint32_t chunk, u32x4 (&xr)[XLOADS]) {
#pragma unroll
        for (int q = 0; q < XLOADS; ++q) xr[q] = ld16_off(X, xOff[q] + chunk * (ER_GEMM_KC * 2u));
    };
    auto store_stage = [&](uint32_t stage, uint32_t chunk, const WRaw &wr, const u32x4 (&xr)[XLOADS]) {
        uint16_t *As = smem + stage * (ASZ + BSZ);
        uint16_t *Bs = As + ASZ;
        uint32_t wd[16];
        dequant_w<Q4K>(wr, chunk, wh, wd);
        uint16_t *brow = Bs + (tid >> 1) * ER_GEMM_PITCH;
        if (Q4K) {
            *(u32x4 *)(brow + 16u * wh) = u32x4{wd[0], wd[1], wd[2], wd[3]};
            *(u32x4 *)(brow + 16u * wh + 8u) = u32x4{wd[4], wd[5], wd[6], wd[7]};
            *(u32x4 *)(brow + 32u + 16u * wh) = u32x4{wd[8], wd[9], wd[10], wd[11]};
            *(u32x4 *)(brow + 32u + 16u * wh + 8u) = u32x4{wd[12], wd[13], wd[14], wd[15]};
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *(u32x4 *)(brow + 32u * wh + 8u * q) = u32x4{wd[4 * q], wd[4 * q + 1], wd[4 * q + 2], wd[4 * q + 3]};
        }
#pragma unroll
        for (int q = 0; q < XLOADS; ++q) {
            const uint32_t p = tid + 256u * q;
            *(u32x4 *)(As + (p >> 3) * ER_GEMM_PITCH + 8u * (p & 7u)) = xr[q];
        }
    };

    f32x16 acc[AI][2];
#pragma unroll
    for (int i = 0; i < AI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Register buffers rotate over 3 chunks: the global loads of chunk c+3
    // are issued in iteration c, two iterations before they are stored to LDS.
    WRaw wr[3];
    u32x4 xr[3][XLOADS];
    const uint32_t wt = wave >> 1, wn = wave & 1u;
    auto mfma_stage = [&](uint32_t stage) {
        const uint16_t *As = smem + stage * (ASZ + BSZ);
        const uint16_t *Bs = As + ASZ;
#pragma unroll
        for (int ks = 0; ks < ER_GEMM_KC / 16; ++ks) {
            const uint32_t kof = 16u * ks + 8u * (lane >> 5);
            bf16x8 a[AI], b[2];
#pragma unroll
            for (int i = 0; i < AI; ++i)
                a[i] = *(const bf16x8 *)(As + (wt * WT + 32u * i + (lane & 31u)) * ER_GEMM_PITCH + kof);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *(const bf16x8 *)(Bs + (wn * 64u + 32u * j + (lane & 31u)) * ER_GEMM_PITCH + kof);
#pragma unroll
            for (int i = 0; i < AI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };
    // chunk c's data sits in register buffer c % 3
    load_w_off<Q4K>(W, wRowOff, cBeg, wh, wr[0]);
    load_x(cBeg, xr[0]);
    if (NC > 1) {
        load_w_off<Q4K>(W, wRowOff, cBeg + 1, wh, wr[1]);
        load_x(cBeg + 1, xr[1]);
    }
    if (NC > 2) {
        load_w_off<Q4K>(W, wRowOff, cBeg + 2, wh, wr[2]);
        load_x(cBeg + 2, xr[2]);
    }
    store_stage(0, cBeg, wr[0], xr[0]);
    // iteration c: barrier; MFMAs of stage c%2 (issued first, so the dequant
    // VALU work below overlaps them on the matrix pipe); store chunk c+1
    // (buffer (c+1)%3) into stage (c+1)%2; load chunk c+3 into buffer c%3
    // (free: chunk c was stored last iteration)
#define ER_GEMM_STEP(B)                                                                  \
    {                                                                                    \
        const uint32_t c = c3 + (B);                                                     \
        if (c < NC) {                                                                    \
            __syncthreads();                                                             \
            mfma_stage(c & 1u);                                                          \
            if (c + 1 < NC) store_stage((c + 1) & 1u, cBeg + c + 1, wr[((B) + 1) % 3], xr[((B) + 1) % 3]); \
            if (c + 3 < NC) {                                                            \
                load_w_off<Q4K>(W, wRowOff, cBeg + c + 3, wh, wr[(B)]);                  \
                load_x(cBeg + c + 3, xr[(B)]);                                           \
            }                                                                            \
        }                                                                                \
    }
    for (uint32_t c3 = 0; c3 < NC; c3 += 3) {
        ER_GEMM_STEP(0)
        ER_GEMM_STEP(1)
        ER_GEMM_STEP(2)
    }
#undef ER_GEMM_STEP
#pragma unroll
    for (int i = 0; i < AI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n0 + wn * 64u + 32u * j + (lane & 31u);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t t = t0 + wt * WT + 32u * i + 8u * (r >> 2) + 4u * (lane >> 5) + (r & 3);
                if (t < T && n < N) {
                    if (SK == 1) Y[(size_t)t * N + n] = acc[i][j][r];
                    else atomicAdd(Y + (size_t)t * N + n, acc[i][j][r]);  // Y zero-filled by er_fill_zero
                }
            }
        }
}

// Zero fill for split-K accumulation (a kernel, so that it can be recorded in
// a HIP graph; 16-byte stores, n4 float4 elements).
extern "C" __global__ void __launch_bounds__(256) er_fill_zero(float4 *__restrict__ p, uint64_t n4) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n4; i += (uint64_t)gridDim.x * 256u)
        p[i] = float4{0.0f, 0.0f, 0.0f, 0.0f};
}

// ---------------------------------------------------------------------------
// Warp-specialised variant (512 threads, TT = 128): waves 0-3 run the MFMAs of
// chunk c from LDS stage c % 2 while waves 4-7 dequantise chunk c+1 into the
// other stage; one barrier per chunk for all 8 waves.  The staging waves keep
// 4 chunks of raw weights and X in registers and load unconditionally (chunk
// indices past the split are clamped re-loads), so every vmcnt wait covers
// exactly one chunk.  Requires the split's chunk count NC % 4 == 0 (host);
// a workgroup whose split breaks that returns before any barrier.
// ---------------------------------------------------------------------------
template <bool Q4K, bool FENCE>
ER_DEV void gemm_q_ws(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X, float *__restrict__ Y,
                      uint32_t T, uint32_t N, uint32_t K, uint32_t SK) {
    constexpr int TT = 128, WT = TT / 2, AI = WT / 32, NST = 2, NB = 4;
    constexpr int XLOADS = TT * ER_GEMM_KC * 2 / 16 / 256;
    constexpr int ASZ = TT * ER_GEMM_PITCH, BSZ = ER_GEMM_TN * ER_GEMM_PITCH;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];  // NST x (A stage + B stage)
    const uint32_t nT = (T + TT - 1) / TT, nN = (N + ER_GEMM_TN - 1) / ER_GEMM_TN;
    const uint32_t total = nT * nN * SK, per = (total + 7u) / 8u;
    const uint32_t L = blockIdx.x;
    const uint32_t item = (L % 8u) * per + L / 8u;  // (N tile, K split, token tile), token tile fastest
    if (item >= total) return;
    const uint32_t tt = item % nT, rest = item / nT;
    const uint32_t ks0 = rest % SK, nt = rest / SK;
    const uint32_t n0 = nt * ER_GEMM_TN, t0 = tt * TT;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t NCall = K / ER_GEMM_KC;
    const uint32_t cBeg = (uint32_t)(((uint64_t)NCall * ks0) / SK);
    const uint32_t NC = (uint32_t)(((uint64_t)NCall * (ks0 + 1u)) / SK) - cBeg;
    if (NC == 0 || NC % NB != 0) return;  // never launched so (host); keeps the barrier counts equal
    const uint32_t rowBytes = Q4K ? (K >> 8) * 144u : (K >> 6) * 68u;

    if (wave >= 4) {
        // staging waves: thread d owns weight row n0 + d/2 (half d%2) and XLOADS X pieces
        const uint32_t d = tid - 256u;
        const uint32_t wRowOff = min(n0 + (d >> 1), N - 1u) * rowBytes, wh = d & 1u;
        uint32_t xOff[XLOADS];
#pragma unroll
        for (int q = 0; q < XLOADS; ++q) {
            const uint32_t p = d + 256u * q;
            xOff[q] = (min(t0 + (p >> 3), T - 1u) * K + 8u * (p & 7u)) * 2u;
        }
        WRaw wr[NB];
        u32x4 xr[NB][XLOADS];
        const uint32_t cLast = cBeg + NC - 1u;
        auto load = [&](uint32_t chunk, int b) {
            chunk = min(chunk, cLast);
            load_w_off<Q4K>(W, wRowOff, chunk, wh, wr[b]);
#pragma unroll
            for (int q = 0; q < XLOADS; ++q) xr[b][q] = ld16_off(X, xOff[q] + chunk * (ER_GEMM_KC * 2u));
        };
        auto store = [&](uint32_t stage, uint32_t chunk, int b) {
            chunk = min(chunk, cLast);
            uint16_t *As = smem + stage * (ASZ + BSZ);
            uint16_t *Bs = As + ASZ;
            uint32_t wd[16];
            dequant_w<Q4K>(wr[b], chunk, wh, wd);
            uint16_t *brow = Bs + (d >> 1) * ER_GEMM_PITCH;
            if (Q4K) {
                *(u32x4 *)(brow + 16u * wh) = u32x4{wd[0], wd[1], wd[2], wd[3]};
                *(u32x4 *)(brow + 16u * wh + 8u) = u32x4{wd[4], wd[5], wd[6], wd[7]};
                *(u32x4 *)(brow + 32u + 16u * wh) = u32x4{wd[8], wd[9], wd[10], wd[11]};
                *(u32x4 *)(brow + 32u + 16u * wh + 8u) = u32x4{wd[12], wd[13], wd[14], wd[15]};
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *(u32x4 *)(brow + 32u * wh + 8u * q) = u32x4{wd[4 * q], wd[4 * q + 1], wd[4 * q + 2], wd[4 * q + 3]};
            }
#pragma unroll
            for (int q = 0; q < XLOADS; ++q) {
                const uint32_t p = d + 256u * q;
                *(u32x4 *)(As + (p >> 3) * ER_GEMM_PITCH + 8u * (p & 7u)) = xr[b][q];
            }
        };
#pragma unroll
        for (int b = 0; b < NB; ++b) load(cBeg + (uint32_t)b, b);
        store(0, cBeg, 0);
        __syncthreads();  // stage 0 ready
        // iteration c: fill stage (c+1) % NST with chunk c+1 (buffer (c+1) % NB),
        // refill buffer c % NB with chunk c+NB, barrier
        for (uint32_t c0 = 0; c0 < NC; c0 += NB) {
#pragma unroll
            for (int B = 0; B < NB; ++B) {
                const uint32_t c = c0 + (uint32_t)B;
                store((c + 1u) % NST, cBeg + c + 1u, (B + 1) % NB);
                load(cBeg + c + NB, B);
                __syncthreads();
                // Register arithmetic moves freely across s_barrier: without
                // this fence the scheduler hoists the next steps' Q4_K header
                // decoding into this one, and its vmcnt waits then cover loads
                // issued one or two chunks ago instead of three (512x14336x4096:
                // 103 -> 95 us).  Q8_0 runs faster unfenced (48 -> 45 us at
                // 512x4096x4096), its waits staying three chunks deep.
                if (FENCE) __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        const uint32_t wt = wave >> 1, wn = wave & 1u;
        f32x16 acc[AI][2];
#pragma unroll
        for (int i = 0; i < AI; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        __syncthreads();  // stage 0 ready
        for (uint32_t c = 0; c < NC; ++c) {
            const uint16_t *As = smem + (c % NST) * (ASZ + BSZ);
            const uint16_t *Bs = As + ASZ;
#pragma unroll
            for (int ks = 0; ks < ER_GEMM_KC / 16; ++ks) {
                const uint32_t kof = 16u * ks + 8u * (lane >> 5);
                bf16x8 a[AI], b[2];
#pragma unroll
                for (int i = 0; i < AI; ++i)
                    a[i] = *(const bf16x8 *)(As + (wt * WT + 32u * i + (lane & 31u)) * ER_GEMM_PITCH + kof);
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    b[j] = *(const bf16x8 *)(Bs + (wn * 64u + 32u * j + (lane & 31u)) * ER_GEMM_PITCH + kof);
#pragma unroll
                for (int i = 0; i < AI; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
            __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < AI; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t n = n0 + wn * 64u + 32u * j + (lane & 31u);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t t = t0 + wt * WT + 32u * i + 8u * (r >> 2) + 4u * (lane >> 5) + (r & 3);
                    if (t < T && n < N) {
                        if (SK == 1) Y[(size_t)t * N + n] = acc[i][j][r];
                        else atomicAdd(Y + (size_t)t * N + n, acc[i][j][r]);  // Y zero-filled by er_fill_zero
                    }
                }
            }
    }
}

extern "C" __global__ void __launch_bounds__(512)
    er_gemmw_q4k_t128(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X, float *__restrict__ Y,
                      uint32_t T, uint32_t N, uint32_t K, uint32_t SK) {
    gemm_q_ws<true, true>(W, X, Y, T, N, K, SK);
}
extern "C" __global__ void __launch_bounds__(512)
    er_gemmw_q8_0_t128(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X, float *__restrict__ Y,
                       uint32_t T, uint32_t N, uint32_t K, uint32_t SK) {
    gemm_q_ws<false, false>(W, X, Y, T, N, K, SK);
}

#define ER_GEMMP_ENTRY(fmt, q4k, tt)                                                             \
    extern "C" __global__ void __launch_bounds__(256)                                          \
        er_gemmp_##fmt##_t##tt(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X,  \
                               float *__restrict__ Y, uint32_t T, uint32_t N, uint32_t K,       \
                               uint32_t SK) {                                                   \
        gemm_q_pipe<q4k, tt>(W, X, Y, T, N, K, SK);                                             \
    }

ER_GEMMP_ENTRY(q4k, true, 64)
ER_GEMMP_ENTRY(q8_0, false, 64)
ER_GEMMP_ENTRY(q4k, true, 128)
ER_GEMMP_ENTRY(q4k, true, 256)
ER_GEMMP_ENTRY(q8_0, false, 128)
ER_GEMMP_ENTRY(q8_0, false, 256)

// ---------------------------------------------------------------------------
// Loader-specialised variant (512 threads, 128 R weight rows x 128 tokens per
// workgroup, K % 256 == 0).  Waves 4-5 copy the X tile and waves 6-7 the raw
// weight bytes of each 64-wide chunk into LDS rings with global_load_lds, each
// pair with its own vmcnt queue, so an X copy never waits behind a weight
// fetch from HBM (a wave's loads complete in issue order).  Waves 0-3 never
// touch global memory until the epilogue: wave w dequantises the raw bytes of
// its 32 R rows straight into MFMA operand registers and multiplies them
// against all 128 tokens (R x 4 blocks of 32x32 accumulators), so only X
// passes through LDS as bf16.
//
// Compute waves, per chunk c and MFMA step s (one scheduling region each):
// the LDS reads of the next step's X fragments are issued first (after step
// 3: the next chunk's step 0 and the raw weights of chunk c + 2), then the
// step's matrix instructions, each followed by a share of the dequantisation
// of step s of chunk c + 1, so the LDS latency and the conversion both run
// under the matrix instructions.
//
// Per chunk c, one barrier for all 8 waves (barrier c):
//   - before it, the X pair waits until chunk c + 1 is in LDS and the weight
//     pair until chunk c + 2 is (both are read ahead during chunk c);
//   - after it, the X pair copies chunk c + DX into the stage of chunk c - 1
//     (DX = NX - 1) and the weight pair chunk c + DW into the stage of chunk c
//     (DW = NW; those raw bytes were read during chunk c - 2).
// Copies past the last chunk re-copy the last chunk into a free stage, so each
// loader's wait is the same every iteration.
//
// LDS: X stages of 128 token rows x 144 bytes (128 of data + 16 of padding,
// so the 16-byte A-fragment reads of 32 consecutive rows fall on distinct
// banks); weight stages of 128 R rows x WROWB bytes:
//   Q4_K: 32 = the chunk's qs bytes; the 16-byte super-block headers sit in a
//         ring of 4 slots (one super-block each) that the weight pair fills a
//         quarter per chunk copy, so each header is copied once, not once per
//         chunk (48 bytes per row and chunk before: 3.8% faster at
//         512 x 4096 x 4096, 1.8% at 512 x 14336 x 4096);
//   Q8_0: 80 = the 16-byte-aligned window [68c & ~15, +80) of the row's bytes,
//         which holds the chunk's two 34-byte blocks at offset 4 (c % 4).
// Header slot S % 4 is refilled from copy 4 S - 4 on, issued after barrier
// 4 S - 4 - DW; its previous header, S - 4, was last read for chunk 4 S - 13,
// whose raw bytes were consumed before barrier 4 S - 13.
//
// Inside a chunk the k order of each MFMA step s is the one the raw bytes give
// lane half h (gemml_acol): Q4_K low nibbles of qs bytes [16h, 16h + 16) for
// s < 2, their high nibbles for s >= 2; Q8_0 block h; the A fragments read X
// at the same k, so every product pairs the right operands.
// ---------------------------------------------------------------------------
#define ER_GEMML_TT 128
#define ER_GEMML_XROWB 144
#define ER_GEMML_XSTAGE (ER_GEMML_TT * ER_GEMML_XROWB)  // 18432

// R: 32-row blocks per compute wave; the workgroup tile is TN = 128 R weight
// rows (R = 2: 256 rows, for grids that fill the chip with 256-row tiles;
// R = 1: 128 rows, twice the workgroups for narrower matrices).
template <bool Q4K, int R>
struct GemmL {
    static constexpr uint32_t TN = 128u * R;
    static constexpr uint32_t WROWB = Q4K ? 32u : 80u;
    static constexpr uint32_t WSTAGE = TN * WROWB;            // R = 2: 8192 / 20480, R = 1: 4096 / 10240
    static constexpr int NX = 4;                              // X stages
    static constexpr int NW = R == 2 ? (Q4K ? 6 : 4) : (Q4K ? 8 : 6);  // weight stages
    static constexpr int DX = NX - 1, DW = NW;                // copy-ahead distances (chunks)
    static constexpr int LX = ER_GEMML_XSTAGE / 1024 / 2;     // 9 copies per X wave per chunk
    static constexpr int LWQ = (int)(WSTAGE / 1024u / 2u);    // 1 KB copies per weight wave per chunk
    // Q4_K super-block headers: NH slots of TN rows x 16 bytes; each chunk copy
    // carries a quarter of a header in 256-byte copies (4 bytes per lane)
    static constexpr int NH = Q4K ? 4 : 0;
    static constexpr uint32_t HSTAGE = Q4K ? TN * 16u : 0u;
    static constexpr int LWH = (int)(HSTAGE / 4u / 256u / 2u);  // 256-byte copies per weight wave per chunk
    static constexpr int LW = LWQ + LWH;                        // copies per weight wave per chunk
    static constexpr uint32_t LDS = NX * ER_GEMML_XSTAGE + NW * WSTAGE + NH * HSTAGE;
    static_assert(WSTAGE % 2048u == 0, "weight stages split into 1 KB copies over two waves");
    static_assert(HSTAGE % 2048u == 0, "header quarters split into 256-byte copies over two waves");
    static_assert(4 * LWH + DW * LW < 64 && (DX - 1) * LX < 64, "waits fit the load counter");
};

ER_DEV uint32_t gemml_acol(bool q4k, uint32_t s, uint32_t h) {
    // bf16 column of the chunk that step s / lane half h reads
    return q4k ? 32u * (s >> 1) + 16u * h + 8u * (s & 1u) : 32u * h + 8u * s;
}

// Scales of one lane's weights for a chunk: Q4_K (s0, m0) for the low
// nibbles (sub-block 2p of pair p = chunk % 4) and (s1, m1) for the high
// nibbles (sub-block 2p + 1); Q8_0 s0 = d of block 2 chunk + h.
struct DqScale {
    float s0, m0, s1, m1;
};

template <bool Q4K>
ER_DEV DqScale dq_scale(const WRaw &r, uint32_t chunk, uint32_t h) {
    DqScale q;
    if (Q4K) {
        const float d = f16_to_f32(r.a.x & 0xffffu), dmin = f16_to_f32(r.a.x >> 16);
        uint32_t sc2, m2;
        q4k_scales_pair(r.a.y, r.a.z, r.a.w, chunk & 3u, &sc2, &m2);
        q.s0 = d * ub0(sc2);
        q.m0 = dmin * ub0(m2);
        q.s1 = d * ub1(sc2);
        q.m1 = dmin * ub1(m2);
    } else {
        q.s0 = f16_to_f32(h ? (r.a.x >> 16) : (r.a.x & 0xffffu));
        q.m0 = -128.0f * q.s0;  // exact: a power-of-two multiple of d
        q.s1 = q.m1 = 0.0f;
    }
    return q;
}

// The four packed bf16 pairs of MFMA step s (0..3) that dequant_w puts at
// out[4s .. 4s + 3], with the same operations, so a chunk can be
// dequantised one step at a time between the matrix instructions.
template <bool Q4K>
ER_DEV void dq_step(const WRaw &r, const DqScale &q, uint32_t h, int s, uint32_t *out) {
    if (Q4K) {
        const uint32_t qw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        const uint32_t M0F = vreg_const(0x0f0f0f0fu);
        const bool hi = s >= 2;
        const float sc = hi ? q.s1 : q.s0, mn = hi ? q.m1 : q.m0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t w = qw[2 * (s & 1) + j];
            const uint32_t v = hi ? ((w >> 4) & M0F) : (w & M0F);
            out[2 * j + 0] = pack_bf16x2(__builtin_fmaf(sc, ub0(v), -mn), __builtin_fmaf(sc, ub1(v), -mn));
            out[2 * j + 1] = pack_bf16x2(__builtin_fmaf(sc, ub2(v), -mn), __builtin_fmaf(sc, ub3(v), -mn));
        }
    } else {
        const uint32_t v[9] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c};
        // byte b as u = b + 128 (flipping the sign bit), then d * u - 128 d:
        // for finite d, d * u and 128 d are exact and so is their difference d * b, which
        // equals the d * b of dequant_w
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int k = 2 * s + j;
            const uint32_t w = (h ? v[k + 1] : alignbyte(v[k + 1], v[k], 2)) ^ 0x80808080u;
            out[2 * j + 0] = pack_bf16x2(__builtin_fmaf(q.s0, ub0(w), q.m0), __builtin_fmaf(q.s0, ub1(w), q.m0));
            out[2 * j + 1] = pack_bf16x2(__builtin_fmaf(q.s0, ub2(w), q.m0), __builtin_fmaf(q.s0, ub3(w), q.m0));
        }
    }
}

template <int N>
ER_DEV void gemml_vmwait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(N) & 0xc07f);
}

// s_barrier with only a compiler ordering fence around it: a release fence
// would also wait for the loader's global_load_lds copies in flight (they
// write LDS) and so drain the prefetch.
ER_DEV void gemml_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// STAMPED (the measurement build's clock probe only; the product kernels are
// built without it): thread 0 of each work item's workgroup writes
// stamps[4 item ..] = the 100 MHz real-time counter and the shader-clock
// counter at its start and after its epilogue, so the clock the workgroup ran
// at is d(shader clock) / d(real time) x 100 MHz.
template <bool Q4K, int R, bool STAMPED = false>
ER_DEV void gemm_ls(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X, float *__restrict__ Y,
                    uint32_t T, uint32_t N, uint32_t K, uint64_t *__restrict__ stamps = nullptr) {
    using G = GemmL<Q4K, R>;
    uint64_t rt0 = 0, ct0 = 0;
    if constexpr (STAMPED) {
        rt0 = __builtin_amdgcn_s_memrealtime();
        ct0 = __builtin_amdgcn_s_memtime();
    }
    extern __shared__ __attribute__((aligned(16))) uint8_t glds[];
    uint8_t *xs = glds;                             // NX X stages
    uint8_t *wsm = glds + G::NX * ER_GEMML_XSTAGE;  // NW weight stages
    uint8_t *hsm = wsm + G::NW * G::WSTAGE;         // NH Q4_K header slots
    const uint32_t nT = (T + ER_GEMML_TT - 1) / ER_GEMML_TT, nN = (N + G::TN - 1) / G::TN;
    const uint32_t total = nT * nN, per = (total + 7u) / 8u;
    const uint32_t L = blockIdx.x;
    // the items of one XCD (L % 8) are consecutive, token tile fastest, so the
    // workgroups reading one weight tile share that XCD's L2
    const uint32_t item = (L % 8u) * per + L / 8u;
    if (item >= total) return;
    const uint32_t tt = item % nT, nt = item / nT;
    const uint32_t n0 = nt * G::TN, t0 = tt * ER_GEMML_TT;
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t NC = K / 64u;
    const uint32_t rowBytes = Q4K ? (K >> 8) * 144u : (K >> 6) * 68u;

    if (wave >= 6) {
        // weight copies: unit u (of the stage's 2 LWQ units of 1 KB) puts 16
        // bytes at stage byte 1024 u + 16 lane = row r, byte b of the row
        // (Q4_K: qs bytes [32 p + b, +16) of the chunk's pair p; Q8_0: the
        // chunk's aligned window)
        const uint32_t wv = wave - 6u, ub = wv * G::LWQ;
        uint32_t wa[G::LWQ];
#pragma unroll
        for (int q = 0; q < G::LWQ; ++q) {
            const uint32_t o = 1024u * (ub + q) + 16u * lane, r = o / G::WROWB, b = o % G::WROWB;
            wa[q] = min(n0 + r, N - 1u) * rowBytes + (Q4K ? 16u : 0u) + b;
        }
        // Q4_K header copies: copy k of quarter hq puts 4 bytes at quarter byte
        // 256 (wv LWH + k) + 4 lane = header byte 4 (lane % 4) of row
        // hq TN / 4 + 16 (wv LWH + k) + lane / 4; a slot holds row r's header
        // at byte 16 r
        uint32_t ha[4][G::LWH > 0 ? G::LWH : 1];
#pragma unroll
        for (int hq = 0; hq < 4; ++hq)
#pragma unroll
            for (int k = 0; k < G::LWH; ++k) {
                const uint32_t r = (uint32_t)hq * (G::TN / 4u) + 16u * (wv * G::LWH + (uint32_t)k) + lane / 4u;
                ha[hq][k] = min(n0 + r, N - 1u) * rowBytes + 4u * (lane % 4u);
            }
        // quarter hq of super-block sb's header into slot sl
        auto issueHeader = [&](uint32_t sb, uint32_t sl, uint32_t hq) {
            uint8_t *hd = hsm + sl * G::HSTAGE + hq * (G::HSTAGE / 4u) + 256u * wv * G::LWH;
#pragma unroll
            for (int k = 0; k < G::LWH; ++k)
                __builtin_amdgcn_global_load_lds((const void *)(W + ha[hq][k] + sb * 144u), (void *)(hd + 256u * k),
                                                 4, 0, 0);
        };
        // copy j: chunk j's weight bytes into stage `slot` and (Q4_K) quarter
        // j % 4 of super-block j / 4 + 1's header into slot (j / 4 + 1) % NH,
        // so the header of super-block S is in with chunks 4 S - 4 .. 4 S - 1,
        // before chunk 4 S is read; copies past the end re-copy the last chunk
        // and header
        auto issue = [&](uint32_t j, uint32_t slot) {
            const uint32_t chunk = min(j, NC - 1u);
            uint8_t *st = wsm + slot * G::WSTAGE + 1024u * ub;
            const uint32_t cq = Q4K ? (chunk >> 2) * 144u + 32u * (chunk & 3u) : (68u * chunk) & ~15u;
#pragma unroll
            for (int q = 0; q < G::LWQ; ++q)
                __builtin_amdgcn_global_load_lds((const void *)(W + wa[q] + cq), (void *)(st + 1024u * q), 16, 0, 0);
            if (Q4K) {
                const uint32_t sh = j / 4u + 1u;
                issueHeader(min(sh, NC / 4u - 1u), sh % (uint32_t)G::NH, j & 3u);
            }
        };
        if (Q4K) {
#pragma unroll
            for (uint32_t hq = 0; hq < 4u; ++hq) issueHeader(0u, 0u, hq);  // super-block 0's header
        }
        // chunks 0..2 first, the rest of the copy-ahead after the first
        // barrier, so the launch's first requests are the ones the compute
        // waves wait for
#pragma unroll
        for (int j = 0; j < 3; ++j) issue((uint32_t)j, (uint32_t)j);
        gemml_vmwait<G::LW>();  // header 0 and chunks 0 and 1 are in
        gemml_barrier();
#pragma unroll
        for (int j = 3; j < G::DW; ++j) issue((uint32_t)j, (uint32_t)j);
        for (uint32_t c = 0; c < NC; ++c) {
            gemml_vmwait<(G::DW - 3) * G::LW>();  // chunks <= c + 2 are in
            gemml_barrier();
            issue(c + G::DW, (c + G::DW) % G::NW);
        }
        gemml_vmwait<0>();
        return;
    }
    if (wave >= 4) {
        // X copies: unit u (of the stage's 2 LX units) puts 16 bytes at stage
        // byte 1024 u + 16 lane = token row r, byte column b; the padding bytes
        // (b >= 128) take a copy of the row's first 16 bytes
        const uint32_t ub = (wave - 4u) * G::LX;
        uint32_t xo[G::LX];
#pragma unroll
        for (int q = 0; q < G::LX; ++q) {
            const uint32_t o = 1024u * (ub + q) + 16u * lane, r = o / ER_GEMML_XROWB, b = o % ER_GEMML_XROWB;
            xo[q] = min(t0 + r, T - 1u) * K * 2u + (b < 128u ? b : 0u);
        }
        auto issue = [&](uint32_t chunk, uint32_t slot) {
            chunk = min(chunk, NC - 1u);
            uint8_t *st = xs + slot * ER_GEMML_XSTAGE + 1024u * ub;
#pragma unroll
            for (int q = 0; q < G::LX; ++q)
                __builtin_amdgcn_global_load_lds((const void *)((const uint8_t *)X + xo[q] + 128u * chunk),
                                                 (void *)(st + 1024u * q), 16, 0, 0);
        };
#pragma unroll
        for (int j = 0; j < G::DX; ++j) issue((uint32_t)j, (uint32_t)j);
        gemml_vmwait<(G::DX - 1) * G::LX>();  // chunk 0 is in
        gemml_barrier();
        for (uint32_t c = 0; c < NC; ++c) {
            gemml_vmwait<(G::DX - 2) * G::LX>();  // chunks <= c + 1 are in
            gemml_barrier();
            issue(c + G::DX, (c + G::DX) % G::NX);
        }
        gemml_vmwait<0>();
        return;
    }

    // compute waves
    const uint32_t h = lane >> 5, l32 = lane & 31u;
    f32x16 acc[R][4];
#pragma unroll
    for (int f = 0; f < R; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[f][i][r] = 0.0f;
    // raw bytes of row 32 R wave + 32 f + l32 for `chunk` from its stage (sh =
    // chunk % 4, a constant at every call: the chunk loop is unrolled by 4)
    auto rawW = [&](uint32_t chunk, uint32_t sh, int f, WRaw &r) {
        const uint32_t rr = 32u * R * wave + 32u * (uint32_t)f + l32;
        const uint8_t *row = wsm + (chunk % G::NW) * G::WSTAGE + rr * G::WROWB;
        if (Q4K) {
            r.a = *(const u32x4 *)(hsm + ((chunk >> 2) % (uint32_t)G::NH) * G::HSTAGE + 16u * rr);
            r.b = *(const u32x4 *)(row + 16u * h);
            r.c = 0;
        } else {
            // blocks 2 chunk + h start at window byte 4 sh + 34 h; the 4-byte-aligned
            // 36-byte window dequant_w expects is dwords sh .. sh + 8 of the three
            // aligned 16-byte granules 2h .. 2h + 2, read whole: rows 80 bytes
            // apart put the 16 lanes of each read pass on distinct banks, where
            // dword reads of the window hit 16 of the 64 banks (4-way conflicts)
            const u32x4 *gp = (const u32x4 *)__builtin_assume_aligned(row + 32u * h, 16);
            const u32x4 g0 = gp[0], g1 = gp[1], g2 = gp[2];
            const uint32_t gd[12] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w, g2.x, g2.y, g2.z, g2.w};
            r.a = u32x4{gd[sh], gd[sh + 1], gd[sh + 2], gd[sh + 3]};
            r.b = u32x4{gd[sh + 4], gd[sh + 5], gd[sh + 6], gd[sh + 7]};
            r.c = gd[sh + 8];
        }
    };
    auto readA = [&](uint32_t chunk, int s, bf16x8 (&a)[4]) {
        const uint8_t *xst = xs + (chunk % G::NX) * ER_GEMML_XSTAGE;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            a[i] = *(const bf16x8 *)(xst + (32u * i + l32) * ER_GEMML_XROWB + 2u * gemml_acol(Q4K, s, h));
    };
    // Software pipeline, per chunk c and MFMA step s (one scheduling region
    // each): the LDS reads of the next step's X fragments (after step 3: the
    // next chunk's step 0 and the raw weights of chunk c + 2), then the
    // step's 8 MFMAs interleaved with the dequantisation of step s of chunk
    // c + 1.  B operands: wd[c % 2]; raw weights of chunk c + 1: rw[c % 2].
    uint32_t wd[2][R][16];
    WRaw rw[2][R];
    bf16x8 a[2][4];
    DqScale sc[R];
    gemml_barrier();  // X chunk 0 and weight chunks 0, 1 are in
#pragma unroll
    for (int f = 0; f < R; ++f) {
        WRaw r0;
        rawW(0u, 0u, f, r0);
        const DqScale q0 = dq_scale<Q4K>(r0, 0u, h);
#pragma unroll
        for (int s = 0; s < 4; ++s) dq_step<Q4K>(r0, q0, h, s, &wd[0][f][4 * s]);
        rawW(1u, 1u, f, rw[0][f]);
    }
    readA(0u, 0, a[0]);
    for (uint32_t c = 0; c < NC; c += 4u) {
#pragma unroll
        for (int Q = 0; Q < 4; ++Q) {
            const int P = Q & 1;
            const uint32_t cc = c + (uint32_t)Q;
            // NC is a multiple of 4 (K % 256 == 0), so cc < NC in every quarter
            gemml_barrier();  // X chunk cc + 1 and weight chunk cc + 2 are in
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if (s < 3) {
                    readA(cc, s + 1, a[(s + 1) & 1]);
                } else {
                    readA(cc + 1u, 0, a[0]);
#pragma unroll
                    for (int f = 0; f < R; ++f) rawW(cc + 2u, (uint32_t)((Q + 2) & 3), f, rw[P ^ 1][f]);
                }
                if (s == 0) {
#pragma unroll
                    for (int f = 0; f < R; ++f) sc[f] = dq_scale<Q4K>(rw[P][f], cc + 1u, h);
                }
#pragma unroll
                for (int f = 0; f < R; ++f) dq_step<Q4K>(rw[P][f], sc[f], h, s, &wd[P ^ 1][f][4 * s]);
#pragma unroll
                for (int f = 0; f < R; ++f) {
                    const bf16x8 b = __builtin_bit_cast(
                        bf16x8, u32x4{wd[P][f][4 * s], wd[P][f][4 * s + 1], wd[P][f][4 * s + 2], wd[P][f][4 * s + 3]});
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[f][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s & 1][i], b, acc[f][i], 0, 0, 0);
                }
                // reads first, then matrix instructions each followed by a share
                // of the dequantisation
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
                for (int m = 0; m < 4 * R; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (s == 0) __builtin_amdgcn_sched_group_barrier(0x002, 9, 0);
                    else __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    // Branch-free epilogue: an element outside Y (last tiles) is the exact
    // duplicate of the clamped element, because its X row and weight row were
    // copied clamped the same way, so a plain store of it writes the value
    // already there.  Offsets are 32-bit byte offsets from Y (host:
    // T * N * 4 < 2^32).
    uint32_t tl = t0 + 4u * h;
    asm volatile("" : "+v"(tl));
#pragma unroll
    for (int f = 0; f < R; ++f) {
        const uint32_t nc = min(n0 + 32u * R * wave + 32u * (uint32_t)f + l32, N - 1u);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t t = min(tl + 32u * (uint32_t)i + 8u * (uint32_t)(r >> 2) + (uint32_t)(r & 3), T - 1u);
                *(float *)((uint8_t *)Y + (t * N + nc) * 4u) = acc[f][i][r];
            }
    }
    if (STAMPED && threadIdx.x == 0) {
        const uint64_t rt1 = __builtin_amdgcn_s_memrealtime(), ct1 = __builtin_amdgcn_s_memtime();
        stamps[4u * item + 0u] = rt0;
        stamps[4u * item + 1u] = rt1;
        stamps[4u * item + 2u] = ct0;
        stamps[4u * item + 3u] = ct1;
    }
}

#define ER_GEMML_ENTRY(name, q4k, r)                                                                         \
    extern "C" __global__ void __launch_bounds__(512, 1)                                                     \
        name(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X, float *__restrict__ Y, uint32_t T, \
             uint32_t N, uint32_t K) {                                                                       \
        gemm_ls<q4k, r>(W, X, Y, T, N, K);                                                                   \
    }

ER_GEMML_ENTRY(er_gemml_q4k, true, 2)
ER_GEMML_ENTRY(er_gemml_q8_0, false, 2)
ER_GEMML_ENTRY(er_gemml_q4k_r1, true, 1)
ER_GEMML_ENTRY(er_gemml_q8_0_r1, false, 1)

#ifdef ER_WITH_PROBES
// measurement build: the same kernels with per-workgroup clock stamps
#define ER_GEMML_STAMPED_ENTRY(name, q4k, r)                                                                 \
    extern "C" __global__ void __launch_bounds__(512, 1)                                                     \
        name(const uint8_t *__restrict__ W, const uint16_t *__restrict__ X, float *__restrict__ Y, uint32_t T, \
             uint32_t N, uint32_t K, uint64_t *__restrict__ stamps) {                                        \
        gemm_ls<q4k, r, true>(W, X, Y, T, N, K, stamps);                                                     \
    }
ER_GEMML_STAMPED_ENTRY(er_gemml_q4k_stamped, true, 2)
ER_GEMML_STAMPED_ENTRY(er_gemml_q8_0_stamped, false, 2)
ER_GEMML_STAMPED_ENTRY(er_gemml_q4k_r1_stamped, true, 1)
ER_GEMML_STAMPED_ENTRY(er_gemml_q8_0_r1_stamped, false, 1)
#endif
