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
