// er_gemv.hip -- decode GEMV y[M] = W[M,K] . x[K] over raw GGUF blocks.
//
// Replaces q4_k_gemv_f32 (Dequant_Q4_K_M.metal:70-139), q6_k_gemv_f32
// (Dequant_Q6_K.metal:60-127), dequant_q8_0_gemv (Dequant_Q8_0.metal:86-141)
// and their token-batched forms (Dequant_Q4_K_M.metal:141-214,
// Dequant_Q8_0.metal:143-197).  Bandwidth-bound: no MFMA.
//
// Two kernel families:
//
// 1. Integer-dot kernels (Q4_K, Q6_K, and Q8_0 with K % 64 == 0): x is staged once
//    per workgroup as three int8 limbs per value (er_xlimbs.h) and every
//    weight x activation product is formed with v_dot4_i32_i8, exactly, in
//    int32.  A "slot" is 64 weights of one row: a Q4_K sub-block pair
//    (32 qs bytes + the block header), two Q8_0 blocks (68 bytes) or a
//    quarter of a Q6_K block (48 bytes of ql/qh, 4 scales, d).  A wave
//    is split into 64/LPR lane groups of LPR lanes; a group owns R rows and
//    each lane NS slots of each row.  Every weight load of a lane is issued
//    up front (after the L2-resident x loads, before x staging), and the
//    slots are consumed in issue order, so the wave computes on the first
//    slot while the rest are still in flight.
//
// 2. fp32 kernels (Q8_0 with an odd number of blocks per row; rows longer
//    than the integer kernels cover): x is staged in LDS as fp32, a
//    16-byte "slot" of raw bytes is unpacked in registers and accumulated
//    with fp32 FMAs.
//
// gridDim.y is the token count of the batched form: token t reads x + t*K and
// writes y + t*M (the reference's grid-y = token layout).
#include "er_gemv_cfg.h"
#include "er_nonfinite.h"
#include "er_xlimbs.h"

#ifndef ER_Q4K_ROWS
#define ER_Q4K_ROWS 4
#endif
#ifndef ER_Q6K_ROWS
#define ER_Q6K_ROWS 2
#endif
#ifndef ER_Q8_0_ROWS
#define ER_Q8_0_ROWS 2
#endif

#define ER_GEMV_THREADS 256

// ===========================================================================
// Family 1: integer-dot kernels
// ===========================================================================

// x chunks held in registers per thread: ceil(4*LPR*NS/256) (the x of one row
// slice of LPR*NS slots), at most 4; chunks beyond that are staged by
// xl_store_tail after the weight loads.
template <int LPR, int NS>
struct I8Cfg {
    static constexpr int G = 64 / LPR;
    static constexpr int XG0 = (4 * LPR * NS + 255) / 256;
    static constexpr int XG = XG0 < 1 ? 1 : (XG0 > 4 ? 4 : XG0);
};

// Q4_K slot s of a row = super-block s/4, sub-block pair p = s%4: header
// (d, dmin, 12 scale bytes) + qs bytes [32p, 32p+32) = weights 64s..64s+63
// (low nibbles: sub-block 2p, high nibbles: sub-block 2p+1).

// Per-lane constants of pair p for the scale / min byte extraction:
//   p < 2 : sc = s[2p..2p+1] & 63,   m = s[2p+4..2p+5] & 63
//   p >= 2: sc = (s[q+8] & 15) | (s[q] >> 6) << 4,  m = (s[q+8] >> 4) | (s[q+4] >> 6) << 4,
//           q = 2p - 4
struct Q4Sel {
    uint32_t sel1, sel2, maskLo, shM;
};
ER_DEV Q4Sel q4k_sel(uint32_t p) {
    const bool lowp = p < 2u;
    const uint32_t q4 = 2u * p - 4u;
    Q4Sel c;
    c.sel1 = lowp ? (0x0c0c0000u | ((2u * p + 1u) << 8) | (2u * p)) : (0x0c0c0000u | ((q4 + 5u) << 8) | (q4 + 4u));
    c.sel2 = lowp ? 0x0c0c0c0cu : (0x0c0c0000u | ((q4 + 1u) << 8) | q4);
    c.maskLo = lowp ? 0x3f3fu : 0x0f0fu;
    c.shM = lowp ? 0u : 4u;
    return c;
}

// Contribution of one slot (header h, qs qa|qb) against the staged x limbs xv
// of the same 64 positions: (d * s_g) * sum(sc * q * xi) - dmin * sum(m * X_sub).
ER_DEV float q4k_slot_dot(const u32x4 &h, const u32x4 &qa, const u32x4 &qb,
                          const u32x4 (&xv)[ER_XL_PLANES][4], float XL, float XH, float sg, float live,
                          const Q4Sel &c, uint32_t M0F) {
    const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    // low nibbles: positions 4k..4k+3 of sub-block 2p (granule k/4);
    // high nibbles: the same positions of sub-block 2p+1 (granule 2 + k/4)
    int cL[ER_XL_PLANES] = {}, cH[ER_XL_PLANES] = {};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int lo = (int)(qw[k] & M0F);
        const int hi = (int)((qw[k] >> 4) & M0F);
#pragma unroll
        for (int l = 0; l < ER_XL_PLANES; ++l) {
            cL[l] = sdot4_acc(lo, (int)xv[l][k >> 2][k & 3], cL[l], k == 0);
            cH[l] = sdot4_acc(hi, (int)xv[l][2 + (k >> 2)][k & 3], cH[l], k == 0);
        }
    }
    const float T0 = xl_combine(cL[0], cL[1], cL[2]);
    const float T1 = xl_combine(cH[0], cH[1], cH[2]);
    // perm(S0, S1, sel): selector bytes 0-3 pick S1, 4-7 pick S0
    const uint32_t X1 = __builtin_amdgcn_perm(h.w, h.y, c.sel1);
    const uint32_t X2 = __builtin_amdgcn_perm(h.w, h.y, c.sel2);
    const uint32_t sc = (X1 & c.maskLo) | ((X2 >> 2) & 0x3030u);
    const uint32_t Y1 = __builtin_amdgcn_perm(h.w, h.z, c.sel1);
    const uint32_t Y2 = __builtin_amdgcn_perm(h.w, h.z, c.sel2);
    const uint32_t mm = ((Y1 >> c.shM) & c.maskLo) | ((Y2 >> 2) & 0x3030u);
    const float d = f16_to_f32(h.x & 0xffffu), dmin = f16_to_f32(h.x >> 16);
    const float sT = __builtin_fmaf(ub0(sc), T0, ub1(sc) * T1);
    const float mX = __builtin_fmaf(ub0(mm), XL, ub1(mm) * XH);
    return __builtin_fmaf(d * sg, sT, -(live * dmin) * mX);
}

// Output epilogues of the row-list kernel.
#define ER_EPI_STORE 0  // every row r writes yrow[r]
#define ER_EPI_GEGLU 1  // rows [0, R/2) are gate rows, [R/2, R) the matching up rows:
                        // writes gelu_tanh(gate) * up to the gate row's output

// GELU, tanh approximation, saturated outside [-10, 10] (as the reference's
// q4_k_gelu_tanh, Dequant_Q4_K_M.metal:913-923).
ER_DEV float gelu_tanh(float g) {
    if (g > 10.0f) return g;
    if (g < -10.0f) return 0.0f;
    const float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    return g * 0.5f * (1.0f + tanhf(inner));
}

// Integer-dot Q4_K GEMV over the R rows (given by pointer) of this thread's
// lane group; x is staged by the whole workgroup.  Every lane of the
// workgroup must call it (it contains a barrier).
// rowAt(lane, r): row r of lane `lane`'s group, recomputed for the
// non-finite path so that no row pointer stays live across the dot products.
template <int LPR, int NS, int R, int EPI, class RowAt>
ER_DEV void gemv_q4k_i8_core(const uint8_t *const (&rowp)[R], float *const (&yrow)[R], const bool (&rowLive)[R],
                             const float *__restrict__ x, uint32_t K, RowAt rowAt) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    __shared__ float4 chkw[ER_GEMV_WAVES];  // the waves' shares of the launch's checks
    using C = I8Cfg<LPR, NS>;
    constexpr uint32_t NT = 64u * ER_GEMV_WAVES;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t li = lane % LPR;
    const uint32_t S = K >> 6;

    float4 xr[C::XG][4];
    xl_load<C::XG, NT>(x, K, xr);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 hdr[NS][R], qa[NS][R], qb[NS][R];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const uint32_t s = min(li + (uint32_t)LPR * j, S - 1u);
        const uint32_t p = s & 3u;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *bp = rowp[r] + (s >> 2) * 144u;
            hdr[j][r] = ld16_a16(bp);
            qa[j][r] = ld16_a16(bp + 16u + 32u * p);
            qb[j][r] = ld16_a16(bp + 32u + 32u * p);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    XlCheck ck;
    xl_store<C::XG, NT>(lds, K, xr, &ck);
    xl_store_tail<C::XG, NT>(x, lds, K, &ck);
    {  // this wave's share of the launch's checks, gathered by the conversion
        const float4 sh = xl_check_share(ck);
        if ((threadIdx.x & 63u) == 0) chkw[threadIdx.x >> 6] = sh;
    }
    __syncthreads();
    // the launch's check decisions, read while the first weights are in flight
    bool ill, nfx;
    xl_check_decide(chkw, ER_GEMV_WAVES, 4.0f, ill, nfx);
    __builtin_amdgcn_sched_barrier(0);

    const XLimbs X = xl_view(lds, K);
    const uint32_t M0F = vreg_const(0x0f0f0f0fu);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const uint32_t sRaw = li + (uint32_t)LPR * j;
        const uint32_t s = min(sRaw, S - 1u);
        const float live = sRaw < S ? 1.0f : 0.0f;
        u32x4 xv[ER_XL_PLANES][4];
        xl_read_group(X, s, xv);
        const float4 c16 = *(const float4 *)__builtin_assume_aligned(X.x16 + 4u * s, 16);
        const float XL = c16.x + c16.y, XH = c16.z + c16.w;
        const float sg = live * X.sg64[s];
        const Q4Sel sel = q4k_sel(s & 3u);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] += q4k_slot_dot(hdr[j][r], qa[j][r], qb[j][r], xv, XL, XH, sg, live, sel, M0F);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<LPR>(acc[r]);
    if (ill || nfx) {
        float sp[R], hits = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sp[r] = 0.0f;
        const uint32_t ln = lane_id();
        nf_terms<R>([&](int r, uint32_t k) { return q4k_weight_at(rowAt(ln, r), k); },
                    [&](uint32_t k) { return x[k]; }, X.x16, K >> 4, ln % LPR, LPR, sp, hits, ill);
        hits = group_sum<LPR>(hits);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = group_sum<LPR>(sp[r]);
            acc[r] = hits > 0.0f ? v : acc[r];
        }
    }
    if (li == 0) {
        if (EPI == ER_EPI_GEGLU) {
#pragma unroll
            for (int r = 0; r < R / 2; ++r)
                if (rowLive[r]) *yrow[r] = gelu_tanh(acc[r]) * acc[R / 2 + r];
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (rowLive[r]) *yrow[r] = acc[r];
        }
    }
}

template <int LPR, int NS, int R>
ER_DEV void gemv_q4k_i8(const uint8_t *__restrict__ W, const float *__restrict__ x,
                        float *__restrict__ y, uint32_t M, uint32_t K) {
    using C = I8Cfg<LPR, NS>;
    x += (size_t)blockIdx.y * K;
    y += (size_t)blockIdx.y * M;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR;
    const size_t rowBytes = (size_t)(K >> 8) * 144u;
    const uint32_t row0 = ((blockIdx.x * ER_GEMV_WAVES + wave) * C::G + g) * (uint32_t)R;
    const uint32_t waveS = __builtin_amdgcn_readfirstlane(wave);
    auto rowAt = [=](uint32_t ln, int r) {
        const uint32_t row = ((blockIdx.x * ER_GEMV_WAVES + waveS) * C::G + ln / LPR) * (uint32_t)R + (uint32_t)r;
        return W + (size_t)min(row, M - 1u) * rowBytes;
    };
    const uint8_t *rowp[R];
    float *yrow[R];
    bool live[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = min(row0 + (uint32_t)r, M - 1u);
        rowp[r] = W + (size_t)row * rowBytes;
        yrow[r] = y + row;
        live[r] = row0 + (uint32_t)r < M;
    }
    gemv_q4k_i8_core<LPR, NS, R, ER_EPI_STORE>(rowp, yrow, live, x, K, rowAt);
}

// Several Q4_K matrices sharing one x and K (the reference's dual / triple
// projections, q4_k_gemv_dual_f32 / q4_k_gemv_three_f32,
// Dequant_Q4_K_M.metal:704-803, 1024-1202): rows of A, B, C are concatenated
// into one row space; a lane group's R rows may cross a matrix boundary.
// One of three values by index, taken as values.  Indexing a kernel-argument
// array with a per-lane index (mm.W[m]), or a conditional on struct members
// themselves (which selects their addresses), makes every lane load the value
// through the vector memory path -- behind any loads already in flight -- or
// puts the struct in scratch; the three values here are uniform loads
// (scalar registers) and the choice a per-lane select.
template <class T>
__device__ __forceinline__ T pick3(uint32_t m, T a, T b, T c) {
    T v = a;
    v = m == 1u ? b : v;
    v = m == 2u ? c : v;
    return v;
}
template <class T>
__device__ __forceinline__ T pick2(bool second, T a, T b) {
    return second ? b : a;
}

struct Q4Multi {
    const uint8_t *W[3];
    float *y[3];
    uint32_t M[3];
};

template <int LPR, int NS, int R>
ER_DEV void gemv_q4k_i8_multi(const Q4Multi &mm, const float *__restrict__ x, uint32_t K) {
    using C = I8Cfg<LPR, NS>;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR;
    const size_t rowBytes = (size_t)(K >> 8) * 144u;
    const uint32_t Mt = mm.M[0] + mm.M[1] + mm.M[2];
    const uint32_t row0 = ((blockIdx.x * ER_GEMV_WAVES + wave) * C::G + g) * (uint32_t)R;
    const uint32_t waveS = __builtin_amdgcn_readfirstlane(wave);
    auto rowAt = [&](uint32_t ln, int r) {
        uint32_t v = min(((blockIdx.x * ER_GEMV_WAVES + waveS) * C::G + ln / LPR) * (uint32_t)R + (uint32_t)r, Mt - 1u);
        const uint8_t *base = mm.W[0];
        if (v >= mm.M[0]) {
            v -= mm.M[0];
            base = mm.W[1];
            if (v >= mm.M[1]) {
                v -= mm.M[1];
                base = mm.W[2];
            }
        }
        return base + (size_t)v * rowBytes;
    };
    const uint8_t *rowp[R];
    float *yrow[R];
    bool live[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        uint32_t v = min(row0 + (uint32_t)r, Mt - 1u);
        int m = 0;
        if (v >= mm.M[0]) {
            v -= mm.M[0];
            m = 1;
            if (v >= mm.M[1]) {
                v -= mm.M[1];
                m = 2;
            }
        }
        rowp[r] = pick3((uint32_t)m, mm.W[0], mm.W[1], mm.W[2]) + (size_t)v * rowBytes;
        yrow[r] = pick3((uint32_t)m, mm.y[0], mm.y[1], mm.y[2]) + v;
        live[r] = row0 + (uint32_t)r < Mt;
    }
    gemv_q4k_i8_core<LPR, NS, R, ER_EPI_STORE>(rowp, yrow, live, x, K, rowAt);
}

// Fused gate/up GeGLU (q4_k_gemv_dual_geglu_f32, Dequant_Q4_K_M.metal:925-1022):
// y[r] = gelu_tanh(gate[r] . x) * (up[r] . x).  A lane group owns R/2 output
// rows and computes the gate and up dot products of each in the same lanes.
template <int LPR, int NS, int R>
ER_DEV void gemv_q4k_i8_geglu(const uint8_t *__restrict__ Wg, const uint8_t *__restrict__ Wu,
                              const float *__restrict__ x, float *__restrict__ y, uint32_t M, uint32_t K) {
    static_assert(R % 2 == 0, "GeGLU pairs gate and up rows");
    using C = I8Cfg<LPR, NS>;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR;
    const size_t rowBytes = (size_t)(K >> 8) * 144u;
    const uint32_t row0 = ((blockIdx.x * ER_GEMV_WAVES + wave) * C::G + g) * (uint32_t)(R / 2);
    const uint32_t waveS = __builtin_amdgcn_readfirstlane(wave);
    auto rowAt = [=](uint32_t ln, int r) {
        const uint32_t row = ((blockIdx.x * ER_GEMV_WAVES + waveS) * C::G + ln / LPR) * (uint32_t)(R / 2) +
                             (uint32_t)(r % (R / 2));
        return (r < R / 2 ? Wg : Wu) + (size_t)min(row, M - 1u) * rowBytes;
    };
    const uint8_t *rowp[R];
    float *yrow[R];
    bool live[R];
#pragma unroll
    for (int r = 0; r < R / 2; ++r) {
        const uint32_t row = min(row0 + (uint32_t)r, M - 1u);
        rowp[r] = Wg + (size_t)row * rowBytes;
        rowp[R / 2 + r] = Wu + (size_t)row * rowBytes;
        yrow[r] = yrow[R / 2 + r] = y + row;
        live[r] = live[R / 2 + r] = row0 + (uint32_t)r < M;
    }
    gemv_q4k_i8_core<LPR, NS, R, ER_EPI_GEGLU>(rowp, yrow, live, x, K, rowAt);
}

// Q8_0 with K % 64 == 0: slot s = blocks 2s, 2s+1 = row bytes [68s, 68s+68)
// (4-byte aligned).  Dwords v0..v16: block A d = v0[15:0], qs = bytes 2..33
// (realigned by 2 bytes), block B d = v8[31:16], qs = v9..v16.  The int8 qs
// bytes feed v_dot4_i32_i8 as they are.
struct Q8Slot {
    u32x4 v0, v1, v2, v3;
    uint32_t v4;
};

ER_DEV Q8Slot q8_slot_load(const uint8_t *p) {
    return Q8Slot{ld16_a4(p), ld16_a4(p + 16), ld16_a4(p + 32), ld16_a4(p + 48), ld4_a4(p + 64)};
}

// acc + sg * (dA * (qA . x) + dB * (qB . x)) over the slot's 64 weights.
// Z0: start the limb chains with sdot4_0 (off where the VOP3P form's
// registers tipped kernels holding 8 slots of weights into spilling).
template <bool Z0 = true>
ER_DEV float q8_slot_dot(const Q8Slot &w, const u32x4 (&xv)[ER_XL_PLANES][4], float sg, float acc) {
    const uint32_t v[17] = {w.v0.x, w.v0.y, w.v0.z, w.v0.w, w.v1.x, w.v1.y, w.v1.z, w.v1.w, w.v2.x,
                            w.v2.y, w.v2.z, w.v2.w, w.v3.x, w.v3.y, w.v3.z, w.v3.w, w.v4};
    int cA[ER_XL_PLANES] = {}, cB[ER_XL_PLANES] = {};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int qa = (int)alignbyte(v[k + 1], v[k], 2);
        const int qb = (int)v[9 + k];
#pragma unroll
        for (int l = 0; l < ER_XL_PLANES; ++l) {
            cA[l] = sdot4_acc(qa, (int)xv[l][k >> 2][k & 3], cA[l], Z0 && k == 0);
            cB[l] = sdot4_acc(qb, (int)xv[l][2 + (k >> 2)][k & 3], cB[l], Z0 && k == 0);
        }
    }
    const float TA = xl_combine(cA[0], cA[1], cA[2]);
    const float TB = xl_combine(cB[0], cB[1], cB[2]);
    const float dA = f16_to_f32(v[0] & 0xffffu), dB = f16_to_f32(v[8] >> 16);
    const float a = __builtin_fmaf(sg * dA, TA, acc);
    return __builtin_fmaf(sg * dB, TB, a);
}

template <int LPR, int NS, int R>
ER_DEV void gemv_q8_0_i8(const uint8_t *__restrict__ W, const float *__restrict__ x,
                         float *__restrict__ y, uint32_t M, uint32_t K) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    __shared__ float4 chkw[ER_GEMV_WAVES];  // the waves' shares of the launch's checks
    using C = I8Cfg<LPR, NS>;
    constexpr uint32_t NT = 64u * ER_GEMV_WAVES;
    x += (size_t)blockIdx.y * K;
    y += (size_t)blockIdx.y * M;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR, li = lane % LPR;
    const uint32_t S = K >> 6;
    const size_t rowBytes = (size_t)S * 68u;
    const uint32_t row0 = ((blockIdx.x * ER_GEMV_WAVES + wave) * C::G + g) * (uint32_t)R;
    const uint32_t waveS = __builtin_amdgcn_readfirstlane(wave);

    float4 xr[C::XG][4];
    xl_load<C::XG, NT>(x, K, xr);
    __builtin_amdgcn_sched_barrier(0);
    Q8Slot w[NS][R];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const uint32_t s = min(li + (uint32_t)LPR * j, S - 1u);
#pragma unroll
        for (int r = 0; r < R; ++r)
            w[j][r] = q8_slot_load(W + (size_t)min(row0 + (uint32_t)r, M - 1u) * rowBytes + (size_t)s * 68u);
    }
    __builtin_amdgcn_sched_barrier(0);
    XlCheck ck;
    xl_store<C::XG, NT>(lds, K, xr, &ck);
    xl_store_tail<C::XG, NT>(x, lds, K, &ck);
    {  // this wave's share of the launch's checks, gathered by the conversion
        const float4 sh = xl_check_share(ck);
        if ((threadIdx.x & 63u) == 0) chkw[threadIdx.x >> 6] = sh;
    }
    __syncthreads();
    // the launch's check decisions, read while the first weights are in flight
    bool ill, nfx;
    xl_check_decide(chkw, ER_GEMV_WAVES, 1.0f, ill, nfx);
    __builtin_amdgcn_sched_barrier(0);

    const XLimbs X = xl_view(lds, K);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const uint32_t sRaw = li + (uint32_t)LPR * j;
        const uint32_t s = min(sRaw, S - 1u);
        const float sg = sRaw < S ? X.sg64[s] : 0.0f;
        u32x4 xv[ER_XL_PLANES][4];
        xl_read_group(X, s, xv);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = q8_slot_dot<(NS * R < 8)>(w[j][r], xv, sg, acc[r]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<LPR>(acc[r]);
    if (ill || nfx) {
        float sp[R], hits = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sp[r] = 0.0f;
        const uint32_t ln = lane_id();
        const uint32_t fr0 = ((blockIdx.x * ER_GEMV_WAVES + waveS) * C::G + ln / LPR) * (uint32_t)R;
        nf_terms<R>([&](int r, uint32_t k) {
                        return q8_0_weight_at(W + (size_t)min(fr0 + (uint32_t)r, M - 1u) * rowBytes, k);
                    },
                    [&](uint32_t k) { return x[k]; }, X.x16, K >> 4, ln % LPR, LPR, sp, hits, ill);
        hits = group_sum<LPR>(hits);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = group_sum<LPR>(sp[r]);
            acc[r] = hits > 0.0f ? v : acc[r];
        }
    }
    if (li == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + (uint32_t)r < M) y[row0 + r] = acc[r];
    }
}

// ---------------------------------------------------------------------------
// Fused Q8_0 projections (the reference's Dequant_Q8_0.metal:199-586):
// dequant_q8_0_fused_qkv, _fused_final_norm_gemv, _gemv_f16out, _gemv_add
// (row-list kernel below) and _fused_gate_up_silu (pair kernel).
//
// RMSNorm prologue (when normW is set): the workgroup sums x^2 over the
// token's row of x while the weight loads are in flight, then stages
// x * (1 / sqrt(sum / K + eps)) * normW instead of x, as
// normed = x * rmsScale * normWeight (Dequant_Q8_0.metal:275-286).  The
// configurations used hold the whole of x in registers (LPR * NS * 64 >= K,
// so XG * 4096 >= K): no chunk is staged outside the normalised set.

#define ER_EPI_Q8_ROWS 0  // per row: + residual (optional), fp32 or fp16 store
#define ER_EPI_Q8_SILU 1  // rows [0, R/2) gate, [R/2, R) up: silu(gate) * up

ER_DEV float silu(float g) { return g / (1.0f + expf(-g)); }

// rowAt(lane, r): as in gemv_q4k_i8_core.
template <int LPR, int NS, int R, int EPI, class RowAt>
ER_DEV void gemv_q8_0_i8_fused_core(const uint8_t *const (&rowp)[R], void *const (&yrow)[R],
                                    const bool (&rowLive)[R], const bool (&rowHalf)[R],
                                    const float *const (&rowRes)[R], const float *__restrict__ x,
                                    const float *__restrict__ normW, float eps, uint32_t K, RowAt rowAt) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    __shared__ float red[ER_GEMV_WAVES];
    __shared__ float4 chkw[ER_GEMV_WAVES];  // the waves' shares of the launch's checks
    using C = I8Cfg<LPR, NS>;
    constexpr uint32_t NT = 64u * ER_GEMV_WAVES;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t li = lane % LPR;
    const uint32_t S = K >> 6, C16 = K >> 4;

    float4 xr[C::XG][4], wr[C::XG][4];
    xl_load<C::XG, NT>(x, K, xr);
    if (normW) xl_load<C::XG, NT>(normW, K, wr);
    __builtin_amdgcn_sched_barrier(0);
    Q8Slot w[NS][R];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const uint32_t s = min(li + (uint32_t)LPR * j, S - 1u);
#pragma unroll
        for (int r = 0; r < R; ++r) w[j][r] = q8_slot_load(rowp[r] + (size_t)s * 68u);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (normW) {
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < C::XG; ++c)
            if (threadIdx.x + NT * (uint32_t)c < C16)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    ss += xr[c][q].x * xr[c][q].x + xr[c][q].y * xr[c][q].y + xr[c][q].z * xr[c][q].z +
                          xr[c][q].w * xr[c][q].w;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        ss = 0.0f;
#pragma unroll
        for (int k = 0; k < ER_GEMV_WAVES; ++k) ss += red[k];
        const float rms = 1.0f / __builtin_sqrtf(ss / (float)K + eps);
#pragma unroll
        for (int c = 0; c < C::XG; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                xr[c][q].x = xr[c][q].x * rms * wr[c][q].x;
                xr[c][q].y = xr[c][q].y * rms * wr[c][q].y;
                xr[c][q].z = xr[c][q].z * rms * wr[c][q].z;
                xr[c][q].w = xr[c][q].w * rms * wr[c][q].w;
            }
    }
    XlCheck ck;
    xl_store<C::XG, NT>(lds, K, xr, &ck);
    {  // this wave's share of the launch's checks, gathered by the conversion
        const float4 sh = xl_check_share(ck);
        if ((threadIdx.x & 63u) == 0) chkw[threadIdx.x >> 6] = sh;
    }
    __syncthreads();
    // the launch's check decisions, read while the first weights are in flight
    bool ill, nfx;
    xl_check_decide(chkw, ER_GEMV_WAVES, 1.0f, ill, nfx);
    __builtin_amdgcn_sched_barrier(0);

    const XLimbs X = xl_view(lds, K);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const uint32_t sRaw = li + (uint32_t)LPR * j;
        const uint32_t s = min(sRaw, S - 1u);
        const float sg = sRaw < S ? X.sg64[s] : 0.0f;
        u32x4 xv[ER_XL_PLANES][4];
        xl_read_group(X, s, xv);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = q8_slot_dot<(NS * R < 8)>(w[j][r], xv, sg, acc[r]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<LPR>(acc[r]);
    if (ill || nfx) {
        // the staged values: x, or x * rms * normW as the prologue formed them
        // (rms recomputed from the same wave sums, so it is the same value)
        float rms = 1.0f;
        if (normW) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < ER_GEMV_WAVES; ++k) ss += red[k];
            rms = 1.0f / __builtin_sqrtf(ss / (float)K + eps);
        }
        float sp[R], hits = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sp[r] = 0.0f;
        const uint32_t ln = lane_id();
        nf_terms<R>([&](int r, uint32_t k) { return q8_0_weight_at(rowAt(ln, r), k); },
                    [&](uint32_t k) { return normW ? x[k] * rms * normW[k] : x[k]; }, X.x16, C16, ln % LPR, LPR,
                    sp, hits, ill);
        hits = group_sum<LPR>(hits);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = group_sum<LPR>(sp[r]);
            acc[r] = hits > 0.0f ? v : acc[r];
        }
    }
    if (li != 0) return;
    if constexpr (EPI == ER_EPI_Q8_SILU) {
#pragma unroll
        for (int r = 0; r < R / 2; ++r)
            if (rowLive[r]) *(float *)yrow[r] = silu(acc[r]) * acc[R / 2 + r];
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (!rowLive[r]) continue;
            const float v = rowRes[r] ? acc[r] + *rowRes[r] : acc[r];
            if (rowHalf[r])
                *(_Float16 *)yrow[r] = (_Float16)v;
            else
                *(float *)yrow[r] = v;
        }
    }
}

// Up to three Q8_0 matrices sharing x and K, rows concatenated (Q | K | V);
// token t = blockIdx.y reads x + t K and writes row i of matrix m at
// y[m] + t M[m] + i (fp16 when bit m of halfMask is set), adding
// res[m][t M[m] + i] when res[m] is set.
struct Q8Multi {
    const uint8_t *W[3];
    void *y[3];
    const float *res[3];
    uint32_t M[3];
    uint32_t halfMask;
    const float *normW;
    float eps;
};

template <int LPR, int NS, int R>
ER_DEV void gemv_q8_0_i8_multi(const Q8Multi &mm, const float *__restrict__ x, uint32_t K) {
    using C = I8Cfg<LPR, NS>;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR;
    const uint32_t t = blockIdx.y;
    const size_t rowBytes = (size_t)(K >> 6) * 68u;
    const uint32_t Mt = mm.M[0] + mm.M[1] + mm.M[2];
    const uint32_t row0 = ((blockIdx.x * ER_GEMV_WAVES + wave) * C::G + g) * (uint32_t)R;
    const uint32_t waveS = __builtin_amdgcn_readfirstlane(wave);
    auto rowAt = [&](uint32_t ln, int r) {
        uint32_t v = min(((blockIdx.x * ER_GEMV_WAVES + waveS) * C::G + ln / LPR) * (uint32_t)R + (uint32_t)r, Mt - 1u);
        const uint8_t *base = mm.W[0];
        if (v >= mm.M[0]) {
            v -= mm.M[0];
            base = mm.W[1];
            if (v >= mm.M[1]) {
                v -= mm.M[1];
                base = mm.W[2];
            }
        }
        return base + (size_t)v * rowBytes;
    };
    const uint8_t *rowp[R];
    void *yrow[R];
    bool live[R], half[R];
    const float *res[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        uint32_t v = min(row0 + (uint32_t)r, Mt - 1u);
        int m = 0;
        if (v >= mm.M[0]) {
            v -= mm.M[0];
            m = 1;
            if (v >= mm.M[1]) {
                v -= mm.M[1];
                m = 2;
            }
        }
        const uint32_t mu = (uint32_t)m;
        const size_t out = (size_t)t * pick3(mu, mm.M[0], mm.M[1], mm.M[2]) + v;
        rowp[r] = pick3(mu, mm.W[0], mm.W[1], mm.W[2]) + (size_t)v * rowBytes;
        half[r] = (mm.halfMask >> m) & 1u;
        yrow[r] = (uint8_t *)pick3(mu, mm.y[0], mm.y[1], mm.y[2]) + out * (half[r] ? 2u : 4u);
        const float *rp = pick3(mu, mm.res[0], mm.res[1], mm.res[2]);
        res[r] = rp ? rp + out : nullptr;
        live[r] = row0 + (uint32_t)r < Mt;
    }
    gemv_q8_0_i8_fused_core<LPR, NS, R, ER_EPI_Q8_ROWS>(rowp, yrow, live, half, res, x + (size_t)t * K,
                                                         mm.normW, mm.eps, K, rowAt);
}

// Gate/up pairs: y[t M + i] = silu(gate_i . n) * (up_i . n), n = RMSNorm(x_t)
// (dequant_q8_0_fused_gate_up_silu, Dequant_Q8_0.metal:410-500).
template <int LPR, int NS, int R>
ER_DEV void gemv_q8_0_i8_silu(const uint8_t *__restrict__ Wg, const uint8_t *__restrict__ Wu,
                              const float *__restrict__ x, float *__restrict__ y,
                              const float *__restrict__ normW, float eps, uint32_t M, uint32_t K) {
    static_assert(R % 2 == 0, "SiLU pairs gate and up rows");
    using C = I8Cfg<LPR, NS>;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR;
    const uint32_t t = blockIdx.y;
    const size_t rowBytes = (size_t)(K >> 6) * 68u;
    const uint32_t row0 = ((blockIdx.x * ER_GEMV_WAVES + wave) * C::G + g) * (uint32_t)(R / 2);
    const uint32_t waveS = __builtin_amdgcn_readfirstlane(wave);
    auto rowAt = [=](uint32_t ln, int r) {
        const uint32_t row = ((blockIdx.x * ER_GEMV_WAVES + waveS) * C::G + ln / LPR) * (uint32_t)(R / 2) +
                             (uint32_t)(r % (R / 2));
        return (r < R / 2 ? Wg : Wu) + (size_t)min(row, M - 1u) * rowBytes;
    };
    const uint8_t *rowp[R];
    void *yrow[R];
    bool live[R], half[R];
    const float *res[R];
#pragma unroll
    for (int r = 0; r < R / 2; ++r) {
        const uint32_t row = min(row0 + (uint32_t)r, M - 1u);
        rowp[r] = Wg + (size_t)row * rowBytes;
        rowp[R / 2 + r] = Wu + (size_t)row * rowBytes;
        yrow[r] = yrow[R / 2 + r] = y + (size_t)t * M + row;
        live[r] = live[R / 2 + r] = row0 + (uint32_t)r < M;
        half[r] = half[R / 2 + r] = false;
        res[r] = res[R / 2 + r] = nullptr;
    }
    gemv_q8_0_i8_fused_core<LPR, NS, R, ER_EPI_Q8_SILU>(rowp, yrow, live, half, res, x + (size_t)t * K,
                                                         normW, eps, K, rowAt);
}

// ---------------------------------------------------------------------------
// Greedy top-1 over a Q6_K head (the reference's q6_k_gemv_packed_4row_top1_f32
// + q6_k_top1_reduce, Dequant_Q6_K.metal:196-365).  Selection rule, kept
// exactly: each 4-row quad's candidate is row 4t, replaced by a later row of
// the quad only when strictly larger (so a NaN in row 4t makes the quad's
// candidate NaN); candidates then merge from (-inf, 0), a candidate winning
// when larger, or equal with a lower row index.  That merge is the minimum
// under the order (-value, index) with NaN candidates never taken, so the
// result does not depend on how the merge tree is shaped: each workgroup
// merges its quads into one (value, row) partial, and er_top1_reduce merges
// the partials.

// (v, i) <- (ov, oi) when ov is larger, or equal with a lower index.
ER_DEV void top1_merge(float &v, uint32_t &i, float ov, uint32_t oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

// (v, i) merged with the pair of the lane that CTRL selects, on the rows of
// ROWMASK (other rows merge with their own pair, which changes nothing).
template <int CTRL, int ROWMASK = 0xf>
ER_DEV void top1_dpp_merge(float &v, uint32_t &i) {
    const int vb = __float_as_int(v);
    const float ov = __int_as_float(__builtin_amdgcn_update_dpp(vb, vb, CTRL, ROWMASK, 0xf, false));
    const uint32_t oi = (uint32_t)__builtin_amdgcn_update_dpp((int)i, (int)i, CTRL, ROWMASK, 0xf, false);
    top1_merge(v, i, ov, oi);
}

// Merge over the 64 lanes of pairs that are never NaN (each started from
// (-inf, 0) and takes no NaN), where the merge is order-independent: DPP
// steps as in group_sum leave the result in lane 63, read back into all lanes.
ER_DEV void top1_wave_merge(float &v, uint32_t &i) {
    top1_dpp_merge<ER_DPP_QUAD_XOR1>(v, i);
    top1_dpp_merge<ER_DPP_QUAD_XOR2>(v, i);
    top1_dpp_merge<ER_DPP_ROW_HALF_MIRROR>(v, i);
    top1_dpp_merge<ER_DPP_ROW_MIRROR>(v, i);
    top1_dpp_merge<ER_DPP_ROW_BCAST15, 0xa>(v, i);  // rows 1 and 3 hold the two half-wave results
    top1_dpp_merge<ER_DPP_ROW_BCAST31, 0xc>(v, i);  // row 3 holds the total
    v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    i = (uint32_t)__builtin_amdgcn_readlane((int)i, 63);
}

// Wave 0 of the workgroup: the quads of local rows [0, 4 * nq), whose values
// are tv[0 .. 4 * nq) and whose global rows are rowOf(l) (consecutive within
// a quad), merged into the partial (pv, pi)[blockIdx.x]; quads at rows >= M
// are skipped.
template <class RowOf>
ER_DEV void top1_partial(const float *tv, uint32_t nq, uint32_t M, RowOf rowOf, float *__restrict__ pv,
                         uint32_t *__restrict__ pi) {
    if (threadIdx.x < 64u) {
        float bv = -__builtin_inff();
        uint32_t bi = 0;
        for (uint32_t q = threadIdx.x; q < nq; q += 64u) {
            const uint32_t r0 = rowOf(4u * q);
            if (r0 >= M) continue;
            float v = tv[4u * q];
            uint32_t i = r0;
#pragma unroll
            for (uint32_t k = 1; k < 4; ++k)
                if (tv[4u * q + k] > v) {
                    v = tv[4u * q + k];
                    i = r0 + k;
                }
            top1_merge(bv, bi, v, i);
        }
        top1_wave_merge(bv, bi);
        if (threadIdx.x == 0) {
            pv[blockIdx.x] = bv;
            pi[blockIdx.x] = bi;
        }
    }
}

// Workgroup epilogue: RPW row values of this workgroup (rows blockIdx.x * RPW
// + [0, RPW), RPW a multiple of 4, M a multiple of 4) -> partial
// (pv, pi)[blockIdx.x].  `mine` lanes hold acc[0..R) for local rows
// base + [0, R).
template <uint32_t RPW>
ER_DEV void top1_epilogue(const float *acc, int R, uint32_t base, bool mine, uint32_t M,
                          float *__restrict__ pv, uint32_t *__restrict__ pi) {
    __shared__ float tv[RPW];
    if (mine)
        for (int r = 0; r < R; ++r) tv[base + (uint32_t)r] = acc[r];
    __syncthreads();
    const uint32_t first = blockIdx.x * RPW;
    top1_partial(tv, min(RPW, M - first) / 4u, M, [&](uint32_t l) { return first + l; }, pv, pi);
}

// One workgroup of 256 lanes: merges `count` partials into out[0].
extern "C" __global__ void __launch_bounds__(256)
    er_top1_reduce(const float *__restrict__ pv, const uint32_t *__restrict__ pi,
                   uint32_t *__restrict__ out, uint32_t count) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    float bv = -__builtin_inff();
    uint32_t bi = 0;
    for (uint32_t t = threadIdx.x; t < count; t += 256u) top1_merge(bv, bi, pv[t], pi[t]);
    top1_wave_merge(bv, bi);
    if ((threadIdx.x & 63u) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        bv = sv[0];
        bi = si[0];
        for (int w = 1; w < 4; ++w) top1_merge(bv, bi, sv[w], si[w]);
        out[0] = bi;
    }
}

// Q6_K slot s of a row = super-block b = s/4, half h = (s/2)%2, lane chunk
// c = s%2: ql bytes [64h+16c, +16) (q1 low / q3 high nibbles) and
// [64h+32+16c, +16) (q2 / q4), qh bytes [128+32h+16c, +16) (2 high bits of
// q1..q4), scales sc[8h+2m+c] (m = 0..3) and d.  Its weights are positions
// 256b + 128h + 32m + 16c + [0, 16): x granules G0 + 2m with G0 = 16b+8h+c,
// 64-groups 4b+2h (m < 2) and 4b+2h+1.  Blocks are 2-byte aligned: the
// fields are fetched with one 2-byte-aligned vector load each (ld16_u2 /
// ld8_u2): 5 loads per slot and row, so with R = 4 rows the x loads issued
// before them stay within the 63 outstanding loads a wave can count, and the
// x conversion waits for x alone.  (4-byte-aligned windows plus a realigning
// v_alignbyte, 9 loads per slot, measured 2-5% slower in the CU-resident
// kernel.)
// Value = d * sc * (q6 - 32): the -32 is applied through the x chunk sums.
template <int LPR, int NS, int R, bool TOP1 = false>
ER_DEV void gemv_q6k_i8(const uint8_t *__restrict__ W, const float *__restrict__ x,
                        float *__restrict__ y, uint32_t M, uint32_t K,
                        float *__restrict__ pv = nullptr, uint32_t *__restrict__ pi = nullptr) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    __shared__ float4 chkw[ER_GEMV_WAVES];  // the waves' shares of the launch's checks
    using C = I8Cfg<LPR, NS>;
    constexpr uint32_t NT = 64u * ER_GEMV_WAVES;
    x += (size_t)blockIdx.y * K;
    y += (size_t)blockIdx.y * M;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR, li = lane % LPR;
    const uint32_t S = K >> 6;
    const size_t rowBytes = (size_t)(K >> 8) * 210u;
    const uint32_t row0 = ((blockIdx.x * ER_GEMV_WAVES + wave) * C::G + g) * (uint32_t)R;
    const uint32_t waveS = __builtin_amdgcn_readfirstlane(wave);

    float4 xr[C::XG][4];
    xl_load<C::XG, NT>(x, K, xr);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 fa[NS][R], fb[NS][R], fh[NS][R];
    u32x2 fs[NS][R];
    uint32_t fd[NS][R];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const uint32_t s = min(li + (uint32_t)LPR * j, S - 1u);
        const uint32_t h = (s >> 1) & 1u, c = s & 1u;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = W + (size_t)min(row0 + (uint32_t)r, M - 1u) * rowBytes + (s >> 2) * 210u;
            fa[j][r] = ld16_u2(blk + 64u * h + 16u * c);
            fb[j][r] = ld16_u2(blk + 64u * h + 32u + 16u * c);
            fh[j][r] = ld16_u2(blk + 128u + 32u * h + 16u * c);
            fs[j][r] = ld8_u2(blk + 192u + 8u * h);
            fd[j][r] = ld2(blk + 208u);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    XlCheck ck;
    xl_store<C::XG, NT>(lds, K, xr, &ck);
    xl_store_tail<C::XG, NT>(x, lds, K, &ck);
    {  // this wave's share of the launch's checks, gathered by the conversion
        const float4 sh = xl_check_share(ck);
        if ((threadIdx.x & 63u) == 0) chkw[threadIdx.x >> 6] = sh;
    }
    __syncthreads();
    // the launch's check decisions, read while the first weights are in flight
    bool ill, nfx;
    xl_check_decide(chkw, ER_GEMV_WAVES, 4.0f, ill, nfx);
    __builtin_amdgcn_sched_barrier(0);

    const XLimbs X = xl_view(lds, K);
    const uint32_t M0F = vreg_const(0x0f0f0f0fu), M30 = vreg_const(0x30303030u);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        const uint32_t sRaw = li + (uint32_t)LPR * j;
        const uint32_t s = min(sRaw, S - 1u);
        const float live = sRaw < S ? 1.0f : 0.0f;
        const uint32_t b = s >> 2, h = (s >> 1) & 1u, c = s & 1u;
        const uint32_t G0 = 16u * b + 8u * h + c;
        // x limbs of the 4 granules G0 + 2m, and their sums / group scales
        u32x4 xv[ER_XL_PLANES][4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t off = 16u * xl_gswz(G0 + 2u * m);
#pragma unroll
            for (int l = 0; l < ER_XL_PLANES; ++l)
                xv[l][m] = *(const u32x4 *)__builtin_assume_aligned(X.planes + (size_t)l * X.K + off, 16);
        }
        const float sgA = live * X.sg64[4u * b + 2u * h], sgB = live * X.sg64[4u * b + 2u * h + 1u];
        float X32[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) X32[m] = 32.0f * X.x16[G0 + 2u * m];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t A[4] = {fa[j][r].x, fa[j][r].y, fa[j][r].z, fa[j][r].w};
            const uint32_t B[4] = {fb[j][r].x, fb[j][r].y, fb[j][r].z, fb[j][r].w};
            const uint32_t H[4] = {fh[j][r].x, fh[j][r].y, fh[j][r].z, fh[j][r].w};
            int cq[4][ER_XL_PLANES] = {};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q[4] = {(A[k] & M0F) | ((H[k] << 4) & M30),
                                       (B[k] & M0F) | ((H[k] << 2) & M30),
                                       ((A[k] >> 4) & M0F) | (H[k] & M30),
                                       ((B[k] >> 4) & M0F) | ((H[k] >> 2) & M30)};
#pragma unroll
                for (int m = 0; m < 4; ++m)
#pragma unroll
                    for (int l = 0; l < ER_XL_PLANES; ++l)
                        cq[m][l] = sdot4_acc((int)q[m], (int)xv[l][m][k], cq[m][l], k == 0);
            }
            // scales: m = 0, 1 in dword x (bytes c, 2 + c), m = 2, 3 in dword y
            const float s0 = (float)(int8_t)(fs[j][r].x >> (8u * c));
            const float s1 = (float)(int8_t)(fs[j][r].x >> (8u * c + 16u));
            const float s2 = (float)(int8_t)(fs[j][r].y >> (8u * c));
            const float s3 = (float)(int8_t)(fs[j][r].y >> (8u * c + 16u));
            float v = s0 * __builtin_fmaf(sgA, xl_combine(cq[0][0], cq[0][1], cq[0][2]), -live * X32[0]);
            v = __builtin_fmaf(s1, __builtin_fmaf(sgA, xl_combine(cq[1][0], cq[1][1], cq[1][2]), -live * X32[1]), v);
            v = __builtin_fmaf(s2, __builtin_fmaf(sgB, xl_combine(cq[2][0], cq[2][1], cq[2][2]), -live * X32[2]), v);
            v = __builtin_fmaf(s3, __builtin_fmaf(sgB, xl_combine(cq[3][0], cq[3][1], cq[3][2]), -live * X32[3]), v);
            acc[r] = __builtin_fmaf(f16_to_f32(fd[j][r]), v, acc[r]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<LPR>(acc[r]);
    if (ill || nfx) {
        float sp[R], hits = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sp[r] = 0.0f;
        const uint32_t ln = lane_id();
        const uint32_t fr0 = ((blockIdx.x * ER_GEMV_WAVES + waveS) * C::G + ln / LPR) * (uint32_t)R;
        nf_terms<R>([&](int r, uint32_t k) {
                        return q6k_weight_at(W + (size_t)min(fr0 + (uint32_t)r, M - 1u) * rowBytes, k);
                    },
                    [&](uint32_t k) { return x[k]; }, X.x16, K >> 4, ln % LPR, LPR, sp, hits, ill);
        hits = group_sum<LPR>(hits);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = group_sum<LPR>(sp[r]);
            acc[r] = hits > 0.0f ? v : acc[r];
        }
    }
    if constexpr (TOP1) {
        top1_epilogue<ER_GEMV_WAVES * C::G * R>(acc, R, (wave * C::G + g) * R, li == 0, M, pv, pi);
    } else if (li == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + (uint32_t)r < M) y[row0 + r] = acc[r];
    }
}

// ===========================================================================
// Family 3: CU-resident integer-dot kernels (Q4_K, Q8_0, Q6_K; K % 256 == 0)
// ===========================================================================
//
// The family-1 kernels run ~3.5 workgroups per CU, and each stages x on its
// own.  A CU's vector-memory path returns data in request order, so the x
// loads of every workgroup after the first on a CU wait behind the weight
// loads of those before it, and per-workgroup barriers tie each wave's first
// dot product to the slowest weight-load issue of its workgroup.  Here one
// 8-wave workgroup owns a CU-sized share of the rows (grid ~ one workgroup per
// CU), and:
//   - staging waves copy x into LDS with global_load_lds (issued before a
//     workgroup barrier that precedes every weight load, so the x requests
//     leave the CU first), convert it to limbs (er_xlimbs.h) and each bump an
//     LDS counter.  With one slot per lane, or 5 and more, all 8 waves stage
//     and issue their first weight loads before converting (waiting only for
//     their x pieces, which precede those loads in the in-order load count);
//     with 2-4 slots per lane waves 4..7 stage and issue their weights after
//     converting (each measured best for its case);
//   - every wave walks its rows with D units of weight loads in flight (a
//     unit is one slot of one row step: unit v + D is issued right after unit
//     v is consumed) and waits on the counter, not on a barrier, before its
//     first dot product.  Per-slot refills spread every wave's loads evenly
//     over the launch, so the last data to arrive finds little compute
//     behind it (rows of many slots gained most).
// Row assignment: step i of lane group (wave, g) in workgroup b is row
// (i * gridDim.x + b) * STEP + wave * G + g, G = 64 / LPR rows per wave step,
// STEP = ER_CU_WAVES * G rows per workgroup step: the workgroups' steps
// interleave over the matrix.  Q8_0 (F::SPREAD) puts the waves of a workgroup
// a grid apart instead: row ((i * ER_CU_WAVES + wave) * gridDim.x + b') * G + g
// with b' a permutation of the workgroup index that gives neighbouring rows to
// workgroups on one XCD (the same rows overall; 2% faster for Q8_0 at
// 14336 x 4096, no gain for Q4_K or Q6_K).
// Per-row arithmetic (slot order, lane reduction) is that of the family-1
// kernel with the same LPR and NS.

#define ER_CU_SPIN_LIMIT (1u << 22)   // bound on the staging-counter wait (s_sleep 1 per poll)
// units of weight loads in flight per wave in the unrolled kernels: the
// format's choice (F::UNITS: 3 for Q4_K slots of 48 bytes, which beat 2 and 4
// and the former 2 whole rows; 2 for Q8_0 slots of 68), except 2 for 7-slot
// rows (which then reach their x conversion sooner; 5 and 6 spill, 7 is
// slower) and two rows' worth for 4 slots per lane (2, 3 and 4 units spill
// there, 8 does not); two rows' worth for the rolled loop (whose body of
// ER_CU_UNROLL steps must hold a multiple of D units).  tests/test_build_regs.py
// checks that no kernel spills.
#define ER_CU_UNITS(F, NS, JC) ((JC) == 0 ? 2 * (NS) : (NS) == 4 ? 8 : (NS) >= 7 ? 2 : F::UNITS)
#ifndef ER_CU_UNROLL
#define ER_CU_UNROLL 4                // unroll of the rolled step loop
#endif

// Per-format slot access: weights of one slot (Wt), the x side of one slot
// (Xs), and the slot's contribution.
struct CuQ4K {
    static constexpr int FMT = ER_FMT_Q4_K;
    static constexpr bool SPREAD = false;  // row assignment (family comment)
    static constexpr int NLD = 3;    // load instructions per slot
    static constexpr int UNITS = 3;  // units in flight (ER_CU_UNITS)
    struct Wt {
        u32x4 h, qa, qb;
    };
    struct Xs {
        u32x4 xv[ER_XL_PLANES][4];
        float XL, XH, sg, live;
        Q4Sel sel;
    };
    ER_DEV size_t row_bytes(uint32_t K) { return (size_t)(K >> 8) * 144u; }
    ER_DEV Wt load(const uint8_t *row, uint32_t s) {
        const uint8_t *bp = row + (s >> 2) * 144u;
        const uint32_t p = s & 3u;
        return Wt{ld16_a16(bp), ld16_a16(bp + 16u + 32u * p), ld16_a16(bp + 32u + 32u * p)};
    }
    ER_DEV Xs xside(const XLimbs &X, uint32_t s, float live) {
        Xs o;
        xl_read_group(X, s, o.xv);
        const float4 c16 = *(const float4 *)__builtin_assume_aligned(X.x16 + 4u * s, 16);
        o.XL = c16.x + c16.y;
        o.XH = c16.z + c16.w;
        o.sg = live * X.sg64[s];
        o.live = live;
        o.sel = q4k_sel(s & 3u);
        return o;
    }
    ER_DEV float dot(const Wt &w, const Xs &xs, float acc, uint32_t M0F) {
        return acc + q4k_slot_dot(w.h, w.qa, w.qb, xs.xv, xs.XL, xs.XH, xs.sg, xs.live, xs.sel, M0F);
    }
};

struct CuQ8 {
    static constexpr int FMT = ER_FMT_Q8_0;
    static constexpr bool SPREAD = true;
    static constexpr int NLD = 5;
    static constexpr int UNITS = 2;
    using Wt = Q8Slot;
    struct Xs {
        u32x4 xv[ER_XL_PLANES][4];
        float sg;
    };
    ER_DEV size_t row_bytes(uint32_t K) { return (size_t)(K >> 6) * 68u; }
    ER_DEV Wt load(const uint8_t *row, uint32_t s) { return q8_slot_load(row + (size_t)s * 68u); }
    ER_DEV Xs xside(const XLimbs &X, uint32_t s, float live) {
        Xs o;
        xl_read_group(X, s, o.xv);
        o.sg = live > 0.0f ? X.sg64[s] : 0.0f;
        return o;
    }
    ER_DEV float dot(const Wt &w, const Xs &xs, float acc, uint32_t) { return q8_slot_dot(w, xs.xv, xs.sg, acc); }
};

// Q6_K, slot layout, loads and per-slot arithmetic of gemv_q6k_i8: one
// 2-byte-aligned vector load per field (ld16_u2 / ld8_u2).
struct CuQ6K {
    static constexpr int FMT = ER_FMT_Q6_K;
    static constexpr bool SPREAD = false;
    static constexpr int NLD = 5;
    static constexpr int UNITS = 3;
    struct Wt {
        u32x4 a, b, h;  // ql (q1 / q3 nibbles), ql (q2 / q4), qh
        u32x2 s;        // scales sc[8h .. 8h + 8)
        uint32_t d;
    };
    struct Xs {
        u32x4 xv[ER_XL_PLANES][4];
        float X32[4], sgA, sgB, live;
        uint32_t c;
    };
    ER_DEV size_t row_bytes(uint32_t K) { return (size_t)(K >> 8) * 210u; }
    ER_DEV Wt load(const uint8_t *row, uint32_t s) {
        const uint8_t *blk = row + (s >> 2) * 210u;
        const uint32_t h = (s >> 1) & 1u, c = s & 1u;
        return Wt{ld16_u2(blk + 64u * h + 16u * c), ld16_u2(blk + 64u * h + 32u + 16u * c),
                  ld16_u2(blk + 128u + 32u * h + 16u * c), ld8_u2(blk + 192u + 8u * h), ld2(blk + 208u)};
    }
    ER_DEV Xs xside(const XLimbs &X, uint32_t s, float live) {
        Xs o;
        const uint32_t b = s >> 2, h = (s >> 1) & 1u, c = s & 1u;
        const uint32_t G0 = 16u * b + 8u * h + c;  // granules G0 + 2m, m = 0..3
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t off = 16u * xl_gswz(G0 + 2u * m);
#pragma unroll
            for (int l = 0; l < ER_XL_PLANES; ++l)
                o.xv[l][m] = *(const u32x4 *)__builtin_assume_aligned(X.planes + (size_t)l * X.K + off, 16);
        }
        o.sgA = live * X.sg64[4u * b + 2u * h];
        o.sgB = live * X.sg64[4u * b + 2u * h + 1u];
#pragma unroll
        for (int m = 0; m < 4; ++m) o.X32[m] = 32.0f * X.x16[G0 + 2u * m];
        o.live = live;
        o.c = c;
        return o;
    }
    ER_DEV float dot(const Wt &w, const Xs &xs, float acc, uint32_t M0F) {
        const uint32_t M30 = 0x30303030u;
        const uint32_t A[4] = {w.a.x, w.a.y, w.a.z, w.a.w};
        const uint32_t B[4] = {w.b.x, w.b.y, w.b.z, w.b.w};
        const uint32_t H[4] = {w.h.x, w.h.y, w.h.z, w.h.w};
        int cq[4][ER_XL_PLANES] = {};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q[4] = {(A[k] & M0F) | ((H[k] << 4) & M30), (B[k] & M0F) | ((H[k] << 2) & M30),
                                   ((A[k] >> 4) & M0F) | (H[k] & M30), ((B[k] >> 4) & M0F) | ((H[k] >> 2) & M30)};
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int l = 0; l < ER_XL_PLANES; ++l)
                    cq[m][l] = sdot4_acc((int)q[m], (int)xs.xv[l][m][k], cq[m][l], k == 0);
        }
        // scales: m = 0, 1 in dword x (bytes c, 2 + c), m = 2, 3 in dword y
        const float s0 = (float)(int8_t)(w.s.x >> (8u * xs.c));
        const float s1 = (float)(int8_t)(w.s.x >> (8u * xs.c + 16u));
        const float s2 = (float)(int8_t)(w.s.y >> (8u * xs.c));
        const float s3 = (float)(int8_t)(w.s.y >> (8u * xs.c + 16u));
        float v = s0 * __builtin_fmaf(xs.sgA, xl_combine(cq[0][0], cq[0][1], cq[0][2]), -xs.live * xs.X32[0]);
        v = __builtin_fmaf(s1, __builtin_fmaf(xs.sgA, xl_combine(cq[1][0], cq[1][1], cq[1][2]), -xs.live * xs.X32[1]), v);
        v = __builtin_fmaf(s2, __builtin_fmaf(xs.sgB, xl_combine(cq[2][0], cq[2][1], cq[2][2]), -xs.live * xs.X32[2]), v);
        v = __builtin_fmaf(s3, __builtin_fmaf(xs.sgB, xl_combine(cq[3][0], cq[3][1], cq[3][2]), -xs.live * xs.X32[3]), v);
        return __builtin_fmaf(f16_to_f32(w.d), v, acc);
    }
};

// LDS bytes of the family: limbs, then K fp32 values of raw x.
ER_DEV uint32_t cu_lds_bytes(uint32_t K) { return xl_lds_bytes(K) + 4u * K; }


// D: units (slot, row step) of weight loads in flight per wave.
// JC > 0: exactly JC row steps per wave, fully unrolled (rowsPerWg = STEP * JC).
// JC == 0: a runtime number of steps, at most 64 per lane group (rowsPerWg <=
// STEP * 64), in a loop unrolled by ER_CU_UNROLL.  Either way every step is
// loaded and computed (steps past the workgroup's rows re-read its last row
// and are not stored), and the row sums are parked in lanes - step i's sum in
// lane i % LPR of res[i / LPR] - and stored after the last step, so only
// weight loads are outstanding while rows are computed and each wait covers
// exactly the loads it needs.
// TOP1: instead of storing y, the workgroup's row values go to LDS and wave 0
// merges their quads into the partial (pv, pi)[blockIdx.x] (M a multiple of
// 4 and quads inside one step, so no quad spans two workgroups; the dynamic
// LDS holds at least 4 * rowsPerWg bytes).
template <class F, int LPR, int NS, int D, int JC, bool TOP1 = false>
ER_DEV void gemv_cu(const uint8_t *__restrict__ W, const float *__restrict__ x, float *__restrict__ y,
                    uint32_t M, uint32_t K, uint32_t rowsPerWg, float *__restrict__ pv = nullptr,
                    uint32_t *__restrict__ pi = nullptr) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    __shared__ uint32_t staged;               // staging waves done
    __shared__ float4 chkw[ER_CU_WAVES];      // [staging wave] its share of the launch's checks
    constexpr uint32_t G = 64u / LPR;
    constexpr uint32_t STEP = ER_CU_WAVES * G;  // rows per workgroup step
    constexpr int NPARK = JC > 0 ? (JC + LPR - 1) / LPR : 64 / LPR;
    constexpr int UNR = JC > 0 ? JC : ER_CU_UNROLL;
    constexpr int UPB = UNR * NS;                  // units (step, slot) per unrolled body
    constexpr int D0 = D < UPB ? D : UPB;          // units issued before the first dot
    static_assert(JC > 0 || UPB % D == 0, "the rolled body's unit count is a multiple of D");
    // staging waves (see the family comment); with all waves staging, the
    // first D0 units are issued before the conversion
    constexpr uint32_t STG = (NS == 1 || NS >= 5) ? ER_CU_WAVES : 4u;
    constexpr bool EARLY = STG == ER_CU_WAVES;
    static_assert(D0 * F::NLD < 64, "the early weight loads fit the load counter");
    static_assert(!(TOP1 && F::SPREAD), "the top-1 epilogue maps local rows with the neighbouring-row assignment");
    x += (size_t)blockIdx.y * K;
    y += (size_t)blockIdx.y * M;
    // wave index as a scalar: the staging branch and the step count are wave-uniform
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t g = lane / LPR, li = lane % LPR;
    const uint32_t S = K >> 6;
    // Step i of this workgroup is global step i * gridDim.x + blockIdx.x, so at
    // any moment the CUs read rows spread over the whole matrix rather than
    // each its own contiguous block (contiguous blocks ran 5-7% slower: some
    // CUs' ranges were served more slowly and ended the launch late).  The
    // grid is ceil(M / rowsPerWg), so the global steps cover every row.
    const uint32_t J = rowsPerWg / STEP;  // steps per workgroup (rows past M are skipped)
    const uint32_t JR = JC > 0 ? (uint32_t)JC : max((J + UNR - 1u) / UNR * UNR, (uint32_t)UNR);
    const uint32_t laneRow = wave * G + g;  // row within a step
    // row of lane group (w, gg)'s step i.  With the spread assignment,
    // neighbouring rows of a step go to workgroups dispatched to the same XCD
    // (workgroup b runs on XCD b % 8; bx below orders them XCD by XCD when the
    // grid is a multiple of 8), so y is written back in whole L2 lines.
    const uint32_t bx = gridDim.x % 8u == 0 ? (blockIdx.x % 8u) * (gridDim.x / 8u) + blockIdx.x / 8u : blockIdx.x;
    auto rowAt = [&](uint32_t i, uint32_t w, uint32_t gg) {
        return F::SPREAD ? ((i * ER_CU_WAVES + w) * gridDim.x + bx) * G + gg
                         : (i * gridDim.x + blockIdx.x) * STEP + w * G + gg;
    };
    auto rowOf = [&](uint32_t i) { return rowAt(i, wave, g); };
    const size_t rowBytes = F::row_bytes(K);
    uint32_t *xraw = lds + xl_lds_bytes(K) / 4u;  // 16-byte aligned for K % 256 == 0

    typename F::Wt wb[D];
    auto issue = [&](uint32_t i, int j, int b) {
        const uint32_t row = min(rowOf(i), M - 1u);
        wb[b] = F::load(W + (size_t)row * rowBytes, min(li + (uint32_t)LPR * j, S - 1u));
    };
    auto prologue = [&]() {
#pragma unroll
        for (int v = 0; v < D0; ++v) {
            issue((uint32_t)(v / NS), v % NS, v);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // x is converted in blocks of one pass per wave: 4 KB (16 values per lane,
    // xl_store_chunk) or 2 KB (8 per lane, xl_store_half; the same bytes).
    // Half blocks when that spreads short rows over more waves, or long rows
    // over all 8 (measured: K = 1024 -5%, 14336 -2%; K = 4096 and 8192 +2-4%).
    const bool halfBlocks = K <= 2048u || (STG == ER_CU_WAVES && K > 8192u);
    const uint32_t nPieces = K >> 8;                      // 1 KB pieces of x
    const uint32_t perBlock = halfBlocks ? 2u : 4u;       // pieces per block
    const uint32_t nBlocks = (nPieces + perBlock - 1u) / perBlock;
    if (wave >= ER_CU_WAVES - STG) {
        const uint32_t si = wave - (ER_CU_WAVES - STG);
        if (si == 0 && lane == 0) staged = 0u;
        for (uint32_t b = si; b < nBlocks; b += STG)
            for (uint32_t q = perBlock * b; q < min(perBlock * b + perBlock, nPieces); ++q)
                __builtin_amdgcn_global_load_lds((const void *)(x + 256u * q + 4u * lane), (void *)(xraw + 256u * q),
                                                 16, 0, 0);
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the counter reset has landed
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();  // x requests of the workgroup precede its weight requests
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (EARLY) {
            prologue();
            // the D0 * NLD weight loads just issued are younger than this
            // wave's x pieces: once at most that many are outstanding, x is in LDS
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(D0 * F::NLD));
        } else {
            __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's x pieces are in LDS
        }
        __builtin_amdgcn_sched_barrier(0);
        XlCheck ck;
        if (halfBlocks) {
            for (uint32_t b = si; b < nBlocks; b += STG) {
                const uint32_t t = 64u * b + lane;  // 8-value half-chunk; lanes 8k..8k+7 hold one 64-group
                const uint32_t tc = min(t, (K >> 3) - 1u);
                float4 xr[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) xr[q] = *(const float4 *)(xraw + 8u * tc + 4u * q);
                xl_store_half(lds, K, xr, t, &ck);  // stores only half-chunks t < K / 8
            }
        } else {
            for (uint32_t b = si; b < nBlocks; b += STG) {
                const uint32_t t = 64u * b + lane;  // 16-value chunk; lanes 4k..4k+3 hold one 64-group
                const uint32_t tc = min(t, (K >> 4) - 1u);
                float4 xr[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) xr[q] = *(const float4 *)(xraw + 16u * tc + 4u * q);
                xl_store_chunk(lds, K, xr, t, &ck);  // stores only chunks t < K / 16
            }
        }
        {  // this staging wave's share of the launch's checks, gathered by the conversion
            const float4 sh = xl_check_share(ck);
            if (lane == 0) chkw[si] = sh;
        }
        // publish this wave's limb stores and check share: a release fence on
        // LDS alone (it waits for the LDS stores, lgkmcnt(0), not for the
        // weight loads in flight, which a release on every address space would
        // drain first)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if (lane == 0) __hip_atomic_fetch_add(&staged, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if constexpr (!EARLY) prologue();
    } else {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        prologue();
    }
    __builtin_amdgcn_sched_barrier(0);
    // the staging waves always finish; the bound only keeps a wave from
    // spinning forever should that ever fail, and a wave whose wait ran out
    // (computing on x that may not be staged) reports NaN for its rows
    uint32_t spins = 0;
    for (; __hip_atomic_load(&staged, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < STG && spins < ER_CU_SPIN_LIMIT;
         ++spins)
        __builtin_amdgcn_s_sleep(1);
    const bool stale = spins >= ER_CU_SPIN_LIMIT;
    __builtin_amdgcn_sched_barrier(0);

    const XLimbs X = xl_view(lds, K);
    const uint32_t M0F = vreg_const(0x0f0f0f0fu);
    typename F::Xs xs0;
    if constexpr (NS == 1) xs0 = F::xside(X, min(li, S - 1u), li < S ? 1.0f : 0.0f);
    float res[NPARK];
#pragma unroll
    for (int q = 0; q < NPARK; ++q) res[q] = 0.0f;
    // step i0 + u of a body starting at step i0: unit v = u * NS + j in buffer
    // v % D, refilled after its dot with unit v + D when `last` is false or
    // that unit lies inside the body; then the lane reduction and the parking
    // of the row sum
    auto step = [&](uint32_t i0, int u, bool last) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const int v = u * NS + j;
            if constexpr (NS == 1) {
                acc = F::dot(wb[v % D], xs0, acc, M0F);
            } else {
                // re-read per row: the opaque slot index keeps the compiler from
                // hoisting NS slots of x limbs out of the row loop into registers
                const uint32_t sRaw = li + (uint32_t)LPR * j;
                uint32_t sx = min(sRaw, S - 1u);
                asm volatile("" : "+v"(sx));
                const typename F::Xs xs = F::xside(X, sx, sRaw < S ? 1.0f : 0.0f);
                acc = F::dot(wb[v % D], xs, acc, M0F);
            }
            __builtin_amdgcn_sched_barrier(0);  // one slot of x limbs live at a time
            if (!last || v + D < UPB) issue(i0 + (uint32_t)((v + D) / NS), (v + D) % NS, v % D);
            __builtin_amdgcn_sched_barrier(0);
        }
        acc = group_sum<LPR>(acc);
        const uint32_t i = i0 + (uint32_t)u;
        const bool mine = li == i % LPR;
        const uint32_t q0 = i / LPR;
#pragma unroll
        for (int q = 0; q < NPARK; ++q) res[q] = (mine && q0 == (uint32_t)q) ? acc : res[q];
    };
    uint32_t i0 = 0;
    if constexpr (JC == 0) {
        for (; i0 + UNR < JR; i0 += UNR) {
#pragma unroll
            for (int u = 0; u < UNR; ++u) step(i0, u, false);
        }
    }
    // the launch's check decisions from the staging waves' shares, taken after
    // the next-to-last step of the last body, so the LDS reads run while the
    // last unit's weights are still arriving (before the first dot they
    // measured 1-2% slower on the heads; after the last step, ~2% slower)
    bool ill = false, nfx = false;
    constexpr int UCK = UNR >= 2 ? UNR - 2 : 0;
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
        step(i0, u, true);
        if (u == UCK) {
            xl_check_decide(chkw, (int)STG, F::FMT == ER_FMT_Q8_0 ? 1.0f : 4.0f, ill, nfx);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (ill) {
        // x the limbs do not carry precisely enough: every row of this lane
        // group again, in fp32 over every position from the raw weights, the
        // group's lanes splitting the 16-value chunks as the lane-group kernels
        // do; the sum of step st is parked where the row loop parked it
#pragma unroll 1
        for (uint32_t st = 0; st < J; ++st) {
            const uint32_t row = min(rowAt(st, wave, g), M - 1u);
            float sp1[1] = {0.0f}, h = 0.0f;
            nf_terms<1>([&](int, uint32_t k) { return weight_at<F::FMT>(W + (size_t)row * rowBytes, k); },
                        [&](uint32_t k) { return ((const float *)xraw)[k]; }, X.x16, K >> 4, li, LPR, sp1, h, true);
            const float v = group_sum<LPR>(sp1[0]);
#pragma unroll
            for (int q = 0; q < NPARK; ++q) res[q] = (li == st % LPR && (uint32_t)q == st / LPR) ? v : res[q];
        }
    } else if (nfx) {
        // each lane redoes its own parked rows over every chunk; raw x is in LDS
        float sp[NPARK], hits = 0.0f;
#pragma unroll
        for (int q = 0; q < NPARK; ++q) sp[q] = 0.0f;
        const uint32_t ln = lane_id();
        const uint32_t fg = ln / LPR, fli = ln % LPR;
        nf_terms<NPARK>(
            [&](int q, uint32_t k) {
                const uint32_t st = (uint32_t)q * LPR + fli;
                const uint32_t row = min(rowAt(st, wave, fg), M - 1u);
                return weight_at<F::FMT>(W + (size_t)row * rowBytes, k);
            },
            [&](uint32_t k) { return ((const float *)xraw)[k]; }, X.x16, K >> 4, 0u, 1u, sp, hits);
#pragma unroll
        for (int q = 0; q < NPARK; ++q) res[q] = hits > 0.0f ? sp[q] : res[q];
    }
#pragma unroll
    for (int q = 0; q < NPARK; ++q) res[q] = stale ? __builtin_nanf("") : res[q];
    if constexpr (TOP1) {
        __syncthreads();  // every wave is done with x: LDS now holds the row values
        float *tv = (float *)lds;  // local row i * STEP + laneRow of step i
#pragma unroll
        for (int q = 0; q < NPARK; ++q) {
            const uint32_t st = (uint32_t)q * LPR + li;
            if (st < J) tv[st * STEP + laneRow] = res[q];
        }
        __syncthreads();
        // quads never straddle steps (STEP % 4 == 0); those past M are skipped
        top1_partial(tv, J * STEP / 4u, M, [&](uint32_t l) { return ((l / STEP) * gridDim.x + blockIdx.x) * STEP + l % STEP; },
                     pv, pi);
    } else {
#pragma unroll
        for (int q = 0; q < NPARK; ++q) {
            const uint32_t st = (uint32_t)q * LPR + li;
            const uint32_t row = rowOf(st);
            if (st < J && row < M) y[row] = res[q];
        }
    }
}

// ---------------------------------------------------------------------------
// K-sliced CU-resident kernels: the workgroup's waves split K.
//
// With whole rows per lane group (gemv_cu), every row reads all of x's limbs
// back from LDS (3 bytes per weight: 688 KB per CU at 4096 x 14336, as much
// LDS time as the dot products take), and no wave starts before the whole of
// x is converted.  Here wave w owns the slots [spw w, spw (w + 1)) of every
// row of its workgroup, spw = ceil(S / 8) <= LPR = 64 / PAR (a Q4_K or Q8_0
// slot is one 64-group; a Q6_K slot takes x from two groups of its 256-block,
// so for Q6_K spw is a multiple of 4 and a wave's slice whole blocks: either
// way a slot's x is the wave's own).  It loads and
// converts only that slice of x, keeps each lane's slot of limbs in
// registers, and walks the workgroup's rows PAR at a time: lane LPR g + li
// takes row g of the step and slot spw w + li (lanes past the slice reuse its
// last slot with weight 0).  Row step j, row g is row (j * gridDim.x +
// blockIdx.x) * PAR + g; a step's slot dots are summed over the LPR lanes
// (group_sum) and parked in lane j (steps LPR + j in a second register).  At
// the end the 8 wave partials of each
// row meet in LDS and are added in wave order, so a row's value depends on K
// alone, not on the row partition or the batch.  J row steps per lane group,
// F::UNITS in flight.
// TOP1: instead of storing y, the workgroup's row values go to LDS and wave 0
// merges their quads into the partial (pv, pi)[blockIdx.x] (M a multiple of
// 4).  Quads of 4 consecutive rows stay in one workgroup: with PAR = 2 the
// steps pair up, step j taking rows ((j / 2) * gridDim.x + blockIdx.x) * 4 +
// 2 (j % 2) + g, and J is even.  The row values are the plain kernel's.
// Rows: where row r's bytes are and where its value goes (CukOne: one
// matrix; CukMulti: up to three matrices of one row length, concatenated;
// CukQ8Multi / CukQ8Pairs: the fused Q8_0 projections).  Rows::NORM: x enters
// as x * w (rows.normW, when set) and each row value is multiplied by the
// launch's RMSNorm factor 1 / sqrt(mean(x^2) + eps), formed after the end
// barrier from the waves' sums of x^2 over their slices, added in wave order.
// Rows::PAIRS: rows 2i, 2i + 1 are a gate row and its up row (PAR is even, so
// a pair never straddles a step); the even row's lane group stores
// Rows::act(gate) * up.
template <class F, int PAR, int J, bool TOP1, class Rows>
ER_DEV void gemv_cuk_rows(const Rows &rows, const float *__restrict__ x, uint32_t M, uint32_t K,
                          float *__restrict__ pv, uint32_t *__restrict__ pi) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    constexpr uint32_t LPR = 64u / PAR;  // lanes per row slice
    __shared__ float part[ER_CU_WAVES][PAR * J];  // [wave][local row PAR j + g]
    __shared__ float4 chk[ER_CU_WAVES];           // [wave] its slice's checks: e, r, non-finite
    __shared__ float tv[TOP1 ? PAR * J : 1];      // top-1: the workgroup's row values
    __shared__ float ssw[Rows::NORM ? ER_CU_WAVES : 1];  // RMSNorm: [wave] sum of x^2 over its slice
    static_assert(PAR == 2 || PAR == 4 || PAR == 8, "2, 4 or 8 rows per step");
    static_assert(J >= 1 && J <= 2 * (int)LPR && J <= ER_CUK_MAX_STEPS, "row sums parked two per lane of a slice");
    static_assert(!TOP1 || PAR > 2 || J % 2 == 0, "top-1 quads pair the steps of 2-row slices");
    // units in flight: the format's F::UNITS, or, with 8 rows per step, every
    // unit of a launch of at most 3 steps (Q8_0, 2 units: the fused QKV of
    // 4096 + 2 x 1024 rows x 4096 7.67 -> 7.44 us; with 4 rows per step at
    // K = 8192 7.90 -> 7.97, so those keep 2)
    constexpr int D = (PAR == 8 && J <= 3) ? J : (F::UNITS < J ? F::UNITS : J);
    // x pieces per wave: 16-value chunks (4 spw <= 4 LPR, 64 per pass), or for
    // 8-lane slices 8-value halves (8 spw <= 64: one pass)
    constexpr int VPL = PAR == 8 ? 8 : 16;  // values per lane per pass
    constexpr int NPASS = PAR == 2 ? 2 : 1;
    x += (size_t)blockIdx.y * K;
    const uint32_t lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t g = lane / LPR, li = lane % LPR;
    const uint32_t S = K >> 6;
    const uint32_t spw = F::FMT == ER_FMT_Q6_K ? 4u * ((S + 31u) >> 5) : (S + ER_CU_WAVES - 1u) / ER_CU_WAVES;
    const uint32_t s0 = wave * spw, s1 = min(s0 + spw, S);  // empty (s0 >= S) only for short rows
    auto rowAt = [&](uint32_t j, uint32_t gg) {
        return (TOP1 && PAR == 2) ? ((j >> 1) * gridDim.x + blockIdx.x) * 4u + 2u * (j & 1u) + gg
                                  : (j * gridDim.x + blockIdx.x) * (uint32_t)PAR + gg;
    };
    float res = 0.0f, res2 = 0.0f;  // step j's row sum parked in lane j (res), step LPR + j's in res2
    float4 share = float4{0.0f, 0.0f, 0.0f, 0.0f};  // this wave's share of the launch's checks
    float ssq = 0.0f;                               // RMSNorm: this wave's sum of x^2
    if (s0 < S) {
        const uint32_t s = s0 + li;
        const uint32_t sc = min(s, s1 - 1u);
        const float live = s < s1 ? 1.0f : 0.0f;
        // x slice: pieces [n s0, n s1) of VPL values (n = 64 / VPL), lanes
        // nk..nk+n-1 one 64-group; loads clamped into the slice, issued before
        // the weights
        constexpr uint32_t PPG = 64u / VPL;  // pieces per 64-group
        const uint32_t h0 = PPG * s0, h1 = PPG * s1;
        float4 xr[NPASS][VPL / 4];
#pragma unroll
        for (int p = 0; p < NPASS; ++p) {
            const uint32_t hc = min(h0 + 64u * p + lane, h1 - 1u);
#pragma unroll
            for (int q = 0; q < VPL / 4; ++q) xr[p][q] = *(const float4 *)(x + VPL * hc + 4u * q);
        }
        float4 nw[Rows::NORM ? NPASS : 1][VPL / 4];  // the norm weights of the same pieces
        if constexpr (Rows::NORM) {
            if (rows.normW) {
#pragma unroll
                for (int p = 0; p < NPASS; ++p) {
                    const uint32_t hc = min(h0 + 64u * p + lane, h1 - 1u);
#pragma unroll
                    for (int q = 0; q < VPL / 4; ++q) nw[p][q] = *(const float4 *)(rows.normW + VPL * hc + 4u * q);
                }
            }
        }
        // 2-row steps (the longest x slices, two passes per wave): every
        // wave's x requests leave the CU before any weight request.  The CU
        // returns data in request order, so a wave issuing its x after the
        // weights of the waves before it waited behind their HBM reads.
        // (Waves with no slice take the matching barrier below: every wave
        // passes exactly one.)  With 4 and 8 rows per step the barrier
        // measured slower at most step counts, so those kernels go without.
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PAR == 2) __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        typename F::Wt wb[D];
        auto issue = [&](uint32_t j, int b) {
            const uint32_t row = min(rowAt(j, g), M - 1u);
            wb[b] = F::load(rows.row(row), sc);
        };
#pragma unroll
        for (int v = 0; v < D; ++v) {
            issue((uint32_t)v, v);
            __builtin_amdgcn_sched_barrier(0);
        }
        // convert the slice (pieces past it are not stored: index K / VPL).
        // Every pass runs: a pass under a branch had its x loads sunk behind
        // the weight loads, and the conversion then waited for those too.
        if constexpr (Rows::NORM) {
            if (rows.normW) {
                // sum of x^2 over the slice's pieces (each once: clamped copies
                // past the slice are not counted), then x * w
#pragma unroll
                for (int p = 0; p < NPASS; ++p) {
                    const bool own = h0 + 64u * p + lane < h1;
#pragma unroll
                    for (int q = 0; q < VPL / 4; ++q) {
                        float4 &v = xr[p][q];
                        const float4 w = nw[p][q];
                        const float sq = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                        ssq += own ? sq : 0.0f;
                        v = float4{v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w};
                    }
                }
            }
        }
        XlCheck ck;
#pragma unroll
        for (int p = 0; p < NPASS; ++p) {
            const uint32_t hc = h0 + 64u * p + lane;
            if constexpr (VPL == 16)
                xl_store_chunk(lds, K, xr[p], hc < h1 ? hc : K >> 4, &ck);
            else
                xl_store_half(lds, K, xr[p], hc < h1 ? hc : K >> 3, &ck);
        }
        share = xl_check_share(ck);
        // the wave reads back only what it stored; its LDS accesses run in order
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
        const XLimbs X = xl_view(lds, K);
        const uint32_t M0F = vreg_const(0x0f0f0f0fu);
        const typename F::Xs xs = F::xside(X, sc, live);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            float acc = F::dot(wb[j % D], xs, -0.0f, M0F);  // -0 + v == v: the add folds away
            __builtin_amdgcn_sched_barrier(0);
            if (j + D < J) issue((uint32_t)(j + D), j % D);
            __builtin_amdgcn_sched_barrier(0);
            acc = group_sum<LPR>(acc);
            if ((uint32_t)j < LPR)
                res = li == (uint32_t)j ? acc : res;
            else
                res2 = li == (uint32_t)j - LPR ? acc : res2;
        }
    } else if constexpr (PAR == 2) {
        __builtin_amdgcn_s_barrier();  // the x barrier above, for a wave with no slice
    }
    if (li < (uint32_t)J) part[wave][PAR * li + g] = res;
    if (LPR + li < (uint32_t)J) part[wave][PAR * (LPR + li) + g] = res2;
    if (lane == 0) chk[wave] = share;
    if constexpr (Rows::NORM) {
        ssq = group_sum<64>(ssq);
        if (lane == 0) ssw[wave] = ssq;
    }
    __syncthreads();  // every wave's partials and check shares, limbs, chunk sums and scales are in LDS
    const XLimbs X = xl_view(lds, K);
    bool ill, nf;
    xl_check_decide(chk, ER_CU_WAVES, F::FMT == ER_FMT_Q8_0 ? 1.0f : 4.0f, ill, nf);
    float rms = 1.0f;  // RMSNorm factor (Rows::NORM with a norm weight)
    if constexpr (Rows::NORM) {
        if (rows.normW) {
            float ss = 0.0f;
#pragma unroll
            for (int w = 0; w < ER_CU_WAVES; ++w) ss += ssw[w];
            rms = 1.0f / __builtin_sqrtf(ss / (float)K + rows.eps);
        }
    }
    // lane group (wave, g) finishes steps wave, wave + 8, ..., row g
#pragma unroll 1
    for (uint32_t st = wave; st < (uint32_t)J; st += ER_CU_WAVES) {
        const uint32_t lr = PAR * st + g;
        const uint32_t row = rowAt(st, g);
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < ER_CU_WAVES; ++w) v += part[w][lr];
        if constexpr (Rows::NORM) v *= rms;
        if (ill || nf) {
            // fp32 from the raw weights (every term, or the non-finite ones),
            // the group's lanes splitting the 16-value chunks; x as staged
            // (x * rms * w under RMSNorm)
            const uint32_t rc = min(row, M - 1u);
            float sp1[1] = {0.0f}, h = 0.0f;
            nf_terms<1>([&](int, uint32_t k) { return weight_at<F::FMT>(rows.row(rc), k); },
                        [&](uint32_t k) {
                            if constexpr (Rows::NORM) return rows.normW ? x[k] * rms * rows.normW[k] : x[k];
                            else return x[k];
                        },
                        X.x16, K >> 4, li, LPR, sp1, h, ill);
            const float fv = group_sum<LPR>(sp1[0]);
            h = group_sum<LPR>(h);
            v = (ill || h > 0.0f) ? fv : v;
        }
        if constexpr (TOP1) {
            if (li == 0) tv[lr] = v;
        } else if constexpr (Rows::PAIRS) {
            const float up = __shfl_down(v, LPR);  // the up row: lane group g + 1
            if ((g & 1u) == 0u && li == 0 && row < M) rows.store(row, Rows::act(v) * up);
        } else {
            if (li == 0 && row < M) rows.store(row, v);
        }
    }
    if constexpr (TOP1) {
        __syncthreads();
        top1_partial(tv, PAR * J / 4u, M, [&](uint32_t l) { return rowAt(l / PAR, l % PAR); }, pv, pi);
    }
}

struct CukOne {
    static constexpr bool NORM = false, PAIRS = false;
    const uint8_t *W;
    float *y;
    size_t rowBytes;
    __device__ __forceinline__ const uint8_t *row(uint32_t r) const { return W + (size_t)r * rowBytes; }
    __device__ __forceinline__ void store(uint32_t r, float v) const { y[r] = v; }
};

// Rows [0, M0) of W[0], then M1 of W[1], then M2 of W[2]; each row's value
// is the one the matrix's own K-sliced launch gives it.  Pointers and row
// counts are held as values (uniform: scalar registers).
struct CukMulti {
    static constexpr bool NORM = false, PAIRS = false;
    const uint8_t *W0, *W1, *W2;
    float *y0, *y1, *y2;
    uint32_t m1, m2;  // M0, M0 + M1
    size_t rowBytes;
    __device__ __forceinline__ CukMulti(const Q4Multi &mm, size_t rb)
        : W0(mm.W[0]), W1(mm.W[1]), W2(mm.W[2]), y0(mm.y[0]), y1(mm.y[1]), y2(mm.y[2]), m1(mm.M[0]),
          m2(mm.M[0] + mm.M[1]), rowBytes(rb) {}
    __device__ __forceinline__ uint32_t seg(uint32_t r, uint32_t &l) const {
        l = r < m1 ? r : (r < m2 ? r - m1 : r - m2);
        return r < m1 ? 0u : (r < m2 ? 1u : 2u);
    }
    __device__ __forceinline__ const uint8_t *row(uint32_t r) const {
        uint32_t l;
        const uint32_t m = seg(r, l);
        return pick3(m, W0, W1, W2) + (size_t)l * rowBytes;
    }
    __device__ __forceinline__ void store(uint32_t r, float v) const {
        uint32_t l;
        const uint32_t m = seg(r, l);
        pick3(m, y0, y1, y2)[l] = v;
    }
};

// The fused Q8_0 rows (Q8Multi): matrices concatenated as CukMulti; token t =
// blockIdx.y writes row l of matrix m at y[m] + t M[m] + l, fp16 when bit m of
// halfMask is set, adding res[m][t M[m] + l] when res[m] is set.
struct CukQ8Multi {
    static constexpr bool NORM = true, PAIRS = false;
    const uint8_t *W0, *W1, *W2;
    void *y0, *y1, *y2;
    const float *r0, *r1, *r2;
    uint32_t M0, M1, M2, halfMask;
    size_t rowBytes;
    const float *normW;
    float eps;
    __device__ __forceinline__ CukQ8Multi(const Q8Multi &mm, size_t rb)
        : W0(mm.W[0]), W1(mm.W[1]), W2(mm.W[2]), y0(mm.y[0]), y1(mm.y[1]), y2(mm.y[2]), r0(mm.res[0]),
          r1(mm.res[1]), r2(mm.res[2]), M0(mm.M[0]), M1(mm.M[1]), M2(mm.M[2]), halfMask(mm.halfMask), rowBytes(rb),
          normW(mm.normW), eps(mm.eps) {}
    __device__ __forceinline__ uint32_t seg(uint32_t r, uint32_t &l) const {
        const uint32_t m2 = M0 + M1;
        l = r < M0 ? r : (r < m2 ? r - M0 : r - m2);
        return r < M0 ? 0u : (r < m2 ? 1u : 2u);
    }
    __device__ __forceinline__ const uint8_t *row(uint32_t r) const {
        uint32_t l;
        const uint32_t m = seg(r, l);
        return pick3(m, W0, W1, W2) + (size_t)l * rowBytes;
    }
    __device__ __forceinline__ void store(uint32_t r, float v) const {
        uint32_t l;
        const uint32_t m = seg(r, l);
        const size_t out = (size_t)blockIdx.y * pick3(m, M0, M1, M2) + l;
        const float *rp = pick3(m, r0, r1, r2);
        void *yp = pick3(m, y0, y1, y2);
        const float o = rp ? v + rp[out] : v;
        if ((halfMask >> m) & 1u)
            ((_Float16 *)yp)[out] = (_Float16)o;
        else
            ((float *)yp)[out] = o;
    }
};

// Gate/up pairs: row 2i is gate row i, 2i + 1 up row i; token t writes
// y[t M + i].  CukQ8Pairs: the fused Q8_0 SiLU (RMSNorm, silu);
// CukGegluPairs: the Q4_K dual GeGLU (gelu_tanh, no norm).
struct CukQ8Pairs {
    static constexpr bool NORM = true, PAIRS = true;
    __device__ __forceinline__ static float act(float g) { return silu(g); }
    const uint8_t *Wg, *Wu;
    float *y;
    size_t rowBytes;
    const float *normW;
    float eps;
    uint32_t M;
    __device__ __forceinline__ const uint8_t *row(uint32_t r) const {
        return pick2((r & 1u) != 0u, Wg, Wu) + (size_t)(r >> 1) * rowBytes;
    }
    __device__ __forceinline__ void store(uint32_t r, float v) const { y[(size_t)blockIdx.y * M + (r >> 1)] = v; }
};

struct CukGegluPairs {
    static constexpr bool NORM = false, PAIRS = true;
    __device__ __forceinline__ static float act(float g) { return gelu_tanh(g); }
    const uint8_t *Wg, *Wu;
    float *y;
    size_t rowBytes;
    uint32_t M;
    __device__ __forceinline__ const uint8_t *row(uint32_t r) const {
        return pick2((r & 1u) != 0u, Wg, Wu) + (size_t)(r >> 1) * rowBytes;
    }
    __device__ __forceinline__ void store(uint32_t r, float v) const { y[(size_t)blockIdx.y * M + (r >> 1)] = v; }
};

template <class F, int PAR, int J, bool TOP1 = false>
ER_DEV void gemv_cuk(const uint8_t *__restrict__ W, const float *__restrict__ x, float *__restrict__ y,
                     uint32_t M, uint32_t K, float *__restrict__ pv = nullptr, uint32_t *__restrict__ pi = nullptr) {
    const CukOne rows{W, y + (size_t)blockIdx.y * M, F::row_bytes(K)};
    gemv_cuk_rows<F, PAR, J, TOP1>(rows, x, M, K, pv, pi);
}

// ===========================================================================
// Family 2: fp32 kernels
// ===========================================================================

// Stages x[0..K) in LDS; returns the pointer the slot loop reads x from.
template <bool XG>
ER_DEV const float *stage_x(const float *__restrict__ x, float *xs, uint32_t K) {
    if (XG) return x;
    const uint32_t K4 = K >> 2;
    const float4 *xg = (const float4 *)x;
    float4 *xs4 = (float4 *)xs;
    for (uint32_t i = threadIdx.x; i < K4; i += blockDim.x) xs4[i] = xg[i];
    __syncthreads();
    return xs;
}

ER_DEV void ld_x16(const float *p, float v[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 f = ((const float4 *)p)[i];
        v[4 * i + 0] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
}

ER_DEV float sum16(const float v[16]) {
    float s0 = (v[0] + v[1]) + (v[2] + v[3]);
    float s1 = (v[4] + v[5]) + (v[6] + v[7]);
    float s2 = (v[8] + v[9]) + (v[10] + v[11]);
    float s3 = (v[12] + v[13]) + (v[14] + v[15]);
    return (s0 + s1) + (s2 + s3);
}

// sum over 4 packed bytes of u (as unsigned) times x[0..4)
ER_DEV float dot4u(uint32_t u, const float *x, float acc) {
    acc = __builtin_fmaf(ub0(u), x[0], acc);
    acc = __builtin_fmaf(ub1(u), x[1], acc);
    acc = __builtin_fmaf(ub2(u), x[2], acc);
    acc = __builtin_fmaf(ub3(u), x[3], acc);
    return acc;
}

// ---------------------------------------------------------------------------
// Q4_K: slot s of a row -> super-block b = s/8, qs bytes [16i, 16i+16) with
// i = s%8, i.e. pair p = i/2 and positions l in [16(i&1), 16(i&1)+16) of
// sub-blocks 2p (low nibbles) and 2p+1 (high nibbles).
// ---------------------------------------------------------------------------
// EPI = ER_EPI_GEGLU: the dual gate/up GeGLU for rows longer than the
// integer-dot kernels cover: a lane group's rows [0, R/2) are gate rows of W,
// [R/2, R) the matching up rows of Wu, and the gate row's output is
// gelu_tanh(gate) * up.
template <int LPR, int R, bool XG, int EPI = ER_EPI_STORE>
ER_DEV void gemv_q4k(const uint8_t *__restrict__ W, const float *__restrict__ x,
                     float *__restrict__ y, uint32_t M, uint32_t K,
                     const uint8_t *__restrict__ Wu = nullptr) {
    extern __shared__ float xs_dyn[];
    x += (size_t)blockIdx.y * K;
    y += (size_t)blockIdx.y * M;
    const float *xv = stage_x<XG>(x, xs_dyn, K);

    constexpr int G = 64 / LPR;
    constexpr int OR = EPI == ER_EPI_GEGLU ? R / 2 : R;  // output rows per lane group
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR, li = lane % LPR;
    const uint32_t nb = K >> 8, S = nb << 3;
    const size_t rowBytes = (size_t)nb * 144u;
    const uint32_t row0 =
        ((blockIdx.x * (ER_GEMV_THREADS / 64) + wave) * G + g) * (uint32_t)OR;

    const uint8_t *rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = min(row0 + (uint32_t)(r % OR), M - 1u);
        rowp[r] = (EPI == ER_EPI_GEGLU && r >= OR ? Wu : W) + (size_t)row * rowBytes;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (uint32_t s = li; s < S; s += LPR) {
        const uint32_t b = s >> 3, i = s & 7u, p = i >> 1;
        const uint32_t blkOff = b * 144u;
        u32x4 hdr[R], qv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            hdr[r] = ld16_a16(rowp[r] + blkOff);
            qv[r] = ld16_a16(rowp[r] + blkOff + 16u + (i << 4));
        }
        const float *xa = xv + (b << 8) + (p << 6) + ((i & 1u) << 4);
        float xlo[16], xhi[16];
        ld_x16(xa, xlo);
        ld_x16(xa + 32, xhi);
        const float sLo = sum16(xlo), sHi = sum16(xhi);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = f16_to_f32(hdr[r].x & 0xffffu);
            const float dmin = f16_to_f32(hdr[r].x >> 16);
            uint32_t sc2, m2;
            q4k_scales_pair(hdr[r].y, hdr[r].z, hdr[r].w, p, &sc2, &m2);
            float fLo = 0.0f, fHi = 0.0f;
            const uint32_t qw[4] = {qv[r].x, qv[r].y, qv[r].z, qv[r].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = qw[k] & 0x0f0f0f0fu;
                const uint32_t hi = (qw[k] >> 4) & 0x0f0f0f0fu;
                fLo = dot4u(lo, xlo + 4 * k, fLo);
                fHi = dot4u(hi, xhi + 4 * k, fHi);
            }
            float a = acc[r];
            a = __builtin_fmaf(d * ub0(sc2), fLo, a);
            a = __builtin_fmaf(-(dmin * ub0(m2)), sLo, a);
            a = __builtin_fmaf(d * ub1(sc2), fHi, a);
            a = __builtin_fmaf(-(dmin * ub1(m2)), sHi, a);
            acc[r] = a;
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<LPR>(acc[r]);
    if (nf_any_value(xv, K)) {
        float sp[R], hits = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sp[r] = 0.0f;
        nf_terms<R>([&](int r, uint32_t k) { return q4k_weight_at(rowp[r], k); }, [&](uint32_t k) { return xv[k]; },
                    nullptr, K >> 4, li, LPR, sp, hits);
        hits = group_sum<LPR>(hits);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = group_sum<LPR>(sp[r]);
            acc[r] = hits > 0.0f ? v : acc[r];
        }
    }
    if (li == 0) {
        if constexpr (EPI == ER_EPI_GEGLU) {
#pragma unroll
            for (int r = 0; r < OR; ++r)
                if (row0 + (uint32_t)r < M) y[row0 + r] = gelu_tanh(acc[r]) * acc[OR + r];
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + (uint32_t)r < M) y[row0 + r] = acc[r];
        }
    }
}

// ---------------------------------------------------------------------------
// Q6_K: slot s -> super-block b = s/4, half h = (s/2)&1, lane chunk
// c = s&1 covering l in [16c, 16c+16): ql bytes [64h+16c, +16) (q1 low, q3
// high nibbles), [64h+32+16c, +16) (q2, q4), qh bytes [128+32h+16c, +16),
// scales sc[8h+c+{0,2,4,6}].  Blocks are 2-byte aligned: ld16_a2/ld8_a2.
// ---------------------------------------------------------------------------
// TOP1: the greedy top-1 partial epilogue in place of the store (one
// partial per workgroup; row values as the plain kernel computes them).
template <int LPR, int R, bool XG, bool TOP1 = false>
ER_DEV void gemv_q6k(const uint8_t *__restrict__ W, const float *__restrict__ x,
                     float *__restrict__ y, uint32_t M, uint32_t K,
                     float *__restrict__ pv = nullptr, uint32_t *__restrict__ pi = nullptr) {
    extern __shared__ float xs_dyn[];
    x += (size_t)blockIdx.y * K;
    y += (size_t)blockIdx.y * M;
    const float *xv = stage_x<XG>(x, xs_dyn, K);

    constexpr int G = 64 / LPR;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR, li = lane % LPR;
    const uint32_t nb = K >> 8, S = nb << 2;
    const size_t rowBytes = (size_t)nb * 210u;
    const uint32_t row0 =
        ((blockIdx.x * (ER_GEMV_THREADS / 64) + wave) * G + g) * (uint32_t)R;

    const uint8_t *rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = min(row0 + (uint32_t)r, M - 1u);
        rowp[r] = W + (size_t)row * rowBytes;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (uint32_t s = li; s < S; s += LPR) {
        const uint32_t b = s >> 2, h = (s >> 1) & 1u, c = s & 1u;
        const uint32_t blkOff = b * 210u;
        u32x4 qa[R], qb[R], qh[R];
        u32x2 sc[R];
        uint32_t dbits[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *blk = rowp[r] + blkOff;
            qa[r] = ld16_a2(blk + 64u * h + 16u * c);
            qb[r] = ld16_a2(blk + 64u * h + 32u + 16u * c);
            qh[r] = ld16_a2(blk + 128u + 32u * h + 16u * c);
            sc[r] = ld8_a2(blk + 192u + 8u * h);
            dbits[r] = ld2(blk + 208u);
        }
        const float *xb = xv + (b << 8) + (h << 7) + (c << 4);
        float x1[16], x2[16], x3[16], x4[16];
        ld_x16(xb, x1);
        ld_x16(xb + 32, x2);
        ld_x16(xb + 64, x3);
        ld_x16(xb + 96, x4);
        const float X1 = 32.0f * sum16(x1), X2 = 32.0f * sum16(x2);
        const float X3 = 32.0f * sum16(x3), X4 = 32.0f * sum16(x4);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t A[4] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w};
            const uint32_t B[4] = {qb[r].x, qb[r].y, qb[r].z, qb[r].w};
            const uint32_t H[4] = {qh[r].x, qh[r].y, qh[r].z, qh[r].w};
            float f1 = 0.0f, f2 = 0.0f, f3 = 0.0f, f4 = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q1 = (A[k] & 0x0f0f0f0fu) | ((H[k] << 4) & 0x30303030u);
                const uint32_t q2 = (B[k] & 0x0f0f0f0fu) | ((H[k] << 2) & 0x30303030u);
                const uint32_t q3 = ((A[k] >> 4) & 0x0f0f0f0fu) | (H[k] & 0x30303030u);
                const uint32_t q4 = ((B[k] >> 4) & 0x0f0f0f0fu) | ((H[k] >> 2) & 0x30303030u);
                f1 = dot4u(q1, x1 + 4 * k, f1);
                f2 = dot4u(q2, x2 + 4 * k, f2);
                f3 = dot4u(q3, x3 + 4 * k, f3);
                f4 = dot4u(q4, x4 + 4 * k, f4);
            }
            const float d = f16_to_f32(dbits[r]);
            float t = sb(sc[r].x, c) * (f1 - X1);
            t = __builtin_fmaf(sb(sc[r].x, c + 2u), f2 - X2, t);
            t = __builtin_fmaf(sb(sc[r].y, c), f3 - X3, t);
            t = __builtin_fmaf(sb(sc[r].y, c + 2u), f4 - X4, t);
            acc[r] = __builtin_fmaf(d, t, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<LPR>(acc[r]);
    if (nf_any_value(xv, K)) {
        float sp[R], hits = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sp[r] = 0.0f;
        nf_terms<R>([&](int r, uint32_t k) { return q6k_weight_at(rowp[r], k); }, [&](uint32_t k) { return xv[k]; },
                    nullptr, K >> 4, li, LPR, sp, hits);
        hits = group_sum<LPR>(hits);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = group_sum<LPR>(sp[r]);
            acc[r] = hits > 0.0f ? v : acc[r];
        }
    }
    if constexpr (TOP1) {
        top1_epilogue<ER_GEMV_WAVES * G * R>(acc, R, (wave * G + g) * R, li == 0, M, pv, pi);
    } else if (li == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + (uint32_t)r < M) y[row0 + r] = acc[r];
    }
}

// ---------------------------------------------------------------------------
// Q8_0, K % 64 == 0: slot s -> blocks 2s and 2s+1 = bytes [68s, 68s+68) of
// the row, 4-byte aligned because rows are 68*(K/64) bytes.
//   dwords v0..v16: block A d = v0[15:0], qs = bytes 2..33 (realigned by 2),
//                   block B d = v8[31:16], qs = v9..v16.
// ---------------------------------------------------------------------------
template <int LPR, int R, bool XG>
ER_DEV void gemv_q8_0(const uint8_t *__restrict__ W, const float *__restrict__ x,
                      float *__restrict__ y, uint32_t M, uint32_t K) {
    extern __shared__ float xs_dyn[];
    x += (size_t)blockIdx.y * K;
    y += (size_t)blockIdx.y * M;
    const float *xv = stage_x<XG>(x, xs_dyn, K);

    constexpr int G = 64 / LPR;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane / LPR, li = lane % LPR;
    const uint32_t S = K >> 6;
    const size_t rowBytes = (size_t)S * 68u;
    const uint32_t row0 =
        ((blockIdx.x * (ER_GEMV_THREADS / 64) + wave) * G + g) * (uint32_t)R;

    const uint8_t *rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = min(row0 + (uint32_t)r, M - 1u);
        rowp[r] = W + (size_t)row * rowBytes;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (uint32_t s = li; s < S; s += LPR) {
        uint32_t v[R][17];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *p = rowp[r] + (size_t)s * 68u;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 t = ld16_a4(p + 16 * j);
                v[r][4 * j + 0] = t.x;
                v[r][4 * j + 1] = t.y;
                v[r][4 * j + 2] = t.z;
                v[r][4 * j + 3] = t.w;
            }
            v[r][16] = ld4_a4(p + 64);
        }
        const float *xb = xv + (s << 6);
        float xa[32], xc[32];
        ld_x16(xb, xa);
        ld_x16(xb + 16, xa + 16);
        ld_x16(xb + 32, xc);
        ld_x16(xb + 48, xc + 16);
        const float XA = 128.0f * (sum16(xa) + sum16(xa + 16));
        const float XC = 128.0f * (sum16(xc) + sum16(xc + 16));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float fa = 0.0f, fc = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t qa = alignbyte(v[r][k + 1], v[r][k], 2) ^ 0x80808080u;
                const uint32_t qc = v[r][9 + k] ^ 0x80808080u;
                fa = dot4u(qa, xa + 4 * k, fa);
                fc = dot4u(qc, xc + 4 * k, fc);
            }
            const float dA = f16_to_f32(v[r][0] & 0xffffu);
            const float dC = f16_to_f32(v[r][8] >> 16);
            float a = __builtin_fmaf(dA, fa - XA, acc[r]);
            acc[r] = __builtin_fmaf(dC, fc - XC, a);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<LPR>(acc[r]);
    if (nf_any_value(xv, K)) {
        float sp[R], hits = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sp[r] = 0.0f;
        nf_terms<R>([&](int r, uint32_t k) { return q8_0_weight_at(rowp[r], k); }, [&](uint32_t k) { return xv[k]; },
                    nullptr, K >> 4, li, LPR, sp, hits);
        hits = group_sum<LPR>(hits);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = group_sum<LPR>(sp[r]);
            acc[r] = hits > 0.0f ? v : acc[r];
        }
    }
    if (li == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + (uint32_t)r < M) y[row0 + r] = acc[r];
    }
}

// Q8_0 for any K % 32 == 0 (rows only 2-byte aligned when K/32 is odd): one
// lane group per row, one block per lane step, 16-bit loads.  Not used at the
// BASELINE shapes; kept for the reference's full shape contract.
template <int R>
ER_DEV void gemv_q8_0_any(const uint8_t *__restrict__ W, const float *__restrict__ x,
                          float *__restrict__ y, uint32_t M, uint32_t K) {
    x += (size_t)blockIdx.y * K;
    y += (size_t)blockIdx.y * M;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t nb = K >> 5;
    const size_t rowBytes = (size_t)nb * 34u;
    const uint32_t row0 = (blockIdx.x * (ER_GEMV_THREADS / 64) + wave) * (uint32_t)R;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    for (uint32_t b = lane; b < nb; b += 64) {
        const float *xb = x + (b << 5);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = min(row0 + (uint32_t)r, M - 1u);
            const uint8_t *p = W + (size_t)row * rowBytes + (size_t)b * 34u;
            const float d = f16_to_f32(ld2(p));
            float f = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t q = ld4_a2(p + 2 + 4 * k);
                f = __builtin_fmaf(sb(q, 0), xb[4 * k + 0], f);
                f = __builtin_fmaf(sb(q, 1), xb[4 * k + 1], f);
                f = __builtin_fmaf(sb(q, 2), xb[4 * k + 2], f);
                f = __builtin_fmaf(sb(q, 3), xb[4 * k + 3], f);
            }
            acc[r] = __builtin_fmaf(d, f, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<64>(acc[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + (uint32_t)r < M) y[row0 + r] = acc[r];
    }
}

// Fused Q8_0 projections for any K % 32 == 0: rows only 2-byte aligned (odd
// K/32) or longer than the integer-dot kernels cover.  The arithmetic of
// gemv_q8_0_any over the concatenated rows of mm (EPI = ER_EPI_Q8_ROWS:
// + residual, fp32 or fp16 store) or over gate/up pairs (ER_EPI_Q8_SILU:
// W[0] gate, W[1] up, M[0] rows, silu(gate) * up into y[0]); R row
// computations per wave.  RMSNorm, when mm.normW is set: the workgroup sums
// x^2 over the token's row and every x value enters as x * rms * normW, the
// expression the integer-dot prologue stages.
template <int R, int EPI>
ER_DEV void gemv_q8_0_any_fused(const Q8Multi &mm, const float *__restrict__ x, uint32_t K) {
    __shared__ float red[ER_GEMV_WAVES];
    constexpr int OR = EPI == ER_EPI_Q8_SILU ? R / 2 : R;  // output rows per wave
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.y;
    const uint32_t nb = K >> 5;
    const size_t rowBytes = (size_t)nb * 34u;
    const uint32_t Mt = EPI == ER_EPI_Q8_SILU ? mm.M[0] : mm.M[0] + mm.M[1] + mm.M[2];
    const uint32_t row0 = (blockIdx.x * ER_GEMV_WAVES + wave) * (uint32_t)OR;
    x += (size_t)t * K;
    const float *__restrict__ nw = mm.normW;
    float rms = 1.0f;
    if (nw) {
        float ss = 0.0f;
        for (uint32_t k = threadIdx.x; k < K; k += ER_GEMV_THREADS) ss = __builtin_fmaf(x[k], x[k], ss);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        ss = 0.0f;
#pragma unroll
        for (int k = 0; k < ER_GEMV_WAVES; ++k) ss += red[k];
        rms = 1.0f / __builtin_sqrtf(ss / (float)K + mm.eps);
    }
    const uint8_t *rowp[R];
    void *yrow[OR];
    bool live[OR], half[OR];
    const float *res[OR];
#pragma unroll
    for (int r = 0; r < OR; ++r) {
        uint32_t v = min(row0 + (uint32_t)r, Mt - 1u);
        int m = 0;
        if (EPI == ER_EPI_Q8_ROWS && v >= mm.M[0]) {
            v -= mm.M[0];
            m = 1;
            if (v >= mm.M[1]) {
                v -= mm.M[1];
                m = 2;
            }
        }
        const uint32_t mu = (uint32_t)m;
        const size_t out = (size_t)t * pick3(mu, mm.M[0], mm.M[1], mm.M[2]) + v;
        rowp[r] = pick3(mu, mm.W[0], mm.W[1], mm.W[2]) + (size_t)v * rowBytes;
        if (EPI == ER_EPI_Q8_SILU) rowp[OR + r] = mm.W[1] + (size_t)v * rowBytes;
        half[r] = EPI == ER_EPI_Q8_ROWS && ((mm.halfMask >> m) & 1u);
        yrow[r] = (uint8_t *)pick3(mu, mm.y[0], mm.y[1], mm.y[2]) + out * (half[r] ? 2u : 4u);
        const float *rp = pick3(mu, mm.res[0], mm.res[1], mm.res[2]);
        res[r] = EPI == ER_EPI_Q8_ROWS && rp ? rp + out : nullptr;
        live[r] = row0 + (uint32_t)r < Mt;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    for (uint32_t b = lane; b < nb; b += 64) {
        float xb[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 f = ((const float4 *)(x + (b << 5)))[i];
            xb[4 * i + 0] = f.x;
            xb[4 * i + 1] = f.y;
            xb[4 * i + 2] = f.z;
            xb[4 * i + 3] = f.w;
        }
        if (nw) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 w = ((const float4 *)(nw + (b << 5)))[i];
                xb[4 * i + 0] = xb[4 * i + 0] * rms * w.x;
                xb[4 * i + 1] = xb[4 * i + 1] * rms * w.y;
                xb[4 * i + 2] = xb[4 * i + 2] * rms * w.z;
                xb[4 * i + 3] = xb[4 * i + 3] * rms * w.w;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *p = rowp[r] + (size_t)b * 34u;
            const float d = f16_to_f32(ld2(p));
            float f = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t q = ld4_a2(p + 2 + 4 * k);
                f = __builtin_fmaf(sb(q, 0), xb[4 * k + 0], f);
                f = __builtin_fmaf(sb(q, 1), xb[4 * k + 1], f);
                f = __builtin_fmaf(sb(q, 2), xb[4 * k + 2], f);
                f = __builtin_fmaf(sb(q, 3), xb[4 * k + 3], f);
            }
            acc[r] = __builtin_fmaf(d, f, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = group_sum<64>(acc[r]);
    if (lane != 0) return;
#pragma unroll
    for (int r = 0; r < OR; ++r) {
        if (!live[r]) continue;
        if constexpr (EPI == ER_EPI_Q8_SILU) {
            *(float *)yrow[r] = silu(acc[r]) * acc[OR + r];
        } else {
            const float v = res[r] ? acc[r] + *res[r] : acc[r];
            if (half[r])
                *(_Float16 *)yrow[r] = (_Float16)v;
            else
                *(float *)yrow[r] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Entry points (extern "C" so hipModuleGetFunction resolves them by name).
//   er_gemv_<fmt>_i8_l<LPR>_n<NS>_r<R> : integer-dot family (er_gemv_cfg.h; q4k, q8_0, q6k)
//   er_gemv_q6k_top1_l<LPR>_n<NS>_r<R> : Q6_K with the top-1 partial epilogue
//   er_gemv_<fmt>_l<LPR>_<s|g>         : fp32 family, x staged in LDS (s) or
//                                        read from global memory (g)
// ---------------------------------------------------------------------------
#define ER_I8_ENTRY(LPR, NS, R)                                                                \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q4k_i8_l##LPR##_n##NS##_r##R(const uint8_t *__restrict__ W,                  \
                                             const float *__restrict__ x,                     \
                                             float *__restrict__ y, uint32_t M, uint32_t K) { \
        gemv_q4k_i8<LPR, NS, R>(W, x, y, M, K);                                              \
    }                                                                                          \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q8_0_i8_l##LPR##_n##NS##_r##R(const uint8_t *__restrict__ W,                 \
                                              const float *__restrict__ x,                    \
                                              float *__restrict__ y, uint32_t M, uint32_t K) { \
        gemv_q8_0_i8<LPR, NS, R>(W, x, y, M, K);                                             \
    }                                                                                          \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q6k_i8_l##LPR##_n##NS##_r##R(const uint8_t *__restrict__ W,                  \
                                             const float *__restrict__ x,                     \
                                             float *__restrict__ y, uint32_t M, uint32_t K) { \
        gemv_q6k_i8<LPR, NS, R>(W, x, y, M, K);                                              \
    }                                                                                          \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q6k_top1_l##LPR##_n##NS##_r##R(const uint8_t *__restrict__ W,                \
                                               const float *__restrict__ x,                   \
                                               float *__restrict__ pv, uint32_t *__restrict__ pi, \
                                               uint32_t M, uint32_t K) {                      \
        gemv_q6k_i8<LPR, NS, R, true>(W, x, nullptr, M, K, pv, pi);                          \
    }
ER_I8_CONFIGS(ER_I8_ENTRY)

// CU-resident family: er_gemv_<fmt>_cu_l<LPR>_n<NS>_j<JC> (JC row steps per
// wave, unrolled) and _jr (rolled, up to 64 steps per lane group); grid
// (ceil(M / rowsPerWg), batch), rowsPerWg = ER_CU_WAVES * 64 / LPR * steps.
// er_gemv_q6k_top1_cu_*: the same kernels with the top-1 partial epilogue
// (grid ceil(M / rowsPerWg), one partial per workgroup).
#define ER_CU_ENTRY_J(fmt, F, LPR, NS, JC, tag)                                                 \
    extern "C" __global__ void __launch_bounds__(64 * ER_CU_WAVES)                           \
        er_gemv_##fmt##_cu_l##LPR##_n##NS##_j##tag(const uint8_t *__restrict__ W,              \
                                                   const float *__restrict__ x,               \
                                                   float *__restrict__ y, uint32_t M, uint32_t K, \
                                                   uint32_t rowsPerWg) {                      \
        gemv_cu<F, LPR, NS, ER_CU_UNITS(F, NS, JC), JC>(W, x, y, M, K, rowsPerWg);               \
    }
#define ER_CU_TOP1_J(fmt, F, LPR, NS, JC, tag)                                                     \
    extern "C" __global__ void __launch_bounds__(64 * ER_CU_WAVES)                              \
        er_gemv_##fmt##_top1_cu_l##LPR##_n##NS##_j##tag(const uint8_t *__restrict__ W,            \
                                                        const float *__restrict__ x,             \
                                                        float *__restrict__ pv,                  \
                                                        uint32_t *__restrict__ pi, uint32_t M,   \
                                                        uint32_t K, uint32_t rowsPerWg) {        \
        gemv_cu<F, LPR, NS, ER_CU_UNITS(F, NS, JC), JC, true>(W, x, nullptr, M, K, rowsPerWg, pv, pi); \
    }
#define ER_CU_STEPS_1(E, fmt, F, LPR, NS) E(fmt, F, LPR, NS, 1, 1)
#define ER_CU_STEPS_2(E, fmt, F, LPR, NS) ER_CU_STEPS_1(E, fmt, F, LPR, NS) E(fmt, F, LPR, NS, 2, 2)
#define ER_CU_STEPS_8(E, fmt, F, LPR, NS)                                                              \
    ER_CU_STEPS_2(E, fmt, F, LPR, NS) E(fmt, F, LPR, NS, 3, 3) E(fmt, F, LPR, NS, 4, 4)                  \
    E(fmt, F, LPR, NS, 5, 5) E(fmt, F, LPR, NS, 6, 6) E(fmt, F, LPR, NS, 7, 7) E(fmt, F, LPR, NS, 8, 8) \
    E(fmt, F, LPR, NS, 0, r)
#define ER_CU_ENTRY_Q4K(LPR, NS, MAXJ) ER_CU_STEPS_##MAXJ(ER_CU_ENTRY_J, q4k, CuQ4K, LPR, NS)
#define ER_CU_ENTRY_Q8(LPR, NS, MAXJ) ER_CU_STEPS_##MAXJ(ER_CU_ENTRY_J, q8_0, CuQ8, LPR, NS)
#define ER_CU_ENTRY_Q6K(LPR, NS, MAXJ)                        \
    ER_CU_STEPS_##MAXJ(ER_CU_ENTRY_J, q6k, CuQ6K, LPR, NS) \
    ER_CU_STEPS_##MAXJ(ER_CU_TOP1_J, q6k, CuQ6K, LPR, NS)
ER_CU_CONFIGS_Q4K(ER_CU_ENTRY_Q4K)
ER_CU_CONFIGS_Q8(ER_CU_ENTRY_Q8)
ER_CU_CONFIGS_Q6K(ER_CU_ENTRY_Q6K)

// K-sliced CU-resident kernels: er_gemv_<fmt>_cuk<PAR>_j<J>, J = 1..ER_CUK_MAX_STEPS
// row steps of PAR rows per workgroup (J <= 2 * 64 / PAR), grid (ceil(M / (PAR J)),
// batch), dynamic LDS xl_lds_bytes(K).
#define ER_CUK_ENTRY(fmt, F, PAR, J)                                                                \
    extern "C" __global__ void __launch_bounds__(64 * ER_CU_WAVES)                                 \
        er_gemv_##fmt##_cuk##PAR##_j##J(const uint8_t *__restrict__ W, const float *__restrict__ x,  \
                                        float *__restrict__ y, uint32_t M, uint32_t K) {            \
        gemv_cuk<F, PAR, J>(W, x, y, M, K);                                                         \
    }
#define ER_CUK_ENTRIES8(fmt, F, PAR)                                                                        \
    ER_CUK_ENTRY(fmt, F, PAR, 1) ER_CUK_ENTRY(fmt, F, PAR, 2) ER_CUK_ENTRY(fmt, F, PAR, 3)                  \
    ER_CUK_ENTRY(fmt, F, PAR, 4) ER_CUK_ENTRY(fmt, F, PAR, 5) ER_CUK_ENTRY(fmt, F, PAR, 6)                  \
    ER_CUK_ENTRY(fmt, F, PAR, 7) ER_CUK_ENTRY(fmt, F, PAR, 8)
#define ER_CUK_ENTRIES16(fmt, F, PAR)                                                                       \
    ER_CUK_ENTRIES8(fmt, F, PAR) ER_CUK_ENTRY(fmt, F, PAR, 9) ER_CUK_ENTRY(fmt, F, PAR, 10)                 \
    ER_CUK_ENTRY(fmt, F, PAR, 11) ER_CUK_ENTRY(fmt, F, PAR, 12) ER_CUK_ENTRY(fmt, F, PAR, 13)               \
    ER_CUK_ENTRY(fmt, F, PAR, 14) ER_CUK_ENTRY(fmt, F, PAR, 15) ER_CUK_ENTRY(fmt, F, PAR, 16)
ER_CUK_ENTRIES16(q4k, CuQ4K, 2)
ER_CUK_ENTRIES16(q4k, CuQ4K, 4)
ER_CUK_ENTRIES16(q4k, CuQ4K, 8)
ER_CUK_ENTRIES16(q8_0, CuQ8, 2)
ER_CUK_ENTRIES16(q8_0, CuQ8, 4)
ER_CUK_ENTRIES16(q8_0, CuQ8, 8)
// The Q4_K dual / triple over the K-sliced kernels: er_gemv_q4k_multi_cuk<PAR>_j<J>
// (mm, x, K), rows of the matrices concatenated, one token; and the dual GeGLU,
// er_gemv_q4k_geglu_cuk<PAR>_j<J> (Wg, Wu, x, y, M, K; 2M rows).
#define ER_CUK_MULTI_ENTRY(PAR, J)                                                          \
    extern "C" __global__ void __launch_bounds__(64 * ER_CU_WAVES)                                 \
        er_gemv_q4k_multi_cuk##PAR##_j##J(Q4Multi mm, const float *__restrict__ x, uint32_t K) {     \
        const CukMulti rows(mm, CuQ4K::row_bytes(K));                                               \
        gemv_cuk_rows<CuQ4K, PAR, J, false>(rows, x, mm.M[0] + mm.M[1] + mm.M[2], K, nullptr, nullptr); \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(64 * ER_CU_WAVES)                                 \
        er_gemv_q4k_geglu_cuk##PAR##_j##J(const uint8_t *__restrict__ Wg, const uint8_t *__restrict__ Wu, \
                                          const float *__restrict__ x, float *__restrict__ y, uint32_t M, \
                                          uint32_t K) {                                            \
        const CukGegluPairs rows{Wg, Wu, y, CuQ4K::row_bytes(K), M};                                \
        gemv_cuk_rows<CuQ4K, PAR, J, false>(rows, x, 2u * M, K, nullptr, nullptr);                  \
    }
#define ER_CUK_MULTI8(PAR)                                                                                   \
    ER_CUK_MULTI_ENTRY(PAR, 1) ER_CUK_MULTI_ENTRY(PAR, 2) ER_CUK_MULTI_ENTRY(PAR, 3)             \
    ER_CUK_MULTI_ENTRY(PAR, 4) ER_CUK_MULTI_ENTRY(PAR, 5) ER_CUK_MULTI_ENTRY(PAR, 6)             \
    ER_CUK_MULTI_ENTRY(PAR, 7) ER_CUK_MULTI_ENTRY(PAR, 8)
#define ER_CUK_MULTI16(PAR)                                                                                  \
    ER_CUK_MULTI8(PAR) ER_CUK_MULTI_ENTRY(PAR, 9) ER_CUK_MULTI_ENTRY(PAR, 10)                        \
    ER_CUK_MULTI_ENTRY(PAR, 11) ER_CUK_MULTI_ENTRY(PAR, 12) ER_CUK_MULTI_ENTRY(PAR, 13)          \
    ER_CUK_MULTI_ENTRY(PAR, 14) ER_CUK_MULTI_ENTRY(PAR, 15) ER_CUK_MULTI_ENTRY(PAR, 16)
ER_CUK_MULTI16(2)
ER_CUK_MULTI16(4)
ER_CUK_MULTI16(8)
// The fused Q8_0 projections over the K-sliced kernels: er_gemv_q8_0_multi_cuk<PAR>_j<J>
// (mm, x, K) and er_gemv_q8_0_silu_cuk<PAR>_j<J> (Wg, Wu, x, y, normW, eps, M, K;
// 2M rows), grid (ceil(rows / (PAR J)), tokens).
#define ER_CUK_Q8F_ENTRY(PAR, J)                                                                              \
    extern "C" __global__ void __launch_bounds__(64 * ER_CU_WAVES)                                           \
        er_gemv_q8_0_multi_cuk##PAR##_j##J(Q8Multi mm, const float *__restrict__ x, uint32_t K) {              \
        const CukQ8Multi rows(mm, CuQ8::row_bytes(K));                                      \
        gemv_cuk_rows<CuQ8, PAR, J, false>(rows, x, mm.M[0] + mm.M[1] + mm.M[2], K, nullptr, nullptr);        \
    }                                                                                                          \
    extern "C" __global__ void __launch_bounds__(64 * ER_CU_WAVES)                                           \
        er_gemv_q8_0_silu_cuk##PAR##_j##J(const uint8_t *__restrict__ Wg, const uint8_t *__restrict__ Wu,      \
                                          const float *__restrict__ x, float *__restrict__ y,                 \
                                          const float *__restrict__ normW, float eps, uint32_t M, uint32_t K) { \
        const CukQ8Pairs rows{Wg, Wu, y, CuQ8::row_bytes(K), normW, eps, M};                                  \
        gemv_cuk_rows<CuQ8, PAR, J, false>(rows, x, 2u * M, K, nullptr, nullptr);                             \
    }
#define ER_CUK_Q8F8(PAR)                                                                                     \
    ER_CUK_Q8F_ENTRY(PAR, 1) ER_CUK_Q8F_ENTRY(PAR, 2) ER_CUK_Q8F_ENTRY(PAR, 3) ER_CUK_Q8F_ENTRY(PAR, 4)       \
    ER_CUK_Q8F_ENTRY(PAR, 5) ER_CUK_Q8F_ENTRY(PAR, 6) ER_CUK_Q8F_ENTRY(PAR, 7) ER_CUK_Q8F_ENTRY(PAR, 8)
#define ER_CUK_Q8F16(PAR)                                                                                    \
    ER_CUK_Q8F8(PAR) ER_CUK_Q8F_ENTRY(PAR, 9) ER_CUK_Q8F_ENTRY(PAR, 10) ER_CUK_Q8F_ENTRY(PAR, 11)            \
    ER_CUK_Q8F_ENTRY(PAR, 12) ER_CUK_Q8F_ENTRY(PAR, 13) ER_CUK_Q8F_ENTRY(PAR, 14) ER_CUK_Q8F_ENTRY(PAR, 15)  \
    ER_CUK_Q8F_ENTRY(PAR, 16)
ER_CUK_Q8F16(2)
ER_CUK_Q8F16(4)
ER_CUK_Q8F16(8)
// Q6_K: rows of more than 64 slots (2 and 4 rows per step), and the top-1
// forms (er_gemv_q6k_top1_cuk<PAR>_j<J>: (W, x, pv, pi, M, K), even J for PAR 2)
ER_CUK_ENTRIES16(q6k, CuQ6K, 2)
ER_CUK_ENTRIES16(q6k, CuQ6K, 4)
#define ER_CUK_TOP1_ENTRY(PAR, J)                                                                      \
    extern "C" __global__ void __launch_bounds__(64 * ER_CU_WAVES)                                    \
        er_gemv_q6k_top1_cuk##PAR##_j##J(const uint8_t *__restrict__ W, const float *__restrict__ x,    \
                                         float *__restrict__ pv, uint32_t *__restrict__ pi, uint32_t M, \
                                         uint32_t K) {                                                  \
        gemv_cuk<CuQ6K, PAR, J, true>(W, x, nullptr, M, K, pv, pi);                                   \
    }
ER_CUK_TOP1_ENTRY(2, 2) ER_CUK_TOP1_ENTRY(2, 4) ER_CUK_TOP1_ENTRY(2, 6) ER_CUK_TOP1_ENTRY(2, 8)
ER_CUK_TOP1_ENTRY(2, 10) ER_CUK_TOP1_ENTRY(2, 12) ER_CUK_TOP1_ENTRY(2, 14) ER_CUK_TOP1_ENTRY(2, 16)
ER_CUK_TOP1_ENTRY(4, 1) ER_CUK_TOP1_ENTRY(4, 2) ER_CUK_TOP1_ENTRY(4, 3) ER_CUK_TOP1_ENTRY(4, 4)
ER_CUK_TOP1_ENTRY(4, 5) ER_CUK_TOP1_ENTRY(4, 6) ER_CUK_TOP1_ENTRY(4, 7) ER_CUK_TOP1_ENTRY(4, 8)
ER_CUK_TOP1_ENTRY(4, 9) ER_CUK_TOP1_ENTRY(4, 10) ER_CUK_TOP1_ENTRY(4, 11) ER_CUK_TOP1_ENTRY(4, 12)
ER_CUK_TOP1_ENTRY(4, 13) ER_CUK_TOP1_ENTRY(4, 14) ER_CUK_TOP1_ENTRY(4, 15) ER_CUK_TOP1_ENTRY(4, 16)

// Multi-matrix and GeGLU Q4_K kernels: R counts row computations per lane
// group (GeGLU: R/2 gate rows + the matching up rows).
#define ER_I8_MULTI_ENTRY(LPR, NS, R)                                                          \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q4k_multi_l##LPR##_n##NS##_r##R(Q4Multi mm, const float *__restrict__ x,       \
                                                uint32_t K) {                                 \
        gemv_q4k_i8_multi<LPR, NS, R>(mm, x, K);                                              \
    }                                                                                          \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q4k_geglu_l##LPR##_n##NS##_r##R(const uint8_t *__restrict__ Wg,                \
                                                const uint8_t *__restrict__ Wu,                \
                                                const float *__restrict__ x,                   \
                                                float *__restrict__ y, uint32_t M, uint32_t K) { \
        gemv_q4k_i8_geglu<LPR, NS, R>(Wg, Wu, x, y, M, K);                                    \
    }                                                                                          \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q8_0_multi_l##LPR##_n##NS##_r##R(Q8Multi mm, const float *__restrict__ x,      \
                                                 uint32_t K) {                                \
        gemv_q8_0_i8_multi<LPR, NS, R>(mm, x, K);                                             \
    }                                                                                          \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q8_0_silu_l##LPR##_n##NS##_r##R(const uint8_t *__restrict__ Wg,                \
                                                const uint8_t *__restrict__ Wu,                \
                                                const float *__restrict__ x,                   \
                                                float *__restrict__ y,                         \
                                                const float *__restrict__ normW, float eps,    \
                                                uint32_t M, uint32_t K) {                      \
        gemv_q8_0_i8_silu<LPR, NS, R>(Wg, Wu, x, y, normW, eps, M, K);                        \
    }
ER_I8_MULTI_CONFIGS(ER_I8_MULTI_ENTRY)

// The multi-matrix kernels with one row computation per lane group
// (ER_I8_MULTI1_CONFIGS; same names and arguments as above).
#define ER_I8_MULTI1_ENTRY(LPR, NS, R)                                                         \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q4k_multi_l##LPR##_n##NS##_r##R(Q4Multi mm, const float *__restrict__ x,       \
                                                uint32_t K) {                                 \
        gemv_q4k_i8_multi<LPR, NS, R>(mm, x, K);                                              \
    }                                                                                          \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                            \
        er_gemv_q8_0_multi_l##LPR##_n##NS##_r##R(Q8Multi mm, const float *__restrict__ x,      \
                                                 uint32_t K) {                                \
        gemv_q8_0_i8_multi<LPR, NS, R>(mm, x, K);                                             \
    }
ER_I8_MULTI1_CONFIGS(ER_I8_MULTI1_ENTRY)

#define ER_GEMV_ENTRY(fmt, impl, rows, lpr, xg, tag)                                       \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                        \
        er_gemv_##fmt##_l##lpr##_##tag(const uint8_t *__restrict__ W,                     \
                                         const float *__restrict__ x, float *__restrict__ y, \
                                         uint32_t M, uint32_t K) {                        \
        impl<lpr, rows, xg>(W, x, y, M, K);                                              \
    }

#define ER_GEMV_FAMILY(fmt, impl, rows)        \
    ER_GEMV_ENTRY(fmt, impl, rows, 64, false, s) \
    ER_GEMV_ENTRY(fmt, impl, rows, 32, false, s) \
    ER_GEMV_ENTRY(fmt, impl, rows, 16, false, s) \
    ER_GEMV_ENTRY(fmt, impl, rows, 8, false, s)  \
    ER_GEMV_ENTRY(fmt, impl, rows, 4, false, s)  \
    ER_GEMV_ENTRY(fmt, impl, rows, 64, true, g)  \
    ER_GEMV_ENTRY(fmt, impl, rows, 32, true, g)  \
    ER_GEMV_ENTRY(fmt, impl, rows, 16, true, g)  \
    ER_GEMV_ENTRY(fmt, impl, rows, 8, true, g)   \
    ER_GEMV_ENTRY(fmt, impl, rows, 4, true, g)

ER_GEMV_FAMILY(q6k, gemv_q6k, ER_Q6K_ROWS)
// fp32 fallbacks of the integer-dot formats for rows longer than 32768 weights
ER_GEMV_ENTRY(q4k, gemv_q4k, ER_Q4K_ROWS, 64, true, g)
ER_GEMV_ENTRY(q8_0, gemv_q8_0, ER_Q8_0_ROWS, 64, true, g)

extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)
er_gemv_q8_0_any(const uint8_t *__restrict__ W, const float *__restrict__ x,
                 float *__restrict__ y, uint32_t M, uint32_t K) {
    gemv_q8_0_any<2>(W, x, y, M, K);
}

// Q6_K top-1 over the fp32 family (rows the integer-dot kernels do not take):
// er_gemv_q6k_top1_l<LPR>_<s|g>, one partial per workgroup.
#define ER_GEMV_TOP1_ENTRY(lpr, xg, tag)                                                        \
    extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)                             \
        er_gemv_q6k_top1_l##lpr##_##tag(const uint8_t *__restrict__ W, const float *__restrict__ x, \
                                        float *__restrict__ pv, uint32_t *__restrict__ pi,        \
                                        uint32_t M, uint32_t K) {                                 \
        gemv_q6k<lpr, ER_Q6K_ROWS, xg, true>(W, x, nullptr, M, K, pv, pi);                       \
    }
ER_GEMV_TOP1_ENTRY(64, false, s)
ER_GEMV_TOP1_ENTRY(32, false, s)
ER_GEMV_TOP1_ENTRY(16, false, s)
ER_GEMV_TOP1_ENTRY(8, false, s)
ER_GEMV_TOP1_ENTRY(4, false, s)
ER_GEMV_TOP1_ENTRY(64, true, g)
ER_GEMV_TOP1_ENTRY(32, true, g)
ER_GEMV_TOP1_ENTRY(16, true, g)
ER_GEMV_TOP1_ENTRY(8, true, g)
ER_GEMV_TOP1_ENTRY(4, true, g)

// Q4_K dual GeGLU for rows longer than the integer-dot kernels cover: fp32
// kernel, x from global memory, ER_Q4K_ROWS / 2 output rows per lane group.
extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)
er_gemv_q4k_geglu_l64_g(const uint8_t *__restrict__ Wg, const uint8_t *__restrict__ Wu,
                        const float *__restrict__ x, float *__restrict__ y, uint32_t M, uint32_t K) {
    gemv_q4k<64, ER_Q4K_ROWS, true, ER_EPI_GEGLU>(Wg, x, y, M, K, Wu);
}

// Fused Q8_0 row lists and gate/up SiLU pairs for any K % 32 == 0: 2 rows
// (ROWS) or 2 gate/up pairs (SILU) per wave.
extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)
er_gemv_q8_0_any_multi(Q8Multi mm, const float *__restrict__ x, uint32_t K) {
    gemv_q8_0_any_fused<2, ER_EPI_Q8_ROWS>(mm, x, K);
}
extern "C" __global__ void __launch_bounds__(ER_GEMV_THREADS)
er_gemv_q8_0_any_silu(Q8Multi mm, const float *__restrict__ x, uint32_t K) {
    gemv_q8_0_any_fused<4, ER_EPI_Q8_SILU>(mm, x, K);
}
