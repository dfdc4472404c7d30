// er_hip.cpp -- host side of the EdgeRunnerHIP C ABI (include/er_hip.h).
// Built a second time with -DER_WITH_PROBES (and the code object built the
// same way) as libedgerunner_probe.so, the measurement library: the same
// entry points plus er_hip_probe.h.
//
// The gfx950 code object is embedded in this library at build time
// (er_blob.S) and loaded with hipModuleLoadData; kernels are resolved by name
// once per context (the KernelRegistry.pipeline(for:) analogue,
// Sources/EdgeRunnerMetal/KernelRegistry.swift:38-49) and launched with
// hipModuleLaunchKernel on the caller's stream.  Shape validation reproduces
// GEMVKernel.validateKQuantInputShape / encodeKQuantWeights
// (Sources/EdgeRunnerMetal/GEMVKernel.swift:1276-1300, 1415-1432) and the
// Dequant*Kernel.dequantise checks (Sources/EdgeRunnerIO/DequantQ4KMKernel.swift:23-29).
#include "er_hip.h"
#ifdef ER_WITH_PROBES
#include "er_hip_probe.h"
#endif
#include "er_error.h"
#include "er_gemv_cfg.h"
#include "er_scratch.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>

extern "C" const unsigned char er_kernels_blob[];
extern "C" const unsigned char er_kernels_blob_end[];

namespace er_detail {

thread_local char g_last_error[512] = "";

er_status fail(er_status st, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return st;
}

}  // namespace er_detail

namespace {

using er_detail::fail;

// Kernel table: every kernel the library launches, resolved at create time.
// The integer-dot GEMV kernels (one per er_gemv_cfg.h entry and format) are
// listed separately in kI8Cfg.
#define ER_KERNEL_LIST(X)                                                              \
    X(DEQUANT_Q8_0, "er_dequant_q8_0")                                                 \
    X(DEQUANT_Q4_K, "er_dequant_q4_k")                                                 \
    X(DEQUANT_Q6_K, "er_dequant_q6_k")                                                 \
    X(GEMV_Q6K_L64_S, "er_gemv_q6k_l64_s")                                             \
    X(GEMV_Q6K_L32_S, "er_gemv_q6k_l32_s")                                             \
    X(GEMV_Q6K_L16_S, "er_gemv_q6k_l16_s")                                             \
    X(GEMV_Q6K_L8_S, "er_gemv_q6k_l8_s")                                               \
    X(GEMV_Q6K_L4_S, "er_gemv_q6k_l4_s")                                               \
    X(GEMV_Q6K_L64_G, "er_gemv_q6k_l64_g")                                             \
    X(GEMV_Q6K_L32_G, "er_gemv_q6k_l32_g")                                             \
    X(GEMV_Q6K_L16_G, "er_gemv_q6k_l16_g")                                             \
    X(GEMV_Q6K_L8_G, "er_gemv_q6k_l8_g")                                               \
    X(GEMV_Q6K_L4_G, "er_gemv_q6k_l4_g")                                               \
    X(GEMV_Q4K_L64_G, "er_gemv_q4k_l64_g")                                             \
    X(GEMV_Q8_0_L64_G, "er_gemv_q8_0_l64_g")                                           \
    X(GEMV_Q8_0_ANY, "er_gemv_q8_0_any")                                               \
    X(GEMV_Q6K_TOP1_L64_S, "er_gemv_q6k_top1_l64_s")                                   \
    X(GEMV_Q6K_TOP1_L32_S, "er_gemv_q6k_top1_l32_s")                                   \
    X(GEMV_Q6K_TOP1_L16_S, "er_gemv_q6k_top1_l16_s")                                   \
    X(GEMV_Q6K_TOP1_L8_S, "er_gemv_q6k_top1_l8_s")                                     \
    X(GEMV_Q6K_TOP1_L4_S, "er_gemv_q6k_top1_l4_s")                                     \
    X(GEMV_Q6K_TOP1_L64_G, "er_gemv_q6k_top1_l64_g")                                   \
    X(GEMV_Q6K_TOP1_L32_G, "er_gemv_q6k_top1_l32_g")                                   \
    X(GEMV_Q6K_TOP1_L16_G, "er_gemv_q6k_top1_l16_g")                                   \
    X(GEMV_Q6K_TOP1_L8_G, "er_gemv_q6k_top1_l8_g")                                     \
    X(GEMV_Q6K_TOP1_L4_G, "er_gemv_q6k_top1_l4_g")                                     \
    X(GEMV_Q4K_GEGLU_L64_G, "er_gemv_q4k_geglu_l64_g")                                 \
    X(GEMV_Q8_0_ANY_MULTI, "er_gemv_q8_0_any_multi")                                   \
    X(GEMV_Q8_0_ANY_SILU, "er_gemv_q8_0_any_silu")                                     \
    X(GEMM_Q4K_T128, "er_gemm_q4k_t128")                                               \
    X(GEMM_Q4K_T256, "er_gemm_q4k_t256")                                               \
    X(GEMM_Q8_0_T128, "er_gemm_q8_0_t128")                                             \
    X(GEMM_Q8_0_T256, "er_gemm_q8_0_t256")                                             \
    X(GEMMP_Q4K_T64, "er_gemmp_q4k_t64")                                               \
    X(GEMMP_Q8_0_T64, "er_gemmp_q8_0_t64")                                             \
    X(FILL_ZERO, "er_fill_zero")                                                       \
    X(TOP1_REDUCE, "er_top1_reduce")                                                   \
    X(QUANT_Q8_0_V, "er_quantize_q8_0_rows_v")                                         \
    X(QUANT_Q8_0_S, "er_quantize_q8_0_rows_s")                                         \
    X(GEMMP_Q4K_T128, "er_gemmp_q4k_t128")                                             \
    X(GEMMP_Q4K_T256, "er_gemmp_q4k_t256")                                             \
    X(GEMMP_Q8_0_T128, "er_gemmp_q8_0_t128")                                           \
    X(GEMMP_Q8_0_T256, "er_gemmp_q8_0_t256")                                           \
    X(GEMMW_Q4K_T128, "er_gemmw_q4k_t128")                                             \
    X(GEMMW_Q8_0_T128, "er_gemmw_q8_0_t128")                                           \
    X(GEMML_Q4K, "er_gemml_q4k")                                                       \
    X(GEMML_Q8_0, "er_gemml_q8_0")                                                     \
    X(GEMML_Q4K_R1, "er_gemml_q4k_r1")                                                 \
    X(GEMML_Q8_0_R1, "er_gemml_q8_0_r1")                                               \
    ER_PROBE_KERNEL_LIST(X)

#ifdef ER_WITH_PROBES
#define ER_PROBE_KERNEL_LIST(X)                                                        \
    X(GEMML_Q4K_STAMPED, "er_gemml_q4k_stamped")                                       \
    X(GEMML_Q8_0_STAMPED, "er_gemml_q8_0_stamped")                                     \
    X(GEMML_Q4K_R1_STAMPED, "er_gemml_q4k_r1_stamped")                                 \
    X(GEMML_Q8_0_R1_STAMPED, "er_gemml_q8_0_r1_stamped")                               \
    X(PROBE_STREAM_READ, "er_probe_stream_read")                                       \
    X(PROBE_EMPTY, "er_probe_empty")                                                   \
    X(PROBE_GRID_BARRIER, "er_probe_grid_barrier")                                     \
    X(PROBE_LDS_READ, "er_probe_lds_read")                                             \
    X(PROBE_MFMA_VALU, "er_probe_mfma_valu")
#else
#define ER_PROBE_KERNEL_LIST(X)
#endif

enum KernelId {
#define ER_ENUM(id, name) K_##id,
    ER_KERNEL_LIST(ER_ENUM)
#undef ER_ENUM
        K_COUNT
};

const char *const kKernelNames[K_COUNT] = {
#define ER_NAME(id, name) name,
    ER_KERNEL_LIST(ER_NAME)
#undef ER_NAME
};

// Rows per lane group of the fp32 GEMV family; must match ER_*_ROWS in er_gemv.hip.
constexpr uint32_t kQ4KRows = 4;
constexpr uint32_t kQ6KRows = 2;
constexpr uint32_t kQ8_0Rows = 2;
constexpr uint32_t kGemvThreads = 64u * ER_GEMV_WAVES;
constexpr uint64_t kLdsXLimit = 64u * 1024u;  // bytes of fp32 x staged in LDS

// Integer-dot GEMV configurations {LPR, NS, R} (er_gemv_cfg.h).
struct I8Cfg {
    uint8_t lpr, ns, r;
};
#define ER_I8_ROW(LPR, NS, R) {LPR, NS, R},
constexpr I8Cfg kI8Cfg[] = {ER_I8_CONFIGS(ER_I8_ROW)};
#undef ER_I8_ROW
constexpr int kI8Count = (int)(sizeof(kI8Cfg) / sizeof(kI8Cfg[0]));
// Integer-dot kernels stage 3K + K/4 + K/8 bytes of x in LDS (limb planes,
// chunk sums, group scales and conditioning marks, er_xlimbs.h); rows up to
// this length use them (the default dynamic LDS limit is 64 KiB).
constexpr uint32_t kI8MaxK = 16384;
constexpr uint32_t xl_lds_bytes(uint32_t K) { return 3u * K + (K / 16u) * 4u + (K / 64u) * 8u; }

// CU-resident Q4_K / Q8_0 / Q6_K configurations {LPR, NS, MAXJ} (er_gemv_cfg.h): kernels
// for 1..maxJ unrolled steps, and a rolled one when maxJ == ER_CU_MAX_STEPS.
struct CuCfg {
    uint8_t lpr, ns, maxJ;
};
#define ER_CU_ROW(LPR, NS, MAXJ) {LPR, NS, MAXJ},
constexpr CuCfg kCuCfgQ4K[] = {ER_CU_CONFIGS_Q4K(ER_CU_ROW)};
constexpr CuCfg kCuCfgQ8[] = {ER_CU_CONFIGS_Q8(ER_CU_ROW)};
constexpr CuCfg kCuCfgQ6K[] = {ER_CU_CONFIGS_Q6K(ER_CU_ROW)};
#undef ER_CU_ROW
constexpr int kCuCountQ4K = (int)(sizeof(kCuCfgQ4K) / sizeof(kCuCfgQ4K[0]));
constexpr int kCuCountQ8 = (int)(sizeof(kCuCfgQ8) / sizeof(kCuCfgQ8[0]));
constexpr int kCuCountQ6K = (int)(sizeof(kCuCfgQ6K) / sizeof(kCuCfgQ6K[0]));
// The CU-resident family covers Q4_K rows of up to 256 slots and Q8_0 / Q6_K
// rows of up to 64 (pick_cu finds no configuration beyond), and holds limbs plus raw x
// in LDS: 3K + K/4 + K/8 + 4K bytes.
constexpr uint32_t kCuMaxK = 16384;
constexpr uint32_t cu_lds_bytes(uint32_t K) { return xl_lds_bytes(K) + 4u * K; }

// Multi-matrix / GeGLU Q4_K configurations {LPR, NS, R} (er_gemv_cfg.h).
#define ER_I8_ROW(LPR, NS, R) {LPR, NS, R},
constexpr I8Cfg kI8MultiCfg[] = {ER_I8_MULTI_CONFIGS(ER_I8_ROW)};
#undef ER_I8_ROW
constexpr int kI8MultiCount = (int)(sizeof(kI8MultiCfg) / sizeof(kI8MultiCfg[0]));
// ... and the one-row forms of the unpaired multi-matrix kernels.
#define ER_I8_ROW(LPR, NS, R) {LPR, NS, R},
constexpr I8Cfg kI8Multi1Cfg[] = {ER_I8_MULTI1_CONFIGS(ER_I8_ROW)};
#undef ER_I8_ROW
constexpr int kI8Multi1Count = (int)(sizeof(kI8Multi1Cfg) / sizeof(kI8Multi1Cfg[0]));

// Kernel argument block of er_gemv_q4k_multi_* (matches Q4Multi in er_gemv.hip).
struct Q4MultiArgs {
    const void *W[3];
    void *y[3];
    uint32_t M[3];
};

// Kernel argument block of er_gemv_q8_0_multi_* (matches Q8Multi in er_gemv.hip).
struct Q8MultiArgs {
    const void *W[3];
    void *y[3];
    const float *res[3];
    uint32_t M[3];
    uint32_t halfMask;
    const float *normW;
    float eps;
};

}  // namespace

struct er_hip_ctx {
    int device = 0;
    hipModule_t module = nullptr;
    hipFunction_t fn[K_COUNT] = {};
    hipFunction_t fnQ4KI8[kI8Count] = {};
    hipFunction_t fnQ8I8[kI8Count] = {};
    hipFunction_t fnQ6KI8[kI8Count] = {};
    hipFunction_t fnQ6KTop1[kI8Count] = {};
    hipFunction_t fnQ4KCu[kCuCountQ4K][ER_CU_MAX_STEPS + 1] = {};  // [steps - 1]; [ER_CU_MAX_STEPS]: rolled
    hipFunction_t fnQ8Cu[kCuCountQ8][ER_CU_MAX_STEPS + 1] = {};
    hipFunction_t fnQ6KCu[kCuCountQ6K][ER_CU_MAX_STEPS + 1] = {};
    hipFunction_t fnQ6KTop1Cu[kCuCountQ6K][ER_CU_MAX_STEPS + 1] = {};
    hipFunction_t fnQ4KCuk[3][ER_CUK_MAX_STEPS] = {};  // [2, 4, 8 rows per step][row steps - 1]
    hipFunction_t fnQ4KCukMulti[3][ER_CUK_MAX_STEPS] = {};  // the dual / triple over them
    hipFunction_t fnQ4KCukGeglu[3][ER_CUK_MAX_STEPS] = {};  // the dual GeGLU over them
    hipFunction_t fnQ8CukMulti[3][ER_CUK_MAX_STEPS] = {};   // the fused Q8_0 rows over them
    hipFunction_t fnQ8CukSilu[3][ER_CUK_MAX_STEPS] = {};    // the fused Q8_0 gate/up + SiLU
    hipFunction_t fnQ8Cuk[3][ER_CUK_MAX_STEPS] = {};
    hipFunction_t fnQ6KCuk[2][ER_CUK_MAX_STEPS] = {};      // [2, 4 rows per step][row steps - 1]
    hipFunction_t fnQ6KTop1Cuk[2][ER_CUK_MAX_STEPS] = {};  // even steps only for 2 rows per step
    hipFunction_t fnQ4KMulti[kI8MultiCount] = {};
    hipFunction_t fnQ4KGeglu[kI8MultiCount] = {};
    hipFunction_t fnQ8Multi[kI8MultiCount] = {};
    hipFunction_t fnQ8Silu[kI8MultiCount] = {};
    hipFunction_t fnQ4KMulti1[kI8Multi1Count] = {};  // one row computation per lane group
    hipFunction_t fnQ8Multi1[kI8Multi1Count] = {};
    int cu_count = 0;
    int i8_override = -1;  // ER_HIP_GEMV_CONFIG=lpr:ns:r (benchmark sweeps only)
    int multi_override = -1;  // ER_HIP_GEMV_MULTI_CONFIG=lpr:ns:r for the multi-matrix kernels (tests, sweeps)
    int multi1_override = -1;  // the same with r = 1: the one-row forms (their unpaired kinds only)
    int cu_mode = -1;      // ER_HIP_GEMV_CU: 0 never, 1 whenever it applies, unset: by shape
    int cuk_mode = -1;     // ER_HIP_GEMV_CUK: 0 never, 2 every K <= 16384, unset: K > 8192 (comparisons)
    int gemm_variant = 0;  // ER_HIP_GEMM_VARIANT=1: non-pipelined GEMM, =2: 256-thread pipelined,
                           // =3: warp-specialised, =4 / =5: loader-specialised with 256 / 128-row tiles
                           // wherever it applies (comparisons, tests)
    uint32_t gemm_tt = 0, gemm_sk = 0;  // ER_HIP_GEMM_TILE=tt:sk (benchmark sweeps only)
    int gemv_fp32 = 0;  // ER_HIP_GEMV_FP32=1 selects the fp32 GEMV family (benchmark comparison)
    // device address of this context's copy of the code object's er_scratch
    // array (er_scratch.hip), found once at creation; the allocation-free
    // entry points pass it to kernels in place of caller scratch buffers
    void *scratch = nullptr;
    er_device_info info{};
};

static_assert(ER_HIP_TOP1_NOALLOC_MAX_ROWS / 4u <= ER_SCRATCH_TOP1_PARTIALS,
              "the scratch array holds a partial for every 4 rows of the largest allocation-free head");

namespace {

er_status check_ctx(const er_hip_ctx *ctx) {
    if (!ctx) return fail(ER_ERR_INVALID_ARGUMENT, "null er_hip_ctx");
    return ER_OK;
}

er_status bind_device(const er_hip_ctx *ctx) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != ctx->device) {
        hipError_t e = hipSetDevice(ctx->device);
        if (e != hipSuccess)
            return fail(ER_ERR_DEVICE, "hipSetDevice(%d): %s", ctx->device, hipGetErrorString(e));
    }
    return ER_OK;
}

er_status launch(const er_hip_ctx *ctx, KernelId k, dim3 grid, dim3 block, uint32_t lds,
                 er_stream stream, void **args) {
    hipError_t e = hipModuleLaunchKernel(ctx->fn[k], grid.x, grid.y, grid.z, block.x, block.y,
                                         block.z, lds, (hipStream_t)stream, args, nullptr);
    if (e != hipSuccess)
        return fail(ER_ERR_ENCODING_FAILED, "hipModuleLaunchKernel(%s): %s", kKernelNames[k],
                    hipGetErrorString(e));
    return ER_OK;
}

er_status launch_fn(hipFunction_t f, const char *name, dim3 grid, dim3 block, uint32_t lds,
                    er_stream stream, void **args) {
    hipError_t e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, lds,
                                         (hipStream_t)stream, args, nullptr);
    if (e != hipSuccess)
        return fail(ER_ERR_ENCODING_FAILED, "hipModuleLaunchKernel(%s): %s", name, hipGetErrorString(e));
    return ER_OK;
}

// Lane-group width L (lanes per row) and slots per lane N = ceil(S / L) for
// S slots and M rows, N <= maxN.  Among the widths whose one-row-per-group
// grid (R = 1) gives at least every other CU a workgroup, the one with the
// fewest idle slot lanes; when none does (short matrices, latency-bound), the
// one with the most workgroups.  Sets L = 0 when no width fits.
void pick_lanes(uint32_t S, uint32_t M, uint32_t maxN, int cu, uint32_t &L, uint32_t &N) {
    static const uint32_t lprs[] = {64, 32, 16, 4};
    uint32_t bestWaste = 0xffffffffu;
    uint64_t bestWgs = 0;
    bool bestFull = false;
    L = N = 0;
    for (uint32_t l : lprs) {
        const uint32_t n = (S + l - 1) / l;
        if (n > maxN) continue;
        const uint32_t waste = l * n - S;
        const uint64_t rowsPerWg = (uint64_t)ER_GEMV_WAVES * (64u / l);
        const uint64_t wgs = ((uint64_t)M + rowsPerWg - 1) / rowsPerWg;
        const bool full = 2u * wgs >= (uint64_t)cu;
        bool better;
        if (full)
            better = !bestFull || waste < bestWaste;
        else
            better = !bestFull && (wgs > bestWgs || (wgs == bestWgs && waste < bestWaste));
        if (L == 0 || better) {
            L = l;
            N = n;
            bestWaste = waste;
            bestWgs = wgs;
            bestFull = full;
        }
    }
}

// Rows per lane group R for a launch of the integer-dot kernels, counting the
// workgroups of all its tokens: the most workgroups that fit one per CU, or,
// when even the fewest do not fit, the fewest; equal counts go to fewer rows
// per lane group.  At these sizes a launch is latency-bound, and a second,
// partial round of workgroups cost more than the rounds' extra parallelism
// gave.  Same-box A/B against the earlier rule (the most rows per lane group
// that still give every CU two workgroups per token, else R = 1): one token,
// Q4_K 5120-8192 x 1024 and 3072-3584 x 2048 17-18% faster at 2 rows,
// 12288-16384 x 1024 and 8192 x 2048 10-14% faster at 4 rows; 2-8 tokens of
// 2048-4096 x 1024, 11-18% faster.
struct I8Cand {
    int idx;       // index into its configuration table
    uint32_t r;    // rows per lane group
    uint64_t wgs;  // workgroups, all tokens
};
template <size_t N>
int pick_rows(const I8Cand (&c)[N], int n, int cu) {
    int best = -1, fewest = -1;
    for (int k = 0; k < n; ++k) {
        if (c[k].wgs <= (uint64_t)cu &&
            (best < 0 || c[k].wgs > c[best].wgs || (c[k].wgs == c[best].wgs && c[k].r < c[best].r)))
            best = k;
        if (fewest < 0 || c[k].wgs < c[fewest].wgs || (c[k].wgs == c[fewest].wgs && c[k].r > c[fewest].r))
            fewest = k;
    }
    return best >= 0 ? best : fewest;
}

// Picks the integer-dot configuration for a row of S 64-weight slots, M rows
// and `tokens` tokens: the lane split (LPR, NS) of pick_lanes for one token's
// rows -- so a row's arithmetic (its slots per lane and lane reduction) is the
// same for batched and per-token calls -- then the rows per lane group of
// pick_rows over all tokens' workgroups.  Returns -1 when no configuration
// covers S.
int pick_i8(uint32_t S, uint32_t M, int cu, uint32_t tokens) {
    uint32_t bestL = 0, bestN = 0;
    pick_lanes(S, M, 8, cu, bestL, bestN);
    if (!bestL) return -1;
    const uint32_t G = 64u / bestL;
    I8Cand c[8];
    int n = 0;
    for (int i = 0; i < kI8Count && n < 8; ++i) {
        if (kI8Cfg[i].lpr != bestL || kI8Cfg[i].ns != bestN) continue;
        const uint32_t rows = ER_GEMV_WAVES * G * kI8Cfg[i].r;
        c[n++] = I8Cand{i, kI8Cfg[i].r, ((uint64_t)M + rows - 1) / rows * std::max<uint32_t>(tokens, 1u)};
    }
    const int k = n ? pick_rows(c, n, cu) : -1;
    return k < 0 ? -1 : c[k].idx;
}

// Multi-matrix / GeGLU configuration for S slots, Mt total row computations
// and `tokens` tokens: as pick_i8 (lane split from one token's rows), over
// kI8MultiCfg (R in {4, 2}) and, when
// the kernel's rows stand alone (r1Ok), the one-row forms kI8Multi1Cfg.  Sets
// ci (kI8MultiCfg) or ci1 (kI8Multi1Cfg); both -1 when nothing covers S.
struct MultiPick {
    int ci = -1, ci1 = -1;
};
MultiPick pick_i8_multi(uint32_t S, uint32_t Mt, int cu, bool r1Ok, uint32_t tokens) {
    MultiPick p;
    uint32_t bestL = 0, bestN = 0;
    pick_lanes(S, Mt, 4, cu, bestL, bestN);
    if (!bestL) return p;
    const uint32_t G = 64u / bestL, T = std::max<uint32_t>(tokens, 1u);
    I8Cand c[8];
    bool one[8];
    int n = 0;
    for (int i = 0; i < kI8MultiCount && n < 8; ++i) {
        if (kI8MultiCfg[i].lpr != bestL || kI8MultiCfg[i].ns != bestN) continue;
        const uint32_t rows = ER_GEMV_WAVES * G * kI8MultiCfg[i].r;
        one[n] = false;
        c[n++] = I8Cand{i, kI8MultiCfg[i].r, ((uint64_t)Mt + rows - 1) / rows * T};
    }
    for (int i = 0; r1Ok && i < kI8Multi1Count && n < 8; ++i) {
        if (kI8Multi1Cfg[i].lpr != bestL || kI8Multi1Cfg[i].ns != bestN) continue;
        const uint32_t rows = ER_GEMV_WAVES * G;
        one[n] = true;
        c[n++] = I8Cand{i, 1u, ((uint64_t)Mt + rows - 1) / rows * T};
    }
    const int k = n ? pick_rows(c, n, cu) : -1;
    if (k >= 0) (one[k] ? p.ci1 : p.ci) = c[k].idx;
    return p;
}

// pick_i8_multi, or the context's forced configuration when it covers S slots.
MultiPick pick_multi(const er_hip_ctx *ctx, uint32_t S, uint32_t Mt, bool r1Ok, uint32_t tokens) {
    MultiPick p;
    const int o = ctx->multi_override, o1 = ctx->multi1_override;
    if (o >= 0 && (uint32_t)kI8MultiCfg[o].lpr * kI8MultiCfg[o].ns >= S) {
        p.ci = o;
        return p;
    }
    if (r1Ok && o1 >= 0 && (uint32_t)kI8Multi1Cfg[o1].lpr * kI8Multi1Cfg[o1].ns >= S) {
        p.ci1 = o1;
        return p;
    }
    return pick_i8_multi(S, Mt, ctx->cu_count, r1Ok, tokens);
}

// CU-resident configuration for S slots from cfg[0..count): the fewest idle
// slot lanes per row (LPR * NS - S), wider rows first on ties.  -1 when none
// covers S.
int pick_cu(const CuCfg *cfg, int count, uint32_t S) {
    int best = -1;
    uint32_t bestWaste = 0xffffffffu;
    for (int i = 0; i < count; ++i) {
        const uint32_t cover = (uint32_t)cfg[i].lpr * cfg[i].ns;
        if (cover < S) continue;
        const uint32_t waste = cover - S;
        if (best < 0 || waste < bestWaste || (waste == bestWaste && cfg[i].lpr > cfg[best].lpr)) {
            best = i;
            bestWaste = waste;
        }
    }
    return best;
}

bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Largest power of two in [4, 64] dividing the slot count (4 when none does).
uint32_t lanes_per_row(uint32_t slots) {
    uint32_t l = 64;
    while (l > 4 && (slots % l) != 0) l >>= 1;
    return l;
}

int lpr_index(uint32_t lpr) {
    switch (lpr) {
        case 64: return 0;
        case 32: return 1;
        case 16: return 2;
        case 8: return 3;
        default: return 4;
    }
}

enum class Fmt { Q8_0, Q4_K, Q6_K };

uint32_t block_bytes(Fmt f) {
    return f == Fmt::Q8_0 ? ER_Q8_0_BLOCK_BYTES
                          : (f == Fmt::Q4_K ? ER_Q4_K_BLOCK_BYTES : ER_Q6_K_BLOCK_BYTES);
}
uint32_t block_weights(Fmt f) {
    return f == Fmt::Q8_0 ? ER_Q8_0_BLOCK_WEIGHTS : ER_K_BLOCK_WEIGHTS;
}
const char *fmt_name(Fmt f) {
    return f == Fmt::Q8_0 ? "Q8_0" : (f == Fmt::Q4_K ? "Q4_K" : "Q6_K");
}

// validateKQuantInputShape (GEMVKernel.swift:1415-1432) plus the buffer-length
// guard of encodeKQuantWeights / encodeBatchedKQuantWeights (:1296-1300, :1339-1344).
er_status validate_gemv_shape(Fmt f, er_buffer W, uint64_t xLen, uint64_t yLen, uint32_t batch,
                              uint32_t M, uint32_t K) {
    const uint32_t bw = block_weights(f);
    if (K == 0 || K % bw != 0)
        return fail(ER_ERR_INVALID_VECTOR_SHAPE, "%s GEMV: K=%u must be a positive multiple of %u",
                    fmt_name(f), K, bw);
    const uint64_t expected = (uint64_t)M * (K / bw) * block_bytes(f);
    if (W.length < expected)
        return fail(ER_ERR_INVALID_MATRIX_SHAPE,
                    "%s GEMV: weight buffer holds %llu bytes, M=%u K=%u needs %llu", fmt_name(f),
                    (unsigned long long)W.length, M, K, (unsigned long long)expected);
    if (batch == 0) return fail(ER_ERR_ENCODING_FAILED, "%s GEMV: batchSeq must be > 0", fmt_name(f));
    if (xLen < (uint64_t)batch * K * 4u || yLen < (uint64_t)batch * M * 4u)
        return fail(ER_ERR_ENCODING_FAILED,
                    "%s GEMV: input %llu B / output %llu B too small for batch=%u M=%u K=%u",
                    fmt_name(f), (unsigned long long)xLen, (unsigned long long)yLen, batch, M,
                    K);
    return ER_OK;
}

// validate_gemv_shape, then the pointer rules of the kernels.
er_status validate_gemv(Fmt f, er_buffer W, er_buffer x, er_buffer y, uint32_t batch, uint32_t M,
                        uint32_t K) {
    er_status st = validate_gemv_shape(f, W, x.length, y.length, batch, M, K);
    if (st != ER_OK || M == 0) return st;
    if (!W.data || !x.data || !y.data)
        return fail(ER_ERR_INVALID_ARGUMENT, "%s GEMV: null buffer", fmt_name(f));
    if (!aligned(W.data, 16))
        return fail(ER_ERR_INVALID_ARGUMENT, "%s GEMV: weight pointer must be 16-byte aligned",
                    fmt_name(f));
    if (!aligned(x.data, 16) || !aligned(y.data, 4))
        return fail(ER_ERR_INVALID_ARGUMENT,
                    "%s GEMV: input must be 16-byte and output 4-byte aligned", fmt_name(f));
    return ER_OK;
}

// CU-resident family (er_gemv.hip gemv_cu) for one call: rows of K % 256 == 0
// up to kCuMaxK with a configuration covering K / 64 slots.  Q4_K / Q8_0 take
// it when a CU's share of one token's rows is 3 row steps or more (Q4_K rows
// longer than 8192 weights, whose per-workgroup x staging the lane-group
// family repeats ~512 times, at any share; these reach this plan only when the
// K-sliced kernels are switched off), beyond the unrolled kernels' steps as
// several workgroups per CU with the steps split evenly; their rolled loop
// measured no faster than the lane-group family and runs only when
// ER_HIP_GEMV_CU=1 forces the family.  Q6_K takes it at 3 steps or more, the
// rolled kernel beyond ER_CU_MAX_STEPS steps (the lane-group Q6_K kernel
// waits for its weight loads before converting x).  The choice of configuration
// and family depends on M and K only, so a batched call, its per-token calls
// and the Q6_K top-1 over the same matrix run the same per-row arithmetic;
// the batch only changes the row partition (about one workgroup per CU over
// all tokens).
struct CuPlan {
    int ci = -1;             // configuration index
    int slot = 0;            // steps - 1, or ER_CU_MAX_STEPS for the rolled kernel
    uint32_t rowsPerWg = 0;  // step rows x steps
};
// Steps per workgroup for `need` steps of rows per CU and kernels of at most
// maxSteps: the need split evenly over the fewest workgroups that hold it, so
// every CU gets the same number of workgroups (28672 x 4096 Q4_K: 14 steps as
// 2 x 7, 512 workgroups, instead of 8 + 6 as 448, of which 64 CUs got one).
uint32_t even_steps(uint32_t need, uint32_t maxSteps) {
    const uint32_t parts = (need + maxSteps - 1u) / maxSteps;
    return std::max<uint32_t>(1u, (need + parts - 1u) / parts);
}

bool plan_cu(const er_hip_ctx *ctx, Fmt f, uint32_t M, uint32_t K, uint32_t batch, CuPlan &p) {
    if (K % 256u != 0 || K > kCuMaxK || ctx->gemv_fp32 != 0 || ctx->i8_override >= 0 || ctx->cu_mode == 0 ||
        (uint64_t)cu_lds_bytes(K) + 1024u > ctx->info.lds_per_workgroup || batch == 0)
        return false;
    const CuCfg *cfg = f == Fmt::Q4_K ? kCuCfgQ4K : (f == Fmt::Q8_0 ? kCuCfgQ8 : kCuCfgQ6K);
    const int ci = pick_cu(cfg, f == Fmt::Q4_K ? kCuCountQ4K : (f == Fmt::Q8_0 ? kCuCountQ8 : kCuCountQ6K), K / 64u);
    if (ci < 0) return false;
    const CuCfg &c = cfg[ci];
    const uint32_t step = ER_CU_WAVES * (64u / c.lpr);  // rows per workgroup step
    const uint32_t cu = (uint32_t)ctx->cu_count;
    const uint32_t needed1 = ((M + cu - 1u) / cu + step - 1u) / step;  // steps per CU, one token
    const bool rolled = c.maxJ == ER_CU_MAX_STEPS;
    // Q4_K / Q8_0 by default: the unrolled kernels at any share of 3 steps or
    // more, beyond maxJ as several workgroups per CU (their rolled loop measured
    // no faster than the lane-group kernels; split evenly, the unrolled ones
    // took Q8_0 20480 / 28672 x 4096 from 18.3 / 23.5 to 16.5 / 22.1 us)
    const bool use = ctx->cu_mode == 1 ? (rolled || needed1 <= c.maxJ)
                     : f == Fmt::Q6_K  ? (needed1 >= 3u && (rolled || needed1 <= c.maxJ))
                                       : (needed1 >= 3u || K > 8192u);
    if (!use) return false;
    // unrolled kernels up to maxJ steps, the rolled one (Q6_K, or any format
    // when the family is forced) up to ER_CU_MAX_ROLLED, more workgroups
    // beyond (a CU's steps split evenly over them)
    const uint32_t perToken = std::max<uint32_t>(1u, cu / batch);
    const uint32_t maxSteps = rolled && (f == Fmt::Q6_K || ctx->cu_mode == 1) ? ER_CU_MAX_ROLLED : c.maxJ;
    const uint32_t steps = even_steps(((M + perToken - 1u) / perToken + step - 1u) / step, maxSteps);
    p.ci = ci;
    p.rowsPerWg = step * steps;
    p.slot = steps <= ER_CU_MAX_STEPS ? (int)steps - 1 : ER_CU_MAX_STEPS;
    return true;
}

// K-sliced CU-resident kernels (er_gemv.hip gemv_cuk), PAR = 2, 4 or 8 rows per
// workgroup step as the row has up to 256, 128 or 64 slots (each wave's slice
// then fills 16 of 32, 9 of 16 ... all lanes of its row slices), up to
// ER_CUK_MAX_STEPS steps, about one workgroup per CU for one
// token's rows (more beyond).  Taken by default for Q4_K / Q8_0 rows of
// 4096 < K <= 16384 weights at any M, and for Q4_K rows of K = 4096 when one
// token's rows give each CU at least 8 (A/B in one process against the
// whole-row kernels: 2048 / 8192 / 14336 / 28672 x 4096 -7 / -3 / -1 / -9%,
// 1024 x 4096 +11%; Q8_0 14336 x 4096 +1.6%, so Q8_0 keeps its spread kernel
// there).  ER_HIP_GEMV_CUK=2 takes them for every K <= 16384 (K % 256 == 0),
// =0 never, and ER_HIP_GEMV_CU=0/1 (lane-group / whole-row CU kernels forced)
// turns them off.  The choice depends on M and K alone, and a row's value on
// K alone.  Q6_K takes them for rows of 4096 < K <= 16384 when one token's
// rows fill at most one workgroup per CU (4096 x 14336: 13.5 against 18.3 us
// on the lane-group kernels; 128256 x 4096 heads ran 17% slower over 8
// workgroups per CU), and its top-1 follows the same plan.
struct CukPlan {
    int pi = 0;              // PAR = 2 << pi
    int j = 0;               // row steps per lane group
    uint32_t rowsPerWg = 0;  // PAR j
};
bool plan_cuk(const er_hip_ctx *ctx, Fmt f, uint32_t M, uint32_t K, uint32_t batch, CukPlan &p,
              bool rows64 = false) {
    if (K % 256u != 0 || K > 16384u || ctx->gemv_fp32 != 0 || ctx->i8_override >= 0 ||
        ctx->cu_mode >= 0 || ctx->cuk_mode == 0 || batch == 0 ||
        (uint64_t)xl_lds_bytes(K) + 1024u > ctx->info.lds_per_workgroup)
        return false;
    const uint32_t S = K / 64u, cu = (uint32_t)ctx->cu_count, rows1 = (M + cu - 1u) / cu;
    p.pi = S <= 64u ? 2 : (S <= 128u ? 1 : 0);
    const uint32_t par = 2u << p.pi, maxJ = (uint32_t)ER_CUK_MAX_STEPS;
    if (f == Fmt::Q6_K ? (S <= 64u || rows1 > par * maxJ)
                       : (ctx->cuk_mode != 2 && (S < 64u || (S == 64u && !rows64 && (f != Fmt::Q4_K || rows1 < 8u)))))
        return false;
    const uint32_t perToken = std::max<uint32_t>(1u, cu / batch);
    const uint32_t rows = (M + perToken - 1u) / perToken;  // per CU, one token
    p.j = (int)even_steps(std::max<uint32_t>(1u, (rows + par - 1u) / par), maxJ);
    p.rowsPerWg = par * (uint32_t)p.j;
    return true;
}

er_status encode_gemv(er_hip_ctx *ctx, er_stream stream, Fmt f, er_buffer W, er_buffer x,
                      er_buffer y, uint32_t batch, uint32_t M, uint32_t K) {
    // shape validation first (it needs no device), then the context
    er_status st = validate_gemv(f, W, x, y, batch, M, K);
    if (st != ER_OK) return st;
    st = check_ctx(ctx);
    if (st != ER_OK || M == 0) return st;
    if (batch > 65535u)
        return fail(ER_ERR_ENCODING_FAILED, "GEMV: batchSeq %u exceeds the grid limit 65535", batch);
    st = bind_device(ctx);
    if (st != ER_OK) return st;

    void *args[] = {&W.data, &x.data, &y.data, &M, &K};
    const bool q8Aligned = f == Fmt::Q8_0 && K % 64u == 0;
    CukPlan kp;
    if (plan_cuk(ctx, f, M, K, batch, kp)) {
        dim3 grid((M + kp.rowsPerWg - 1u) / kp.rowsPerWg, batch, 1);
        void *kargs[] = {&W.data, &x.data, &y.data, &M, &K};
        return launch_fn(f == Fmt::Q4_K   ? ctx->fnQ4KCuk[kp.pi][kp.j - 1]
                         : f == Fmt::Q8_0 ? ctx->fnQ8Cuk[kp.pi][kp.j - 1]
                                          : ctx->fnQ6KCuk[kp.pi][kp.j - 1],
                         f == Fmt::Q4_K ? "er_gemv_q4k_cuk" : (f == Fmt::Q8_0 ? "er_gemv_q8_0_cuk" : "er_gemv_q6k_cuk"),
                         grid,
                         dim3(64u * ER_CU_WAVES, 1, 1), xl_lds_bytes(K), stream, kargs);
    }
    CuPlan cp;
    if (plan_cu(ctx, f, M, K, batch, cp)) {
        dim3 grid((M + cp.rowsPerWg - 1u) / cp.rowsPerWg, batch, 1);
        void *cargs[] = {&W.data, &x.data, &y.data, &M, &K, (void *)&cp.rowsPerWg};
        hipFunction_t fn = f == Fmt::Q4_K   ? ctx->fnQ4KCu[cp.ci][cp.slot]
                           : f == Fmt::Q8_0 ? ctx->fnQ8Cu[cp.ci][cp.slot]
                                            : ctx->fnQ6KCu[cp.ci][cp.slot];
        return launch_fn(fn, f == Fmt::Q4_K ? "er_gemv_q4k_cu" : (f == Fmt::Q8_0 ? "er_gemv_q8_0_cu" : "er_gemv_q6k_cu"),
                         grid, dim3(64u * ER_CU_WAVES, 1, 1), cu_lds_bytes(K), stream, cargs);
    }
    if ((f != Fmt::Q8_0 || q8Aligned) && K <= kI8MaxK && ctx->gemv_fp32 == 0) {
        int ci = pick_i8(K / 64u, M, ctx->cu_count, batch);
        if (ctx->i8_override >= 0 && (uint32_t)kI8Cfg[ctx->i8_override].lpr *
                                             kI8Cfg[ctx->i8_override].ns >= K / 64u)
            ci = ctx->i8_override;
        if (ci >= 0) {
            const I8Cfg &c = kI8Cfg[ci];
            const uint32_t rowsPerBlock = ER_GEMV_WAVES * (64u / c.lpr) * c.r;
            const uint32_t lds = xl_lds_bytes(K);
            dim3 grid((M + rowsPerBlock - 1) / rowsPerBlock, batch, 1);
            hipFunction_t fn = f == Fmt::Q4_K ? ctx->fnQ4KI8[ci]
                                              : (f == Fmt::Q8_0 ? ctx->fnQ8I8[ci] : ctx->fnQ6KI8[ci]);
            return launch_fn(fn, f == Fmt::Q4_K ? "er_gemv_q4k_i8" : (f == Fmt::Q8_0 ? "er_gemv_q8_0_i8" : "er_gemv_q6k_i8"),
                             grid, dim3(kGemvThreads, 1, 1), lds, stream, args);
        }
    }
    if (f == Fmt::Q8_0 && !q8Aligned) {
        // odd number of Q8_0 blocks per row: generic kernel, one row group per wave
        const uint32_t rowsPerBlock = ER_GEMV_WAVES * 2u;
        dim3 grid((M + rowsPerBlock - 1) / rowsPerBlock, batch, 1);
        return launch(ctx, K_GEMV_Q8_0_ANY, grid, dim3(kGemvThreads, 1, 1), 0, stream, args);
    }
    if (f != Fmt::Q6_K) {
        // rows longer than the integer-dot kernels cover: fp32 kernel, x from global memory
        const uint32_t rows = f == Fmt::Q4_K ? kQ4KRows : kQ8_0Rows;
        const uint32_t rowsPerBlock = ER_GEMV_WAVES * rows;
        dim3 grid((M + rowsPerBlock - 1) / rowsPerBlock, batch, 1);
        return launch(ctx, f == Fmt::Q4_K ? K_GEMV_Q4K_L64_G : K_GEMV_Q8_0_L64_G, grid,
                      dim3(kGemvThreads, 1, 1), 0, stream, args);
    }
    const bool xg = (uint64_t)K * 4u > kLdsXLimit;
    const uint32_t lds = xg ? 0u : K * 4u;
    const uint32_t slots = (K / 256u) * 4u;
    const uint32_t lpr = lanes_per_row(slots);
    const KernelId k = (KernelId)(K_GEMV_Q6K_L64_S + lpr_index(lpr) + (xg ? 5 : 0));
    const uint32_t rowsPerBlock = ER_GEMV_WAVES * (64u / lpr) * kQ6KRows;
    dim3 grid((M + rowsPerBlock - 1) / rowsPerBlock, batch, 1);
    return launch(ctx, k, grid, dim3(kGemvThreads, 1, 1), lds, stream, args);
}

// GEMVKernel.execute* (GEMVKernel.swift:545-627, 1146-1162, 1363-1413): the
// reference's validation, then device x / y, one encode on the device's null
// stream, a wait and the copy-out.  Host-side allocation or copy failures are
// encodingFailed, as the reference's failed makeBuffer.
// The reference's order of the x.count and shape checks: the single-vector
// forms check x.count == K first (validateKQuantInputShape's vectorCount);
// the batched form runs the K and weight-size rules with vectorCount = K
// first, then batchSeq > 0 && x.count == batchSeq * K
// (executeBatchedQ4KWeights, GEMVKernel.swift:623-640).
er_status check_x_count(Fmt f, uint64_t wBytes, uint64_t xCount, uint32_t batch, bool batched, uint32_t M,
                        uint32_t K) {
    if (batched) {
        er_status st = validate_gemv_shape(f, er_buffer{nullptr, wBytes}, (uint64_t)K * 4u, (uint64_t)M * 4u, 1, M, K);
        if (st != ER_OK) return st;
    }
    if (batched ? (batch == 0 || xCount != (uint64_t)batch * K) : xCount != K)
        return fail(ER_ERR_INVALID_VECTOR_SHAPE, "%s execute: x.count %llu does not match K=%u x batch %u",
                    fmt_name(f), (unsigned long long)xCount, K, batch);
    return ER_OK;
}

er_status execute_gemv(er_hip_ctx *ctx, Fmt f, er_buffer W, const float *x, uint64_t xCount, float *y,
                       uint64_t yCount, uint32_t batch, bool batched, uint32_t M, uint32_t K) {
    if (er_status cs = check_x_count(f, W.length, xCount, batch, batched, M, K); cs != ER_OK) return cs;
    const uint64_t yNeed = (uint64_t)batch * M;
    er_status st = validate_gemv_shape(f, W, xCount * 4u, yNeed * 4u, batch, M, K);
    if (st != ER_OK) return st;
    if (yCount < yNeed)
        return fail(ER_ERR_ENCODING_FAILED, "%s execute: y holds %llu floats, %llu needed", fmt_name(f),
                    (unsigned long long)yCount, (unsigned long long)yNeed);
    st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!x || !y) return fail(ER_ERR_INVALID_ARGUMENT, "%s execute: null host array", fmt_name(f));
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    void *dx = nullptr, *dy = nullptr;
    const size_t xb = (size_t)xCount * 4u, yb = std::max<size_t>(4u, (size_t)yNeed * 4u);
    if (hipMalloc(&dx, std::max<size_t>(xb, 16u)) != hipSuccess || hipMalloc(&dy, yb) != hipSuccess) {
        if (dx) (void)hipFree(dx);
        return fail(ER_ERR_ENCODING_FAILED, "%s execute: device allocation of x / y failed", fmt_name(f));
    }
    hipError_t e = hipMemcpy(dx, x, xb, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        st = encode_gemv(ctx, nullptr, f, W, er_buffer{dx, xb}, er_buffer{dy, yb}, batch, M, K);
        if (st == ER_OK) {
            e = hipStreamSynchronize(nullptr);
            if (e == hipSuccess) e = hipMemcpy(y, dy, (size_t)yNeed * 4u, hipMemcpyDeviceToHost);
        }
    }
    (void)hipFree(dx);
    (void)hipFree(dy);
    if (st != ER_OK) return st;
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "%s execute: %s", fmt_name(f), hipGetErrorString(e));
    return ER_OK;
}

// The host-weight forms: the weights are validated as a buffer of raw_bytes,
// then copied to device memory for the call.
er_status execute_gemv_host(er_hip_ctx *ctx, Fmt f, const void *raw, uint64_t rawBytes, const float *x,
                            uint64_t xCount, float *y, uint64_t yCount, uint32_t batch, bool batched, uint32_t M,
                            uint32_t K) {
    if (er_status cs = check_x_count(f, rawBytes, xCount, batch, batched, M, K); cs != ER_OK) return cs;
    er_status st = validate_gemv_shape(f, er_buffer{nullptr, rawBytes}, xCount * 4u, (uint64_t)batch * M * 4u, batch,
                                       M, K);
    if (st != ER_OK) return st;
    if (yCount < (uint64_t)batch * M)
        return fail(ER_ERR_ENCODING_FAILED, "%s execute: y holds %llu floats, %llu needed", fmt_name(f),
                    (unsigned long long)yCount, (unsigned long long)batch * M);
    st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!raw) return fail(ER_ERR_INVALID_ARGUMENT, "%s execute: null weights", fmt_name(f));
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    void *dw = nullptr;
    if (hipMalloc(&dw, std::max<uint64_t>(rawBytes, 16u)) != hipSuccess)
        return fail(ER_ERR_ENCODING_FAILED, "%s execute: device allocation of %llu weight bytes failed", fmt_name(f),
                    (unsigned long long)rawBytes);
    hipError_t e = hipMemcpy(dw, raw, (size_t)rawBytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(dw);
        return fail(ER_ERR_DEVICE, "%s execute: weight upload: %s", fmt_name(f), hipGetErrorString(e));
    }
    st = execute_gemv(ctx, f, er_buffer{dw, rawBytes}, x, xCount, y, yCount, batch, batched, M, K);
    (void)hipFree(dw);
    return st;
}

// Greedy top-1 over a Q6_K head (GEMVKernel.encodeQ6KWeightsPackedTop1,
// GEMVKernel.swift:1205-1265): M % 4 == 0 (INVALID_MATRIX_SHAPE), then the
// K-quant shape rules, then partial buffers of >= M/4 entries and a 4-byte
// index buffer (ENCODING_FAILED).  Two launches: a Q6_K GEMV with the top-1
// epilogue (the CU-resident kernel when the plain GEMV over this matrix takes
// that family, else the lane-group one, so both compute the same row values;
// one partial per workgroup, at most M/4 of them) and er_top1_reduce.
er_status validate_q6k_top1(er_buffer W, er_buffer x, er_buffer out, uint32_t M, uint32_t K) {
    if (M % 4u != 0)
        return fail(ER_ERR_INVALID_MATRIX_SHAPE, "Q6_K top-1: M=%u must be a multiple of 4", M);
    er_status st = validate_gemv_shape(Fmt::Q6_K, W, x.length, (uint64_t)M * 4u, 1, M, K);
    if (st != ER_OK) return st;
    if (out.length < 4u)
        return fail(ER_ERR_ENCODING_FAILED, "Q6_K top-1: index buffer %llu B too small",
                    (unsigned long long)out.length);
    return ER_OK;
}

// The launches of a validated top-1 call, with the partials at pv / pi
// (room for M/4 entries each).
er_status launch_q6k_top1(er_hip_ctx *ctx, er_stream stream, er_buffer W, er_buffer x, void *pv, void *pi,
                          er_buffer out, uint32_t M, uint32_t K) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!W.data || !x.data || !pv || !pi || !out.data)
        return fail(ER_ERR_INVALID_ARGUMENT, "Q6_K top-1: null buffer");
    if (!aligned(W.data, 16) || !aligned(x.data, 16) || !aligned(pv, 4) || !aligned(pi, 4) ||
        !aligned(out.data, 4))
        return fail(ER_ERR_INVALID_ARGUMENT,
                    "Q6_K top-1: weight and input must be 16-byte, partial and index buffers 4-byte aligned");
    const uint32_t lds = xl_lds_bytes(K);
    // rows the integer-dot kernels do not take run the fp32 family, as the
    // plain GEMV over the same matrix does
    const bool fp32 = K > kI8MaxK || lds + 1024u > ctx->info.lds_per_workgroup || ctx->gemv_fp32 != 0;
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    uint32_t count = 0;
    CuPlan cp;
    CukPlan kp;
    if (M > 0 && fp32) {
        const bool xg = (uint64_t)K * 4u > kLdsXLimit;
        const uint32_t lpr = lanes_per_row((K / 256u) * 4u);
        const KernelId k = (KernelId)(K_GEMV_Q6K_TOP1_L64_S + lpr_index(lpr) + (xg ? 5 : 0));
        const uint32_t rowsPerBlock = ER_GEMV_WAVES * (64u / lpr) * kQ6KRows;  // >= 8: at most M/4 partials
        count = (M + rowsPerBlock - 1u) / rowsPerBlock;
        void *args[] = {&W.data, &x.data, &pv, &pi, &M, &K};
        st = launch(ctx, k, dim3(count, 1, 1), dim3(kGemvThreads, 1, 1), xg ? 0u : K * 4u, stream, args);
        if (st != ER_OK) return st;
    } else if (M > 0 && plan_cuk(ctx, Fmt::Q6_K, M, K, 1u, kp)) {
        // the K-sliced kernel's top-1 form (2 rows per step: an even step
        // count, so quads stay in one workgroup); one partial per workgroup
        // of >= 4 rows, so at most M/4
        const int j = kp.pi == 0 ? (kp.j + 1) & ~1 : kp.j;
        const uint32_t rowsPerWg = (2u << kp.pi) * (uint32_t)j;
        count = (M + rowsPerWg - 1u) / rowsPerWg;
        void *args[] = {&W.data, &x.data, &pv, &pi, &M, &K};
        st = launch_fn(ctx->fnQ6KTop1Cuk[kp.pi][j - 1], "er_gemv_q6k_top1_cuk", dim3(count, 1, 1),
                       dim3(64u * ER_CU_WAVES, 1, 1), xl_lds_bytes(K), stream, args);
        if (st != ER_OK) return st;
    } else if (M > 0 && plan_cu(ctx, Fmt::Q6_K, M, K, 1u, cp)) {
        // one partial per workgroup (rowsPerWg >= 8, so at most M/4); the
        // row values of a workgroup reuse its x area of LDS
        count = (M + cp.rowsPerWg - 1u) / cp.rowsPerWg;
        const uint32_t ldsTop1 = std::max<uint32_t>(cu_lds_bytes(K), 4u * cp.rowsPerWg);
        void *args[] = {&W.data, &x.data, &pv, &pi, &M, &K, (void *)&cp.rowsPerWg};
        st = launch_fn(ctx->fnQ6KTop1Cu[cp.ci][cp.slot], "er_gemv_q6k_top1_cu", dim3(count, 1, 1),
                       dim3(64u * ER_CU_WAVES, 1, 1), ldsTop1, stream, args);
        if (st != ER_OK) return st;
    } else if (M > 0) {
        int ci = pick_i8(K / 64u, M, ctx->cu_count, 1u);
        if (ctx->i8_override >= 0 && (uint32_t)kI8Cfg[ctx->i8_override].lpr *
                                             kI8Cfg[ctx->i8_override].ns >= K / 64u)
            ci = ctx->i8_override;
        if (ci < 0) return fail(ER_ERR_INVALID_VECTOR_SHAPE, "Q6_K top-1: no configuration for K=%u", K);
        const I8Cfg &c = kI8Cfg[ci];
        const uint32_t rowsPerBlock = ER_GEMV_WAVES * (64u / c.lpr) * c.r;
        count = (M + rowsPerBlock - 1) / rowsPerBlock;
        void *args[] = {&W.data, &x.data, &pv, &pi, &M, &K};
        st = launch_fn(ctx->fnQ6KTop1[ci], "er_gemv_q6k_top1", dim3(count, 1, 1), dim3(kGemvThreads, 1, 1),
                       lds, stream, args);
        if (st != ER_OK) return st;
    }
    void *rargs[] = {&pv, &pi, &out.data, &count};
    return launch(ctx, K_TOP1_REDUCE, dim3(1, 1, 1), dim3(256, 1, 1), 0, stream, rargs);
}

er_status encode_q6k_top1(er_hip_ctx *ctx, er_stream stream, er_buffer W, er_buffer x,
                          er_buffer pv, er_buffer pi, er_buffer out, uint32_t M, uint32_t K) {
    er_status st = validate_q6k_top1(W, x, out, M, K);
    if (st != ER_OK) return st;
    const uint64_t partials = M / 4u;
    if (pv.length < partials * 4u || pi.length < partials * 4u)
        return fail(ER_ERR_ENCODING_FAILED,
                    "Q6_K top-1: partial buffers %llu / %llu B too small for M=%u",
                    (unsigned long long)pv.length, (unsigned long long)pi.length, M);
    return launch_q6k_top1(ctx, stream, W, x, pv.data, pi.data, out, M, K);
}

// The same top-1 with its partials in this context's scratch array: no
// caller buffers, no allocation.  Heads of more than
// ER_HIP_TOP1_NOALLOC_MAX_ROWS rows exceed the array (INVALID_MATRIX_SHAPE,
// checked before anything touches the device).
er_status encode_q6k_top1_noalloc(er_hip_ctx *ctx, er_stream stream, er_buffer W, er_buffer x, er_buffer out,
                                  uint32_t M, uint32_t K) {
    er_status st = validate_q6k_top1(W, x, out, M, K);
    if (st != ER_OK) return st;
    if (M > ER_HIP_TOP1_NOALLOC_MAX_ROWS)
        return fail(ER_ERR_INVALID_MATRIX_SHAPE,
                    "Q6_K top-1 without caller scratch: M=%u exceeds the %u rows its scratch array serves", M,
                    (unsigned)ER_HIP_TOP1_NOALLOC_MAX_ROWS);
    st = check_ctx(ctx);
    if (st != ER_OK) return st;
    uint8_t *base = (uint8_t *)ctx->scratch;
    return launch_q6k_top1(ctx, stream, W, x, base, base + 4u * ER_SCRATCH_TOP1_PARTIALS, out, M, K);
}

// Q8_0 row quantizer (quantize_q8_0_rows, Dequant_Q8_0.metal:19-49, encoded
// by LlamaLanguageModel.encodeQ8Rows, LlamaLanguageModel.swift:1820-1850).
// The reference dispatches it without checks; here the source and destination
// extents the parameters imply must fit the buffers (ENCODING_FAILED), so no
// launch can touch memory outside them.
er_status encode_quantize_q8_0(er_hip_ctx *ctx, er_stream stream, er_buffer src, er_buffer dst,
                               uint32_t rowCount, uint32_t srcStride, uint32_t dstRowBase,
                               uint32_t blocksPerRow) {
    if (rowCount == 0 || blocksPerRow == 0) return check_ctx(ctx);
    const uint64_t srcNeed = ((uint64_t)(rowCount - 1u) * srcStride + (uint64_t)blocksPerRow * 32u) * 4u;
    const uint64_t dstNeed = ((uint64_t)dstRowBase + rowCount) * blocksPerRow * 34u;
    if (src.length < srcNeed || dst.length < dstNeed)
        return fail(ER_ERR_ENCODING_FAILED,
                    "quantize_q8_0_rows: source %llu B (needs %llu) / destination %llu B (needs %llu)",
                    (unsigned long long)src.length, (unsigned long long)srcNeed,
                    (unsigned long long)dst.length, (unsigned long long)dstNeed);
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!src.data || !dst.data) return fail(ER_ERR_INVALID_ARGUMENT, "quantize_q8_0_rows: null buffer");
    if (!aligned(src.data, 4) || !aligned(dst.data, 2))
        return fail(ER_ERR_INVALID_ARGUMENT,
                    "quantize_q8_0_rows: source must be 4-byte and destination 2-byte aligned");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    const bool vec = aligned(src.data, 16) && srcStride % 4u == 0;
    const uint64_t blocks = (uint64_t)rowCount * blocksPerRow;
    if (blocks >= (1ull << 32))
        return fail(ER_ERR_ENCODING_FAILED, "quantize_q8_0_rows: %llu blocks exceed 2^32 - 1",
                    (unsigned long long)blocks);
    const uint64_t wgs = std::min<uint64_t>((blocks + 31u) / 32u, 8192u);  // 32 blocks per pass
    void *args[] = {&src.data, &dst.data, &rowCount, &srcStride, &dstRowBase, &blocksPerRow};
    return launch(ctx, vec ? K_QUANT_Q8_0_V : K_QUANT_Q8_0_S, dim3((uint32_t)wgs, 1, 1), dim3(256, 1, 1), 0,
                  stream, args);
}

// Loader-specialised kernel: 256 (or 128) weight rows x 128 tokens per
// workgroup, no K split, so it runs where those tiles alone give (nearly)
// every CU a workgroup (256-row tiles), or at least half of them (128-row
// tiles).  r = 0: another kernel takes the shape.
struct GemmLPlan {
    int r = 0;           // 32-row blocks per compute wave (tile of 128 r rows)
    uint64_t tiles = 0;  // work items = workgroups doing work
};
GemmLPlan plan_gemml(const er_hip_ctx *ctx, uint32_t T, uint32_t N, uint32_t K) {
    GemmLPlan p;
    const uint64_t nT = (T + 127u) / 128u;
    const uint64_t tiles2 = nT * ((N + 255u) / 256u), tiles1 = nT * ((N + 127u) / 128u);
    const uint64_t cu = (uint64_t)ctx->cu_count;
    const bool fits = K % 256u == 0 && (uint64_t)T * N * 4u < (1ull << 32) && tiles1 <= 8ull * 65535u;
    // ER_HIP_GEMM_TILE forces the tile / split-K kernels: the loader kernel
    // then takes no shape (unless ER_HIP_GEMM_VARIANT names it)
    const bool tileForced = ctx->gemm_tt != 0 || ctx->gemm_sk != 0;
    if (fits && ctx->gemm_variant == 0 && !tileForced)
        p.r = 4u * tiles2 >= 3u * cu ? 2 : 2u * tiles1 >= cu ? 1 : 0;
    if (fits && ctx->gemm_variant == 4) p.r = 2;
    if (fits && ctx->gemm_variant == 5) p.r = 1;
    p.tiles = p.r == 2 ? tiles2 : p.r == 1 ? tiles1 : 0;
    return p;
}

// stamps: null, or (measurement build) 32 bytes per work item for the
// clock-stamped copy of the kernel
er_status launch_gemml(er_hip_ctx *ctx, er_stream stream, Fmt f, er_buffer W, er_buffer x, er_buffer y, uint32_t T,
                       uint32_t N, uint32_t K, const GemmLPlan &p, uint64_t *stamps) {
    void *args[] = {&W.data, &x.data, &y.data, &T, &N, &K, &stamps};
    // GemmL<Q4K, R>::LDS: 4 X stages of 18432 bytes + the weight stages
    // (+ 4 Q4_K header slots of 16 bytes per row)
    const uint32_t tn = p.r == 2 ? 256u : 128u;
    const uint32_t wst = tn * (f == Fmt::Q4_K ? 32u : 80u);
    const uint32_t nw = p.r == 2 ? (f == Fmt::Q4_K ? 6u : 4u) : (f == Fmt::Q4_K ? 8u : 6u);
    const uint32_t lds = 4u * 18432u + nw * wst + (f == Fmt::Q4_K ? 4u * tn * 16u : 0u);
    if (lds > ctx->info.lds_per_workgroup)
        return fail(ER_ERR_ENCODING_FAILED, "GEMM: %u B of LDS per workgroup needed, %u available", lds,
                    (unsigned)ctx->info.lds_per_workgroup);
    KernelId k = f == Fmt::Q4_K ? (p.r == 2 ? K_GEMML_Q4K : K_GEMML_Q4K_R1)
                                : (p.r == 2 ? K_GEMML_Q8_0 : K_GEMML_Q8_0_R1);
#ifdef ER_WITH_PROBES
    if (stamps)
        k = f == Fmt::Q4_K ? (p.r == 2 ? K_GEMML_Q4K_STAMPED : K_GEMML_Q4K_R1_STAMPED)
                           : (p.r == 2 ? K_GEMML_Q8_0_STAMPED : K_GEMML_Q8_0_R1_STAMPED);
#endif
    return launch(ctx, k, dim3((uint32_t)(8u * ((p.tiles + 7u) / 8u)), 1, 1), dim3(512, 1, 1), lds, stream, args);
}

// Prefill GEMM: validation mirrors the GEMV rules (K multiple of the block,
// buffer lengths), then the loader-specialised kernel where it takes the
// shape, else a grid of ceil(N/128) x ceil(T/TT) workgroups of the others.
// stamps (the clock probe only): the loader-specialised kernel must take the
// shape, and stamps receives its per-work-item clock stamps
er_status encode_gemm(er_hip_ctx *ctx, er_stream stream, Fmt f, er_buffer W, er_buffer x,
                      er_buffer y, uint32_t T, uint32_t N, uint32_t K, const er_buffer *stamps = nullptr,
                      uint32_t *stampItems = nullptr) {
    const uint32_t kmul = f == Fmt::Q4_K ? 256u : 64u;
    if (K == 0 || K % kmul != 0)
        return fail(ER_ERR_INVALID_VECTOR_SHAPE, "%s GEMM: K=%u must be a positive multiple of %u",
                    fmt_name(f), K, kmul);
    const uint64_t need = (uint64_t)N * (K / block_weights(f)) * block_bytes(f);
    if (W.length < need)
        return fail(ER_ERR_INVALID_MATRIX_SHAPE, "%s GEMM: weight buffer holds %llu bytes, N=%u K=%u needs %llu",
                    fmt_name(f), (unsigned long long)W.length, N, K, (unsigned long long)need);
    if (T == 0) return fail(ER_ERR_ENCODING_FAILED, "%s GEMM: tokens must be > 0", fmt_name(f));
    if (x.length < (uint64_t)T * K * 2u || y.length < (uint64_t)T * N * 4u)
        return fail(ER_ERR_ENCODING_FAILED, "%s GEMM: x %llu B / y %llu B too small for T=%u N=%u K=%u",
                    fmt_name(f), (unsigned long long)x.length, (unsigned long long)y.length, T, N, K);
    er_status st = check_ctx(ctx);
    if (st != ER_OK || N == 0) return st;
    if (!W.data || !x.data || !y.data) return fail(ER_ERR_INVALID_ARGUMENT, "GEMM: null buffer");
    if (!aligned(W.data, 16) || !aligned(x.data, 16) || !aligned(y.data, 4))
        return fail(ER_ERR_INVALID_ARGUMENT, "GEMM: weight and x must be 16-byte, y 4-byte aligned");
    if ((T + 127u) / 128u > 65535u)
        return fail(ER_ERR_ENCODING_FAILED, "GEMM: %u tokens exceed the grid limit", T);
    // the pipelined kernels address W and X with 32-bit byte offsets
    if (need >= (1ull << 32) || (uint64_t)T * K * 2u >= (1ull << 32))
        return fail(ER_ERR_INVALID_MATRIX_SHAPE, "%s GEMM: W (%llu B) and X (%llu B) must each be under 4 GiB",
                    fmt_name(f), (unsigned long long)need, (unsigned long long)T * K * 2u);
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    const GemmLPlan lp = plan_gemml(ctx, T, N, K);
    if (stamps) {
        if (!lp.r)
            return fail(ER_ERR_INVALID_ARGUMENT, "GEMM clock probe: the loader-specialised kernel does not take "
                        "T=%u N=%u K=%u", T, N, K);
        if (!stamps->data || !aligned(stamps->data, 8) || stamps->length < 32u * lp.tiles)
            return fail(ER_ERR_INVALID_ARGUMENT, "GEMM clock probe: stamps need %llu bytes (8-byte aligned), %llu given",
                        (unsigned long long)(32u * lp.tiles), (unsigned long long)stamps->length);
        if (stampItems) *stampItems = (uint32_t)lp.tiles;
    }
    if (lp.r) return launch_gemml(ctx, stream, f, W, x, y, T, N, K, lp, stamps ? (uint64_t *)stamps->data : nullptr);
    // Tile height TT (tokens) and K split SK: 128-token tiles (64 for short
    // inputs), then split K until the grid gives every CU a workgroup
    // (measured on MI355X: 512x14336x4096 is fastest unsplit, 512x4096x4096
    // with two K splits).
    void *args1[] = {&W.data, &x.data, &y.data, &T, &N, &K};
    const uint32_t nN = (N + 127u) / 128u;
    uint32_t TT = T >= 128u ? 128u : 64u, SK = 1u;
    const uint32_t NC = K / 64u;
    while (SK < 8u && 2u * SK <= NC && (uint64_t)nN * ((T + TT - 1u) / TT) * SK < (uint64_t)ctx->cu_count)
        SK *= 2u;
    if (ctx->gemm_tt) TT = ctx->gemm_tt;
    if (ctx->gemm_sk) SK = std::min<uint32_t>(ctx->gemm_sk, NC);
    const uint32_t lds = 2u * (TT + 128u) * 72u * 2u;
    if (ctx->gemm_variant == 1 || lds > ctx->info.lds_per_workgroup) {
        // single-stage kernel (benchmark comparison, or two LDS stages do not fit)
        const bool big = TT == 256u;
        const uint32_t TT1 = big ? 256u : 128u;
        const KernelId k = f == Fmt::Q4_K ? (big ? K_GEMM_Q4K_T256 : K_GEMM_Q4K_T128)
                                          : (big ? K_GEMM_Q8_0_T256 : K_GEMM_Q8_0_T128);
        dim3 grid((N + 127u) / 128u, (T + TT1 - 1u) / TT1, 1);
        return launch(ctx, k, grid, dim3(256, 1, 1), 0, stream, args1);
    }
    if (SK > 1u) {
        // split K accumulates with fp32 atomics into a zero-filled Y
        uint64_t n4 = (uint64_t)T * N / 4u, tail = (uint64_t)T * N % 4u;
        if (tail || !aligned(y.data, 16)) SK = 1u;
        else {
            void *zargs[] = {&y.data, &n4};
            const uint64_t blocks = std::min<uint64_t>((n4 + 255u) / 256u, 4096u);
            st = launch(ctx, K_FILL_ZERO, dim3((uint32_t)blocks, 1, 1), dim3(256, 1, 1), 0, stream, zargs);
            if (st != ER_OK) return st;
        }
    }
    KernelId k;
    if (TT == 256u) k = f == Fmt::Q4_K ? K_GEMMP_Q4K_T256 : K_GEMMP_Q8_0_T256;
    else if (TT == 128u) k = f == Fmt::Q4_K ? K_GEMMP_Q4K_T128 : K_GEMMP_Q8_0_T128;
    else k = f == Fmt::Q4_K ? K_GEMMP_Q4K_T64 : K_GEMMP_Q8_0_T64;
    const uint32_t items = nN * ((T + TT - 1u) / TT) * SK;
    void *args[] = {&W.data, &x.data, &y.data, &T, &N, &K, &SK};
    dim3 grid(8u * ((items + 7u) / 8u), 1, 1);
    // warp-specialised kernel (512 threads): 128-token tiles whose every K split
    // has a multiple of 4 chunks
    if (TT == 128u && ctx->gemm_variant != 2 && NC % (4u * SK) == 0u)
        return launch(ctx, f == Fmt::Q4_K ? K_GEMMW_Q4K_T128 : K_GEMMW_Q8_0_T128, grid, dim3(512, 1, 1), lds,
                      stream, args);
    return launch(ctx, k, grid, dim3(256, 1, 1), lds, stream, args);
}

// Whether fused projections of Mt rows (one token's) of K weights run on the
// K-sliced kernels: where each wave's slice of K fills at least 7/8 of its row
// slice's lanes (K = 4096, 7680, 8192, 14336, 16384 ...), from 12 rows per CU
// at K = 4096 and 8 beyond; or wherever ER_HIP_GEMV_CUK=2 lets them; never
// when a multi-matrix configuration is forced.  Depends on the rows and K
// alone, so batched and per-token calls run the same arithmetic.  Same-box,
// one token, us, multi-matrix kernels -> K-sliced: K = 4096: Q4_K 2 x 1024
// rows 3.72 -> 4.08 and Q8_0 gate/up + SiLU 2 x 1024 4.69 -> 4.97 (8 rows per
// CU); Q4_K 2 x 1536 4.48 -> 4.40, 2 x 2048 4.80 -> 4.67, 2 x 2560 6.86 ->
// 5.18, Q8_0 QKV 2048 + 2 x 512 6.80 -> 5.66, 4096 + 2 x 512 9.85 -> 7.23,
// gate/up + SiLU 2 x 2048 6.94 -> 6.28; K = 8192: Q4_K 2 x 1024 4.91 -> 4.88,
// 2 x 2048 8.13 -> 6.31, Q8_0 QKV 2048 + 2 x 512 10.64 -> 7.90; K = 14336:
// Q4_K 2 x 1024 9.14 -> 6.95, gate/up + SiLU 2 x 1024 13.05 -> 10.13.  A
// slice filling 10 of 16 lanes (K = 5120) lost: 5120 + 2 x 1024 rows 8.88 ->
// 10.28 (before the row sources held their pointers as values).
// min4096: the rows per CU needed at K = 4096 (20 for the Q4_K GeGLU, whose
// paired multi-matrix kernel held 2 x 1536 and 2 x 2048 rows at 4.32 / 4.38
// against 4.63 / 4.90 us, and lost 2 x 2560 at 6.22 against 5.32).
bool fused_on_cuk(const er_hip_ctx *ctx, uint64_t Mt, uint32_t K, uint32_t min4096 = 12u) {
    if (ctx->multi_override >= 0 || ctx->multi1_override >= 0) return false;
    if (ctx->cuk_mode == 2) return true;
    const uint64_t rowsPerCu = (Mt + (uint64_t)ctx->cu_count - 1u) / (uint64_t)ctx->cu_count;
    const uint32_t S = K / 64u, sliceLanes = S <= 64u ? 8u : (S <= 128u ? 16u : 32u);
    return rowsPerCu >= (S <= 64u ? min4096 : 8u) && 8u * ((S + 7u) / 8u) >= 7u * sliceLanes;
}

// Fused Q4_K projections: validation of each weight as encodeQ4KWeights, then
// one launch over all the matrices' rows -- the K-sliced kernels for large
// totals, else the multi-matrix lane-group kernels (fp32 fallback: one GEMV
// per matrix).
er_status encode_q4k_multi(er_hip_ctx *ctx, er_stream stream, const er_buffer *Ws, er_buffer x,
                           const er_buffer *ys, const uint32_t *Ms, int count, uint32_t K) {
    for (int i = 0; i < count; ++i) {
        er_status st = validate_gemv(Fmt::Q4_K, Ws[i], x, ys[i], 1, Ms[i], K);
        if (st != ER_OK) return st;
    }
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    uint64_t Mt = 0;
    for (int i = 0; i < count; ++i) Mt += Ms[i];
    if (Mt == 0) return ER_OK;
    if (Mt > 0xffffffffull) return fail(ER_ERR_INVALID_MATRIX_SHAPE, "Q4_K multi: too many rows");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    Q4MultiArgs a{};
    for (int i = 0; i < 3; ++i) {
        const int j = i < count ? i : 0;
        a.W[i] = Ws[j].data;
        a.y[i] = ys[j].data;
        a.M[i] = i < count ? Ms[i] : 0u;
    }
    // Large totals (fused_on_cuk), where one matrix of all the rows would take
    // the K-sliced kernels: the matrices run there as one launch over their
    // concatenated rows, each row's value the one a K-sliced call gives it (a
    // function of K alone).  Same-box A/B against the multi-matrix kernels,
    // medians of 4 (us): 2 x 14336 x 4096 19.81 -> 16.09, 4096 + 2 x 1024 rows
    // x 4096 6.98 -> 5.42, 2 x 4096 x 4096 7.47 -> 6.23.
    CukPlan kp;
    if (fused_on_cuk(ctx, Mt, K) && plan_cuk(ctx, Fmt::Q4_K, (uint32_t)Mt, K, 1u, kp)) {
        void *kargs[] = {&a, &x.data, &K};
        dim3 grid((uint32_t)((Mt + kp.rowsPerWg - 1u) / kp.rowsPerWg), 1, 1);
        return launch_fn(ctx->fnQ4KCukMulti[kp.pi][kp.j - 1], "er_gemv_q4k_multi_cuk", grid,
                         dim3(64u * ER_CU_WAVES, 1, 1), xl_lds_bytes(K), stream, kargs);
    }
    const MultiPick mp = K <= kI8MaxK ? pick_multi(ctx, K / 64u, (uint32_t)Mt, true, 1u) : MultiPick{};
    if (mp.ci < 0 && mp.ci1 < 0) {
        for (int i = 0; i < count; ++i) {
            st = encode_gemv(ctx, stream, Fmt::Q4_K, Ws[i], x, ys[i], 1, Ms[i], K);
            if (st != ER_OK) return st;
        }
        return ER_OK;
    }
    const I8Cfg &c = mp.ci >= 0 ? kI8MultiCfg[mp.ci] : kI8Multi1Cfg[mp.ci1];
    const uint32_t rowsPerBlock = ER_GEMV_WAVES * (64u / c.lpr) * c.r;
    const uint32_t lds = xl_lds_bytes(K);
    void *args[] = {&a, &x.data, &K};
    dim3 grid((uint32_t)((Mt + rowsPerBlock - 1) / rowsPerBlock), 1, 1);
    return launch_fn(mp.ci >= 0 ? ctx->fnQ4KMulti[mp.ci] : ctx->fnQ4KMulti1[mp.ci1], "er_gemv_q4k_multi", grid,
                     dim3(kGemvThreads, 1, 1), lds, stream, args);
}

er_status encode_q4k_geglu(er_hip_ctx *ctx, er_stream stream, er_buffer Wg, er_buffer Wu, er_buffer x,
                           er_buffer y, uint32_t M, uint32_t K) {
    er_status st = validate_gemv(Fmt::Q4_K, Wg, x, y, 1, M, K);
    if (st != ER_OK) return st;
    st = validate_gemv(Fmt::Q4_K, Wu, x, y, 1, M, K);
    if (st != ER_OK) return st;
    st = check_ctx(ctx);
    if (st != ER_OK || M == 0) return st;
    const int ci = K <= kI8MaxK && ctx->gemv_fp32 == 0 ? pick_multi(ctx, K / 64u, 2u * M, false, 1u).ci : -1;
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    // large totals: the K-sliced kernels over the 2M gate/up rows, interleaved
    // (fused_on_cuk; at K = 4096 from 20 rows per CU).  Same-box A/B, medians
    // of 4 (us): 2 x 14336 x 4096 18.51 -> 15.38, 2 x 3000 x 4096 6.26 -> 5.58,
    // 2 x 2560 x 4096 6.22 -> 5.32, 2 x 1100 x 14336 12.13 -> 7.55; 2 x 2048 x
    // 4096 4.38 -> 4.90 and 2 x 1536 4.32 -> 4.63 (kept).
    CukPlan kp;
    if (M < 0x80000000u && fused_on_cuk(ctx, 2u * (uint64_t)M, K, 20u) &&
        plan_cuk(ctx, Fmt::Q4_K, 2u * M, K, 1u, kp)) {
        void *kargs[] = {&Wg.data, &Wu.data, &x.data, &y.data, &M, &K};
        dim3 grid((2u * M + kp.rowsPerWg - 1u) / kp.rowsPerWg, 1, 1);
        return launch_fn(ctx->fnQ4KCukGeglu[kp.pi][kp.j - 1], "er_gemv_q4k_geglu_cuk", grid,
                         dim3(64u * ER_CU_WAVES, 1, 1), xl_lds_bytes(K), stream, kargs);
    }
    if (ci < 0) {
        // rows longer than the integer-dot kernels cover: fp32 pair kernel,
        // x from global memory
        const uint32_t rowsPerBlock = ER_GEMV_WAVES * (kQ4KRows / 2u);
        void *args[] = {&Wg.data, &Wu.data, &x.data, &y.data, &M, &K};
        return launch(ctx, K_GEMV_Q4K_GEGLU_L64_G, dim3((M + rowsPerBlock - 1) / rowsPerBlock, 1, 1),
                      dim3(kGemvThreads, 1, 1), 0, stream, args);
    }
    const I8Cfg &c = kI8MultiCfg[ci];
    const uint32_t rowsPerBlock = ER_GEMV_WAVES * (64u / c.lpr) * (c.r / 2u);
    const uint32_t lds = xl_lds_bytes(K);
    void *args[] = {&Wg.data, &Wu.data, &x.data, &y.data, &M, &K};
    dim3 grid((M + rowsPerBlock - 1) / rowsPerBlock, 1, 1);
    return launch_fn(ctx->fnQ4KGeglu[ci], "er_gemv_q4k_geglu", grid, dim3(kGemvThreads, 1, 1), lds,
                     stream, args);
}

// Fused Q8_0 projections (Dequant_Q8_0.metal:199-586, encoded by name in
// LlamaLanguageModel.swift:260-275).  The reference dispatches them without
// checks; here every buffer must hold what the shapes imply (weights
// INVALID_MATRIX_SHAPE, vectors ENCODING_FAILED).  Any K % 32 == 0 is taken,
// as the reference's kernels take any blocksPerRow: the integer-dot kernels
// run rows of K % 64 == 0 up to 16384 weights, the fp32 kernels
// (gemv_q8_0_any_fused) the rest.
struct Q8FusedSpec {
    const char *name;
    int count;          // matrices (1..3); 2 for gate/up
    er_buffer W[3], y[3], res[3];
    uint32_t M[3];
    uint32_t halfMask;  // bit m: matrix m's output is fp16
    er_buffer normW;    // data == nullptr: no RMSNorm
    float eps;
    bool silu;          // gate/up pairs, output silu(gate) * up
};

er_status encode_q8_fused(er_hip_ctx *ctx, er_stream stream, const Q8FusedSpec &f, er_buffer x,
                          uint32_t tokens, uint32_t K) {
    if (K == 0 || K % 32u != 0)
        return fail(ER_ERR_INVALID_VECTOR_SHAPE, "%s: K=%u must be a positive multiple of 32", f.name, K);
    // odd block counts (rows only 2-byte aligned) and long rows: fp32 kernels
    bool anyK = K % 64u != 0 || K > kI8MaxK;
    if (tokens == 0 || tokens > 65535u)
        return fail(ER_ERR_ENCODING_FAILED, "%s: tokenCount %u outside [1, 65535]", f.name, tokens);
    uint64_t Mt = 0;
    for (int m = 0; m < f.count; ++m) {
        const uint64_t need = (uint64_t)f.M[m] * (K / 32u) * 34u;
        if (f.W[m].length < need)
            return fail(ER_ERR_INVALID_MATRIX_SHAPE, "%s: weight %d holds %llu bytes, %u rows need %llu", f.name, m,
                        (unsigned long long)f.W[m].length, f.M[m], (unsigned long long)need);
        const uint64_t outNeed = (uint64_t)tokens * f.M[m] * ((f.halfMask >> m) & 1u ? 2u : 4u);
        if (!f.silu || m == 0) {
            if (f.y[m].length < outNeed)
                return fail(ER_ERR_ENCODING_FAILED, "%s: output %d holds %llu bytes, needs %llu", f.name, m,
                            (unsigned long long)f.y[m].length, (unsigned long long)outNeed);
        }
        if (f.res[m].data && f.res[m].length < (uint64_t)tokens * f.M[m] * 4u)
            return fail(ER_ERR_ENCODING_FAILED, "%s: residual holds %llu bytes, needs %llu", f.name,
                        (unsigned long long)f.res[m].length, (unsigned long long)tokens * f.M[m] * 4u);
        Mt += f.M[m];
    }
    if (x.length < (uint64_t)tokens * K * 4u)
        return fail(ER_ERR_ENCODING_FAILED, "%s: input holds %llu bytes, needs %llu", f.name,
                    (unsigned long long)x.length, (unsigned long long)tokens * K * 4u);
    if (f.normW.data && f.normW.length < (uint64_t)K * 4u)
        return fail(ER_ERR_ENCODING_FAILED, "%s: norm weight holds %llu bytes, needs %llu", f.name,
                    (unsigned long long)f.normW.length, (unsigned long long)K * 4u);
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    anyK = anyK || ctx->gemv_fp32 != 0;
    if (f.silu) Mt = f.M[0];
    if (Mt == 0) return ER_OK;
    if (Mt > 0x7fffffffull) return fail(ER_ERR_INVALID_MATRIX_SHAPE, "%s: too many rows", f.name);
    if (!x.data || !aligned(x.data, 16) || (f.normW.data && !aligned(f.normW.data, 16)))
        return fail(ER_ERR_INVALID_ARGUMENT, "%s: input and norm weight must be 16-byte aligned", f.name);
    for (int m = 0; m < f.count; ++m) {
        if (f.M[m] == 0) continue;
        if (!f.W[m].data || !aligned(f.W[m].data, anyK ? 2 : 4) || ((!f.silu || m == 0) && !f.y[m].data) ||
            (f.res[m].data && !aligned(f.res[m].data, 4)))
            return fail(ER_ERR_INVALID_ARGUMENT,
                        "%s: null or misaligned buffer (weights %d-byte, residual 4-byte aligned)", f.name,
                        anyK ? 2 : 4);
        if ((!f.silu || m == 0) && !aligned(f.y[m].data, (f.halfMask >> m) & 1u ? 2 : 4))
            return fail(ER_ERR_INVALID_ARGUMENT, "%s: misaligned output", f.name);
    }
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    const uint32_t S = K / 64u;
    // Large totals: the K-sliced kernels (gate/up pairs as 2M rows), as the
    // Q4_K dual / triple (fused_on_cuk); Q8_0 takes them here at K = 4096 too.
    // Same-box A/B against the multi-matrix kernels, one token, medians of 4
    // (us): QKV 4096 + 2 x 1024 rows x 4096 9.97 -> 7.67, gate/up + SiLU 2 x
    // 14336 x 4096 28.00 -> 24.27.
    CukPlan kp;
    const uint64_t rowsV = f.silu ? 2u * Mt : Mt;
    if (!anyK && fused_on_cuk(ctx, rowsV, K) && plan_cuk(ctx, Fmt::Q8_0, (uint32_t)rowsV, K, tokens, kp, true)) {
        const uint32_t lds = xl_lds_bytes(K);
        dim3 grid((uint32_t)((rowsV + kp.rowsPerWg - 1u) / kp.rowsPerWg), tokens, 1);
        const float *normW = (const float *)f.normW.data;
        float eps = f.eps;
        if (f.silu) {
            uint32_t M = f.M[0];
            void *args[] = {(void *)&f.W[0].data, (void *)&f.W[1].data, &x.data, (void *)&f.y[0].data,
                            &normW, &eps, &M, &K};
            return launch_fn(ctx->fnQ8CukSilu[kp.pi][kp.j - 1], "er_gemv_q8_0_silu_cuk", grid,
                             dim3(64u * ER_CU_WAVES, 1, 1), lds, stream, args);
        }
        Q8MultiArgs a{};
        for (int m = 0; m < 3; ++m) {
            const int j = m < f.count ? m : 0;
            a.W[m] = f.W[j].data;
            a.y[m] = f.y[j].data;
            a.res[m] = m < f.count ? (const float *)f.res[m].data : nullptr;
            a.M[m] = m < f.count ? f.M[m] : 0u;
        }
        a.halfMask = f.halfMask;
        a.normW = normW;
        a.eps = eps;
        void *args[] = {&a, &x.data, &K};
        return launch_fn(ctx->fnQ8CukMulti[kp.pi][kp.j - 1], "er_gemv_q8_0_multi_cuk", grid,
                         dim3(64u * ER_CU_WAVES, 1, 1), lds, stream, args);
    }
    const MultiPick mp = anyK ? MultiPick{} : pick_multi(ctx, S, (uint32_t)(f.silu ? 2u * Mt : Mt), !f.silu, tokens);
    if (mp.ci < 0 && mp.ci1 < 0) {
        Q8MultiArgs a{};
        for (int m = 0; m < 3; ++m) {
            const int j = m < f.count ? m : 0;
            a.W[m] = f.W[j].data;
            a.y[m] = f.y[j].data;
            a.res[m] = m < f.count ? (const float *)f.res[m].data : nullptr;
            a.M[m] = m < f.count ? f.M[m] : 0u;
        }
        a.halfMask = f.halfMask;
        a.normW = (const float *)f.normW.data;
        a.eps = f.eps;
        // 2 rows (or 2 gate/up pairs) per wave
        const uint32_t rowsPerBlock = ER_GEMV_WAVES * 2u;
        void *args[] = {&a, &x.data, &K};
        dim3 grid((uint32_t)((Mt + rowsPerBlock - 1) / rowsPerBlock), tokens, 1);
        return launch(ctx, f.silu ? K_GEMV_Q8_0_ANY_SILU : K_GEMV_Q8_0_ANY_MULTI, grid, dim3(kGemvThreads, 1, 1), 0,
                      stream, args);
    }
    const int ci = mp.ci;  // the paired gate/up + SiLU kernel has no one-row form (r1Ok false above)
    const I8Cfg &c = ci >= 0 ? kI8MultiCfg[ci] : kI8Multi1Cfg[mp.ci1];
    const uint32_t lds = xl_lds_bytes(K);
    const float *normW = (const float *)f.normW.data;
    float eps = f.eps;
    if (f.silu) {
        const uint32_t rowsPerBlock = ER_GEMV_WAVES * (64u / c.lpr) * (c.r / 2u);
        uint32_t M = f.M[0];
        void *args[] = {(void *)&f.W[0].data, (void *)&f.W[1].data, &x.data, (void *)&f.y[0].data,
                        &normW, &eps, &M, &K};
        dim3 grid((M + rowsPerBlock - 1) / rowsPerBlock, tokens, 1);
        return launch_fn(ctx->fnQ8Silu[ci], "er_gemv_q8_0_silu", grid, dim3(kGemvThreads, 1, 1), lds, stream,
                         args);
    }
    Q8MultiArgs a{};
    for (int m = 0; m < 3; ++m) {
        const int j = m < f.count ? m : 0;
        a.W[m] = f.W[j].data;
        a.y[m] = f.y[j].data;
        a.res[m] = m < f.count ? (const float *)f.res[m].data : nullptr;
        a.M[m] = m < f.count ? f.M[m] : 0u;
    }
    a.halfMask = f.halfMask;
    a.normW = normW;
    a.eps = eps;
    const uint32_t rowsPerBlock = ER_GEMV_WAVES * (64u / c.lpr) * c.r;
    void *args[] = {&a, &x.data, &K};
    dim3 grid((uint32_t)((Mt + rowsPerBlock - 1) / rowsPerBlock), tokens, 1);
    return launch_fn(ci >= 0 ? ctx->fnQ8Multi[ci] : ctx->fnQ8Multi1[mp.ci1], "er_gemv_q8_0_multi", grid,
                     dim3(kGemvThreads, 1, 1), lds, stream, args);
}

er_status encode_dequant(er_hip_ctx *ctx, er_stream stream, Fmt f, er_buffer blocks,
                         uint64_t count, er_buffer out) {
    const uint64_t need = count * block_bytes(f);
    if (blocks.length < need)
        return fail(ER_ERR_INVALID_BLOCK_DATA_COUNT,
                    "%s dequant: expected %llu block bytes, buffer holds %llu", fmt_name(f),
                    (unsigned long long)need, (unsigned long long)blocks.length);
    const uint64_t outBytes = count * block_weights(f) * 4u;
    if (out.length < outBytes)
        return fail(ER_ERR_ALLOCATION_FAILED, "%s dequant: output needs %llu bytes, has %llu",
                    fmt_name(f), (unsigned long long)outBytes, (unsigned long long)out.length);
    er_status st = check_ctx(ctx);
    if (st != ER_OK || count == 0) return st;
    if (!blocks.data || !out.data) return fail(ER_ERR_INVALID_ARGUMENT, "dequant: null buffer");
    if (!aligned(blocks.data, f == Fmt::Q4_K ? 16 : 4) || !aligned(out.data, 16))
        return fail(ER_ERR_INVALID_ARGUMENT,
                    "dequant: blocks must be %d-byte and output 16-byte aligned",
                    f == Fmt::Q4_K ? 16 : 4);
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    const uint64_t perBlock = f == Fmt::Q8_0 ? 8u : (f == Fmt::Q4_K ? 32u : 16u);
    const uint64_t threads = count * perBlock;
    const uint64_t maxBlocks = (uint64_t)ctx->cu_count * 64u;
    uint64_t nb = (threads + 255u) / 256u;
    if (nb > maxBlocks) nb = maxBlocks;
    KernelId k = f == Fmt::Q8_0 ? K_DEQUANT_Q8_0 : (f == Fmt::Q4_K ? K_DEQUANT_Q4_K : K_DEQUANT_Q6_K);
    void *args[] = {&blocks.data, &out.data, &count};
    return launch(ctx, k, dim3((uint32_t)nb, 1, 1), dim3(256, 1, 1), 0, stream, args);
}

}  // namespace

extern "C" {

int er_hip_abi_version(void) { return ER_HIP_ABI_VERSION; }

const char *er_hip_last_error(void) { return er_detail::g_last_error; }

const char *er_status_string(er_status s) {
    switch (s) {
        case ER_OK: return "ok";
        case ER_ERR_LIBRARY_NOT_FOUND: return "libraryNotFound";
        case ER_ERR_FUNCTION_NOT_FOUND: return "functionNotFound";
        case ER_ERR_ENCODING_FAILED: return "encodingFailed";
        case ER_ERR_INVALID_MATRIX_SHAPE: return "invalidMatrixShape";
        case ER_ERR_INVALID_VECTOR_SHAPE: return "invalidVectorShape";
        case ER_ERR_INVALID_BLOCK_DATA_COUNT: return "invalidBlockDataCount";
        case ER_ERR_ALLOCATION_FAILED: return "allocationFailed";
        case ER_ERR_INVALID_ARGUMENT: return "invalidArgument";
        case ER_ERR_DEVICE: return "deviceError";
        case ER_ERR_FILE_NOT_FOUND: return "fileNotFound";
        case ER_ERR_INVALID_FORMAT: return "invalidFormat";
        case ER_ERR_UNSUPPORTED_VERSION: return "unsupportedVersion";
        case ER_ERR_UNSUPPORTED_DATA_TYPE: return "unsupportedDataType";
        case ER_ERR_MMAP_FAILED: return "mmapFailed";
        case ER_ERR_MISSING_METADATA: return "missingMetadata";
        case ER_ERR_TENSOR_NOT_FOUND: return "tensorNotFound";
    }
    return "unknown";
}

er_status er_hip_create(int device, er_hip_ctx **out_ctx) {
    if (!out_ctx) return fail(ER_ERR_INVALID_ARGUMENT, "null out_ctx");
    *out_ctx = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return fail(ER_ERR_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    if (device < 0 || device >= count)
        return fail(ER_ERR_INVALID_ARGUMENT, "device %d out of range (%d devices)", device, count);
    e = hipSetDevice(device);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipSetDevice: %s", hipGetErrorString(e));
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess)
        return fail(ER_ERR_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(ER_ERR_LIBRARY_NOT_FOUND, "device %d is %s; this library carries gfx950 code only",
                    device, prop.gcnArchName);
    er_hip_ctx *ctx = new (std::nothrow) er_hip_ctx();
    if (!ctx) return fail(ER_ERR_ALLOCATION_FAILED, "context allocation");
    ctx->device = device;
    ctx->cu_count = prop.multiProcessorCount;
    e = hipModuleLoadData(&ctx->module, er_kernels_blob);
    if (e != hipSuccess) {
        delete ctx;
        return fail(ER_ERR_LIBRARY_NOT_FOUND, "hipModuleLoadData(gfx950 code object, %zu bytes): %s",
                    (size_t)(er_kernels_blob_end - er_kernels_blob), hipGetErrorString(e));
    }
    {
        // this device's copy of the scratch array, found once with the device current
        hipDeviceptr_t sp = nullptr;
        size_t sb = 0;
        e = hipModuleGetGlobal(&sp, &sb, ctx->module, "er_scratch");
        if (e != hipSuccess || sp == nullptr || sb < ER_SCRATCH_BYTES) {
            (void)hipModuleUnload(ctx->module);
            delete ctx;
            return fail(ER_ERR_FUNCTION_NOT_FOUND, "hipModuleGetGlobal(er_scratch): %s (%zu bytes)",
                        hipGetErrorString(e), sb);
        }
        ctx->scratch = (void *)sp;
    }
    for (int i = 0; i < K_COUNT; ++i) {
        e = hipModuleGetFunction(&ctx->fn[i], ctx->module, kKernelNames[i]);
        if (e != hipSuccess) {
            (void)hipModuleUnload(ctx->module);
            delete ctx;
            return fail(ER_ERR_FUNCTION_NOT_FOUND, "functionNotFound(%s): %s", kKernelNames[i],
                        hipGetErrorString(e));
        }
    }
    for (int i = 0; i < kI8Count; ++i) {
        char name[64];
        static const char *const kinds[4] = {"q4k_i8", "q8_0_i8", "q6k_i8", "q6k_top1"};
        hipFunction_t *const slots[4] = {&ctx->fnQ4KI8[i], &ctx->fnQ8I8[i], &ctx->fnQ6KI8[i],
                                         &ctx->fnQ6KTop1[i]};
        for (int fmt = 0; fmt < 4; ++fmt) {
            std::snprintf(name, sizeof(name), "er_gemv_%s_l%u_n%u_r%u", kinds[fmt],
                          (unsigned)kI8Cfg[i].lpr, (unsigned)kI8Cfg[i].ns, (unsigned)kI8Cfg[i].r);
            hipFunction_t *slot = slots[fmt];
            e = hipModuleGetFunction(slot, ctx->module, name);
            if (e != hipSuccess) {
                (void)hipModuleUnload(ctx->module);
                delete ctx;
                return fail(ER_ERR_FUNCTION_NOT_FOUND, "functionNotFound(%s): %s", name,
                            hipGetErrorString(e));
            }
        }
    }
    for (int kind = 0; kind < 4; ++kind) {
        // q4k, q8_0, q6k and the q6k top-1 kernels
        static const char *const names[4] = {"q4k_cu", "q8_0_cu", "q6k_cu", "q6k_top1_cu"};
        const CuCfg *cfg = kind == 0 ? kCuCfgQ4K : (kind == 1 ? kCuCfgQ8 : kCuCfgQ6K);
        const int count = kind == 0 ? kCuCountQ4K : (kind == 1 ? kCuCountQ8 : kCuCountQ6K);
        for (int i = 0; i < count; ++i)
            for (int jc = 1; jc <= ER_CU_MAX_STEPS + 1; ++jc) {
                // kernels exist for steps 1..maxJ, and the rolled one (slot
                // ER_CU_MAX_STEPS) when maxJ == ER_CU_MAX_STEPS
                if (jc <= ER_CU_MAX_STEPS ? jc > cfg[i].maxJ : cfg[i].maxJ != ER_CU_MAX_STEPS) continue;
                char name[64], tag[8];
                if (jc <= ER_CU_MAX_STEPS)
                    std::snprintf(tag, sizeof(tag), "%d", jc);
                else
                    std::snprintf(tag, sizeof(tag), "r");
                std::snprintf(name, sizeof(name), "er_gemv_%s_l%u_n%u_j%s", names[kind], (unsigned)cfg[i].lpr,
                              (unsigned)cfg[i].ns, tag);
                hipFunction_t *slot = kind == 0   ? &ctx->fnQ4KCu[i][jc - 1]
                                      : kind == 1 ? &ctx->fnQ8Cu[i][jc - 1]
                                      : kind == 2 ? &ctx->fnQ6KCu[i][jc - 1]
                                                  : &ctx->fnQ6KTop1Cu[i][jc - 1];
                e = hipModuleGetFunction(slot, ctx->module, name);
                if (e != hipSuccess) {
                    (void)hipModuleUnload(ctx->module);
                    delete ctx;
                    return fail(ER_ERR_FUNCTION_NOT_FOUND, "functionNotFound(%s): %s", name,
                                hipGetErrorString(e));
                }
            }
    }
    for (int pi = 0; pi < 3; ++pi)
        for (int j = 1; j <= ER_CUK_MAX_STEPS; ++j)
            for (int kind = 0; kind < 8; ++kind) {
                // q4k, q8_0, the Q4_K dual / triple and dual GeGLU, the fused
                // Q8_0 rows and gate/up + SiLU (2, 4, 8 rows per step); q6k
                // and its top-1 (2, 4; the top-1 with 2 rows per step at even
                // step counts)
                if ((kind == 2 || kind == 3) && (pi == 2 || (kind == 3 && pi == 0 && j % 2 != 0))) continue;
                static const char *const kinds[8] = {"q4k",       "q8_0",       "q6k",       "q6k_top1",
                                                     "q4k_multi", "q8_0_multi", "q8_0_silu", "q4k_geglu"};
                hipFunction_t *const slot = kind == 0   ? &ctx->fnQ4KCuk[pi][j - 1]
                                            : kind == 1 ? &ctx->fnQ8Cuk[pi][j - 1]
                                            : kind == 2 ? &ctx->fnQ6KCuk[pi][j - 1]
                                            : kind == 3 ? &ctx->fnQ6KTop1Cuk[pi][j - 1]
                                            : kind == 4 ? &ctx->fnQ4KCukMulti[pi][j - 1]
                                            : kind == 5 ? &ctx->fnQ8CukMulti[pi][j - 1]
                                            : kind == 6 ? &ctx->fnQ8CukSilu[pi][j - 1]
                                                        : &ctx->fnQ4KCukGeglu[pi][j - 1];
                char name[64];
                std::snprintf(name, sizeof(name), "er_gemv_%s_cuk%d_j%d", kinds[kind], 2 << pi, j);
                e = hipModuleGetFunction(slot, ctx->module, name);
                if (e != hipSuccess) {
                    (void)hipModuleUnload(ctx->module);
                    delete ctx;
                    return fail(ER_ERR_FUNCTION_NOT_FOUND, "functionNotFound(%s): %s", name, hipGetErrorString(e));
                }
            }
    for (int i = 0; i < kI8MultiCount; ++i) {
        char name[64];
        static const char *const kinds[4] = {"q4k_multi", "q4k_geglu", "q8_0_multi", "q8_0_silu"};
        hipFunction_t *const slots[4] = {&ctx->fnQ4KMulti[i], &ctx->fnQ4KGeglu[i], &ctx->fnQ8Multi[i],
                                         &ctx->fnQ8Silu[i]};
        for (int kind = 0; kind < 4; ++kind) {
            std::snprintf(name, sizeof(name), "er_gemv_%s_l%u_n%u_r%u", kinds[kind],
                          (unsigned)kI8MultiCfg[i].lpr, (unsigned)kI8MultiCfg[i].ns,
                          (unsigned)kI8MultiCfg[i].r);
            e = hipModuleGetFunction(slots[kind], ctx->module, name);
            if (e != hipSuccess) {
                (void)hipModuleUnload(ctx->module);
                delete ctx;
                return fail(ER_ERR_FUNCTION_NOT_FOUND, "functionNotFound(%s): %s", name,
                            hipGetErrorString(e));
            }
        }
    }
    for (int i = 0; i < kI8Multi1Count; ++i) {
        char name[64];
        static const char *const kinds[2] = {"q4k_multi", "q8_0_multi"};
        hipFunction_t *const slots[2] = {&ctx->fnQ4KMulti1[i], &ctx->fnQ8Multi1[i]};
        for (int kind = 0; kind < 2; ++kind) {
            std::snprintf(name, sizeof(name), "er_gemv_%s_l%u_n%u_r%u", kinds[kind], (unsigned)kI8Multi1Cfg[i].lpr,
                          (unsigned)kI8Multi1Cfg[i].ns, (unsigned)kI8Multi1Cfg[i].r);
            e = hipModuleGetFunction(slots[kind], ctx->module, name);
            if (e != hipSuccess) {
                (void)hipModuleUnload(ctx->module);
                delete ctx;
                return fail(ER_ERR_FUNCTION_NOT_FOUND, "functionNotFound(%s): %s", name, hipGetErrorString(e));
            }
        }
    }
    if (const char *gv = std::getenv("ER_HIP_GEMM_VARIANT")) ctx->gemm_variant = std::atoi(gv);
    if (const char *fv = std::getenv("ER_HIP_GEMV_FP32")) ctx->gemv_fp32 = std::atoi(fv);
    if (const char *gt = std::getenv("ER_HIP_GEMM_TILE")) {
        unsigned a = 0, b = 0;
        if (std::sscanf(gt, "%u:%u", &a, &b) == 2 && (a == 64 || a == 128 || a == 256) && b >= 1) {
            ctx->gemm_tt = a;
            ctx->gemm_sk = b;
        }
    }
    if (const char *cv = std::getenv("ER_HIP_GEMV_CU")) ctx->cu_mode = std::atoi(cv) != 0 ? 1 : 0;
    if (const char *kv = std::getenv("ER_HIP_GEMV_CUK")) ctx->cuk_mode = std::atoi(kv);
    if (const char *mv = std::getenv("ER_HIP_GEMV_MULTI_CONFIG")) {
        unsigned l = 0, n = 0, r = 0;
        if (std::sscanf(mv, "%u:%u:%u", &l, &n, &r) == 3)
            for (int i = 0; i < kI8MultiCount; ++i)
                if (kI8MultiCfg[i].lpr == l && kI8MultiCfg[i].ns == n && kI8MultiCfg[i].r == r) ctx->multi_override = i;
        if (std::sscanf(mv, "%u:%u:%u", &l, &n, &r) == 3)
            for (int i = 0; i < kI8Multi1Count; ++i)
                if (kI8Multi1Cfg[i].lpr == l && kI8Multi1Cfg[i].ns == n && kI8Multi1Cfg[i].r == r)
                    ctx->multi1_override = i;
    }
    if (const char *ov = std::getenv("ER_HIP_GEMV_CONFIG")) {
        unsigned l = 0, n = 0, r = 0;
        if (std::sscanf(ov, "%u:%u:%u", &l, &n, &r) == 3)
            for (int i = 0; i < kI8Count; ++i)
                if (kI8Cfg[i].lpr == l && kI8Cfg[i].ns == n && kI8Cfg[i].r == r) ctx->i8_override = i;
    }
    er_device_info &info = ctx->info;
    info.device = device;
    info.compute_units = prop.multiProcessorCount;
    info.clock_khz = prop.clockRate;
    info.memory_clock_khz = prop.memoryClockRate;
    info.memory_bus_width = prop.memoryBusWidth;
    info.total_memory = prop.totalGlobalMem;
    info.lds_per_workgroup = prop.sharedMemPerBlock;
    std::snprintf(info.name, sizeof(info.name), "%.63s", prop.name);
    std::snprintf(info.arch, sizeof(info.arch), "%.63s", prop.gcnArchName);
    *out_ctx = ctx;
    return ER_OK;
}

void er_hip_destroy(er_hip_ctx *ctx) {
    if (!ctx) return;
    if (bind_device(ctx) == ER_OK && ctx->module) (void)hipModuleUnload(ctx->module);
    delete ctx;
}

er_status er_hip_get_device_info(const er_hip_ctx *ctx, er_device_info *out) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!out) return fail(ER_ERR_INVALID_ARGUMENT, "null out");
    *out = ctx->info;
    return ER_OK;
}

er_status er_hip_alloc(er_hip_ctx *ctx, uint64_t bytes, er_buffer *out) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!out) return fail(ER_ERR_INVALID_ARGUMENT, "null out");
    out->data = nullptr;
    out->length = 0;
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess)
        return fail(ER_ERR_ALLOCATION_FAILED, "allocationFailed(byteCount: %llu): %s",
                    (unsigned long long)bytes, hipGetErrorString(e));
    out->data = p;
    out->length = bytes;
    return ER_OK;
}

er_status er_hip_free(er_hip_ctx *ctx, er_buffer buf) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!buf.data) return ER_OK;
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipError_t e = hipFree(buf.data);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipFree: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_upload(er_hip_ctx *ctx, er_stream stream, er_buffer dst, uint64_t dst_offset,
                        const void *src, uint64_t bytes) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (dst_offset > dst.length || bytes > dst.length - dst_offset)
        return fail(ER_ERR_INVALID_ARGUMENT, "upload of %llu bytes at %llu overruns %llu-byte buffer",
                    (unsigned long long)bytes, (unsigned long long)dst_offset,
                    (unsigned long long)dst.length);
    if (bytes == 0) return ER_OK;
    if (!src || !dst.data) return fail(ER_ERR_INVALID_ARGUMENT, "upload: null pointer");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipError_t e = hipMemcpyAsync((char *)dst.data + dst_offset, src, bytes, hipMemcpyHostToDevice,
                                  (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "upload: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_download(er_hip_ctx *ctx, er_stream stream, void *dst, er_buffer src,
                          uint64_t src_offset, uint64_t bytes) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (src_offset > src.length || bytes > src.length - src_offset)
        return fail(ER_ERR_INVALID_ARGUMENT,
                    "download of %llu bytes at %llu overruns %llu-byte buffer",
                    (unsigned long long)bytes, (unsigned long long)src_offset,
                    (unsigned long long)src.length);
    if (bytes == 0) return ER_OK;
    if (!dst || !src.data) return fail(ER_ERR_INVALID_ARGUMENT, "download: null pointer");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipError_t e = hipMemcpyAsync(dst, (const char *)src.data + src_offset, bytes,
                                  hipMemcpyDeviceToHost, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "download: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_copy(er_hip_ctx *ctx, er_stream stream, er_buffer dst, uint64_t dst_offset,
                      er_buffer src, uint64_t src_offset, uint64_t bytes) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (dst_offset > dst.length || bytes > dst.length - dst_offset || src_offset > src.length ||
        bytes > src.length - src_offset)
        return fail(ER_ERR_INVALID_ARGUMENT, "copy of %llu bytes overruns a buffer",
                    (unsigned long long)bytes);
    if (bytes == 0) return ER_OK;
    if (!dst.data || !src.data) return fail(ER_ERR_INVALID_ARGUMENT, "copy: null pointer");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipError_t e = hipMemcpyAsync((char *)dst.data + dst_offset, (const char *)src.data + src_offset,
                                  bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "copy: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_stream_create(er_hip_ctx *ctx, er_stream *out) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!out) return fail(ER_ERR_INVALID_ARGUMENT, "null out");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipStreamCreate: %s", hipGetErrorString(e));
    *out = (er_stream)s;
    return ER_OK;
}

er_status er_hip_stream_destroy(er_hip_ctx *ctx, er_stream stream) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!stream) return ER_OK;
    hipError_t e = hipStreamDestroy((hipStream_t)stream);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipStreamDestroy: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_synchronize(er_hip_ctx *ctx, er_stream stream) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipStreamSynchronize: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_event_create(er_hip_ctx *ctx, er_event *out) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!out) return fail(ER_ERR_INVALID_ARGUMENT, "null out");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipEventCreate: %s", hipGetErrorString(e));
    *out = (er_event)ev;
    return ER_OK;
}

er_status er_hip_event_destroy(er_hip_ctx *ctx, er_event ev) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!ev) return ER_OK;
    hipError_t e = hipEventDestroy((hipEvent_t)ev);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipEventDestroy: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_event_record(er_hip_ctx *ctx, er_event ev, er_stream stream) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!ev) return fail(ER_ERR_INVALID_ARGUMENT, "null event");
    hipError_t e = hipEventRecord((hipEvent_t)ev, (hipStream_t)stream);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipEventRecord: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_event_elapsed_ms(er_hip_ctx *ctx, er_event start, er_event end, float *ms) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!start || !end || !ms) return fail(ER_ERR_INVALID_ARGUMENT, "null event/out");
    hipError_t e = hipEventSynchronize((hipEvent_t)end);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipEventElapsedTime: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_graph_begin(er_hip_ctx *ctx, er_stream stream) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!stream) return fail(ER_ERR_INVALID_ARGUMENT, "graph capture needs a created stream, not the null stream");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipStreamBeginCapture: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_graph_end(er_hip_ctx *ctx, er_stream stream, er_graph *out) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!stream || !out) return fail(ER_ERR_INVALID_ARGUMENT, "null stream/out");
    *out = nullptr;
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipStreamEndCapture: %s", hipGetErrorString(e));
    hipGraphExec_t ge = nullptr;
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipGraphInstantiate: %s", hipGetErrorString(e));
    *out = (er_graph)ge;
    return ER_OK;
}

er_status er_hip_graph_launch(er_hip_ctx *ctx, er_graph graph, er_stream stream) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!graph) return fail(ER_ERR_INVALID_ARGUMENT, "null graph");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    hipError_t e = hipGraphLaunch((hipGraphExec_t)graph, (hipStream_t)stream);
    if (e != hipSuccess) return fail(ER_ERR_ENCODING_FAILED, "hipGraphLaunch: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_graph_destroy(er_hip_ctx *ctx, er_graph graph) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (!graph) return ER_OK;
    hipError_t e = hipGraphExecDestroy((hipGraphExec_t)graph);
    if (e != hipSuccess) return fail(ER_ERR_DEVICE, "hipGraphExecDestroy: %s", hipGetErrorString(e));
    return ER_OK;
}

er_status er_hip_dequant_q8_0(er_hip_ctx *ctx, er_stream stream, er_buffer blocks,
                              uint64_t block_count, er_buffer out) {
    return encode_dequant(ctx, stream, Fmt::Q8_0, blocks, block_count, out);
}

er_status er_hip_dequant_q4_k(er_hip_ctx *ctx, er_stream stream, er_buffer blocks,
                              uint64_t super_block_count, er_buffer out) {
    return encode_dequant(ctx, stream, Fmt::Q4_K, blocks, super_block_count, out);
}

er_status er_hip_dequant_q6_k(er_hip_ctx *ctx, er_stream stream, er_buffer blocks,
                              uint64_t super_block_count, er_buffer out) {
    return encode_dequant(ctx, stream, Fmt::Q6_K, blocks, super_block_count, out);
}

er_status er_hip_encode_q4k_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                    er_buffer input, er_buffer output, uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q4_K, weight, input, output, 1, M, K);
}

er_status er_hip_encode_q6k_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                    er_buffer input, er_buffer output, uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q6_K, weight, input, output, 1, M, K);
}

er_status er_hip_encode_q8_0_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                     er_buffer input, er_buffer output, uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q8_0, weight, input, output, 1, M, K);
}

er_status er_hip_encode_q4k_weights_packed(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                           er_buffer input, er_buffer output, uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q4_K, weight, input, output, 1, M, K);
}

er_status er_hip_encode_q4k_weights_packed_four_rows(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                                     er_buffer input, er_buffer output, uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q4_K, weight, input, output, 1, M, K);
}

er_status er_hip_encode_q4k_weights_llama_style(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                                er_buffer input, er_buffer output, uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q4_K, weight, input, output, 1, M, K);
}

er_status er_hip_encode_q4k_weights_two_rows(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                             er_buffer input, er_buffer output, uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q4_K, weight, input, output, 1, M, K);
}

er_status er_hip_encode_q6k_weights_packed(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                           er_buffer input, er_buffer output, uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q6_K, weight, input, output, 1, M, K);
}

er_status er_hip_encode_q4k_weights_llama_style_dual(er_hip_ctx *ctx, er_stream stream, er_buffer weight_a,
                                                     er_buffer weight_b, er_buffer input, er_buffer output_a,
                                                     er_buffer output_b, uint32_t M, uint32_t K) {
    return er_hip_encode_q4k_weights_dual(ctx, stream, weight_a, weight_b, input, output_a, output_b, M, K);
}

er_status er_hip_encode_q4k_weights_triple_packed(er_hip_ctx *ctx, er_stream stream, er_buffer weight_a,
                                                  er_buffer weight_b, er_buffer weight_c, er_buffer input,
                                                  er_buffer output_a, er_buffer output_b, er_buffer output_c,
                                                  uint32_t rows_a, uint32_t rows_b, uint32_t rows_c, uint32_t K) {
    return er_hip_encode_q4k_weights_triple(ctx, stream, weight_a, weight_b, weight_c, input, output_a, output_b,
                                            output_c, rows_a, rows_b, rows_c, K);
}

er_status er_hip_execute_q4k_weights(er_hip_ctx *ctx, const void *raw_weights, uint64_t raw_bytes, const float *x,
                                     uint64_t x_count, float *y, uint64_t y_count, uint32_t M, uint32_t K) {
    return execute_gemv_host(ctx, Fmt::Q4_K, raw_weights, raw_bytes, x, x_count, y, y_count, 1, false, M, K);
}

er_status er_hip_execute_q6k_weights(er_hip_ctx *ctx, const void *raw_weights, uint64_t raw_bytes, const float *x,
                                     uint64_t x_count, float *y, uint64_t y_count, uint32_t M, uint32_t K) {
    return execute_gemv_host(ctx, Fmt::Q6_K, raw_weights, raw_bytes, x, x_count, y, y_count, 1, false, M, K);
}

er_status er_hip_execute_q4k_weights_with_weight_buffer(er_hip_ctx *ctx, er_buffer weight, const float *x,
                                                        uint64_t x_count, float *y, uint64_t y_count, uint32_t M,
                                                        uint32_t K) {
    return execute_gemv(ctx, Fmt::Q4_K, weight, x, x_count, y, y_count, 1, false, M, K);
}

er_status er_hip_execute_q6k_weights_with_weight_buffer(er_hip_ctx *ctx, er_buffer weight, const float *x,
                                                        uint64_t x_count, float *y, uint64_t y_count, uint32_t M,
                                                        uint32_t K) {
    return execute_gemv(ctx, Fmt::Q6_K, weight, x, x_count, y, y_count, 1, false, M, K);
}

er_status er_hip_execute_batched_q4k_weights(er_hip_ctx *ctx, const void *raw_weights, uint64_t raw_bytes,
                                             const float *x, uint64_t x_count, float *y, uint64_t y_count,
                                             uint32_t batch_seq, uint32_t M, uint32_t K) {
    return execute_gemv_host(ctx, Fmt::Q4_K, raw_weights, raw_bytes, x, x_count, y, y_count, batch_seq, true, M, K);
}

er_status er_hip_encode_q4k_weights_dual(er_hip_ctx *ctx, er_stream stream, er_buffer weight_a,
                                         er_buffer weight_b, er_buffer input, er_buffer output_a,
                                         er_buffer output_b, uint32_t M, uint32_t K) {
    const er_buffer Ws[2] = {weight_a, weight_b}, ys[2] = {output_a, output_b};
    const uint32_t Ms[2] = {M, M};
    return encode_q4k_multi(ctx, stream, Ws, input, ys, Ms, 2, K);
}

er_status er_hip_encode_q4k_weights_triple(er_hip_ctx *ctx, er_stream stream, er_buffer weight_a,
                                           er_buffer weight_b, er_buffer weight_c, er_buffer input,
                                           er_buffer output_a, er_buffer output_b,
                                           er_buffer output_c, uint32_t rows_a, uint32_t rows_b,
                                           uint32_t rows_c, uint32_t K) {
    const er_buffer Ws[3] = {weight_a, weight_b, weight_c}, ys[3] = {output_a, output_b, output_c};
    const uint32_t Ms[3] = {rows_a, rows_b, rows_c};
    return encode_q4k_multi(ctx, stream, Ws, input, ys, Ms, 3, K);
}

er_status er_hip_encode_q4k_weights_dual_geglu(er_hip_ctx *ctx, er_stream stream,
                                               er_buffer gate_weight, er_buffer up_weight,
                                               er_buffer input, er_buffer output, uint32_t M,
                                               uint32_t K) {
    return encode_q4k_geglu(ctx, stream, gate_weight, up_weight, input, output, M, K);
}

er_status er_hip_encode_q6k_weights_packed_top1(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                                er_buffer input, er_buffer partial_values,
                                                er_buffer partial_indices, er_buffer output_index,
                                                uint32_t M, uint32_t K) {
    return encode_q6k_top1(ctx, stream, weight, input, partial_values, partial_indices, output_index, M, K);
}

er_status er_hip_encode_q6k_weights_packed_top1_noalloc(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                                        er_buffer input, er_buffer output_index, uint32_t M,
                                                        uint32_t K) {
    return encode_q6k_top1_noalloc(ctx, stream, weight, input, output_index, M, K);
}

er_status er_hip_quantize_q8_0_rows(er_hip_ctx *ctx, er_stream stream, er_buffer source,
                                    er_buffer destination, uint32_t row_count,
                                    uint32_t source_row_stride, uint32_t destination_row_base,
                                    uint32_t blocks_per_row) {
    return encode_quantize_q8_0(ctx, stream, source, destination, row_count, source_row_stride,
                                destination_row_base, blocks_per_row);
}

er_status q8_fused_qkv(er_hip_ctx *ctx, er_stream stream, const char *name, bool vHalf, er_buffer wq,
                       er_buffer wk, er_buffer wv, er_buffer input, er_buffer out_q, er_buffer out_k,
                       er_buffer out_v, er_buffer norm_weight, uint32_t q_rows, uint32_t kv_rows, uint32_t cols,
                       uint32_t token_count, float rms_eps) {
    Q8FusedSpec f{};
    f.name = name;
    f.count = 3;
    f.W[0] = wq, f.W[1] = wk, f.W[2] = wv;
    f.y[0] = out_q, f.y[1] = out_k, f.y[2] = out_v;
    f.M[0] = q_rows, f.M[1] = kv_rows, f.M[2] = kv_rows;
    f.halfMask = vHalf ? 4u : 0u;
    f.normW = norm_weight;
    f.eps = rms_eps;
    if (!norm_weight.data) return fail(ER_ERR_INVALID_ARGUMENT, "%s: null norm weight", f.name);
    return encode_q8_fused(ctx, stream, f, input, token_count, cols);
}

er_status er_hip_q8_0_fused_qkv(er_hip_ctx *ctx, er_stream stream, er_buffer wq, er_buffer wk, er_buffer wv,
                                er_buffer input, er_buffer out_q, er_buffer out_k, er_buffer out_v_f16,
                                er_buffer norm_weight, uint32_t q_rows, uint32_t kv_rows, uint32_t cols,
                                uint32_t token_count, float rms_eps) {
    return q8_fused_qkv(ctx, stream, "dequant_q8_0_fused_qkv", true, wq, wk, wv, input, out_q, out_k, out_v_f16,
                        norm_weight, q_rows, kv_rows, cols, token_count, rms_eps);
}

er_status er_hip_q8_0_fused_qkv_turbo(er_hip_ctx *ctx, er_stream stream, er_buffer wq, er_buffer wk,
                                      er_buffer wv, er_buffer input, er_buffer out_q, er_buffer out_k,
                                      er_buffer out_v, er_buffer norm_weight, uint32_t q_rows,
                                      uint32_t kv_rows, uint32_t cols, uint32_t token_count, float rms_eps) {
    return q8_fused_qkv(ctx, stream, "dequant_q8_0_fused_qkv_turbo", false, wq, wk, wv, input, out_q, out_k,
                        out_v, norm_weight, q_rows, kv_rows, cols, token_count, rms_eps);
}

er_status er_hip_q8_0_fused_gate_up_silu(er_hip_ctx *ctx, er_stream stream, er_buffer w_gate,
                                         er_buffer w_up, er_buffer input, er_buffer activated,
                                         er_buffer norm_weight, uint32_t rows, uint32_t cols,
                                         uint32_t token_count, float rms_eps) {
    Q8FusedSpec f{};
    f.name = "dequant_q8_0_fused_gate_up_silu";
    f.count = 2;
    f.W[0] = w_gate, f.W[1] = w_up;
    f.y[0] = activated;
    f.M[0] = rows, f.M[1] = rows;
    f.normW = norm_weight;
    f.eps = rms_eps;
    f.silu = true;
    if (!norm_weight.data) return fail(ER_ERR_INVALID_ARGUMENT, "%s: null norm weight", f.name);
    return encode_q8_fused(ctx, stream, f, input, token_count, cols);
}

er_status er_hip_q8_0_fused_final_norm_gemv(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                            er_buffer input, er_buffer output, er_buffer norm_weight,
                                            uint32_t rows, uint32_t cols, float rms_eps) {
    Q8FusedSpec f{};
    f.name = "dequant_q8_0_fused_final_norm_gemv";
    f.count = 1;
    f.W[0] = weight;
    f.y[0] = output;
    f.M[0] = rows;
    f.normW = norm_weight;
    f.eps = rms_eps;
    if (!norm_weight.data) return fail(ER_ERR_INVALID_ARGUMENT, "%s: null norm weight", f.name);
    return encode_q8_fused(ctx, stream, f, input, 1, cols);
}

er_status er_hip_q8_0_gemv_f16out(er_hip_ctx *ctx, er_stream stream, er_buffer weight, er_buffer input,
                                  er_buffer output_f16, uint32_t rows, uint32_t cols) {
    Q8FusedSpec f{};
    f.name = "dequant_q8_0_gemv_f16out";
    f.count = 1;
    f.W[0] = weight;
    f.y[0] = output_f16;
    f.M[0] = rows;
    f.halfMask = 1u;
    return encode_q8_fused(ctx, stream, f, input, 1, cols);
}

er_status er_hip_q8_0_gemv_add(er_hip_ctx *ctx, er_stream stream, er_buffer weight, er_buffer input,
                               er_buffer residual, er_buffer output, uint32_t rows, uint32_t cols) {
    Q8FusedSpec f{};
    f.name = "dequant_q8_0_gemv_add";
    f.count = 1;
    f.W[0] = weight;
    f.y[0] = output;
    f.res[0] = residual;
    f.M[0] = rows;
    if (!residual.data) return fail(ER_ERR_INVALID_ARGUMENT, "%s: null residual", f.name);
    return encode_q8_fused(ctx, stream, f, input, 1, cols);
}

er_status er_hip_encode_batched_q4k_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                            er_buffer input, er_buffer output, uint32_t batch_seq,
                                            uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q4_K, weight, input, output, batch_seq, M, K);
}

er_status er_hip_encode_batched_q6k_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                            er_buffer input, er_buffer output, uint32_t batch_seq,
                                            uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q6_K, weight, input, output, batch_seq, M, K);
}

er_status er_hip_encode_batched_q8_0_weights(er_hip_ctx *ctx, er_stream stream, er_buffer weight,
                                             er_buffer input, er_buffer output, uint32_t batch_seq,
                                             uint32_t M, uint32_t K) {
    return encode_gemv(ctx, stream, Fmt::Q8_0, weight, input, output, batch_seq, M, K);
}

er_status er_hip_gemm_q4_k(er_hip_ctx *ctx, er_stream stream, er_buffer weight, er_buffer x_bf16,
                           er_buffer y, uint32_t tokens, uint32_t N, uint32_t K) {
    return encode_gemm(ctx, stream, Fmt::Q4_K, weight, x_bf16, y, tokens, N, K);
}

er_status er_hip_gemm_q8_0(er_hip_ctx *ctx, er_stream stream, er_buffer weight, er_buffer x_bf16,
                           er_buffer y, uint32_t tokens, uint32_t N, uint32_t K) {
    return encode_gemm(ctx, stream, Fmt::Q8_0, weight, x_bf16, y, tokens, N, K);
}

er_status er_hip_encode_projection(er_hip_ctx *ctx, er_stream stream,
                                   const er_tensor_storage *tensor, er_buffer input,
                                   er_buffer output, uint32_t tokens) {
    if (!tensor) return fail(ER_ERR_INVALID_ARGUMENT, "null tensor");
    if (tensor->ndim != 2 || tensor->shape[0] > 0xffffffffu || tensor->shape[1] > 0xffffffffu)
        return fail(ER_ERR_INVALID_MATRIX_SHAPE, "projection tensor must be 2-D [K, M]");
    if (tensor->byte_offset > tensor->buffer.length)
        return fail(ER_ERR_INVALID_MATRIX_SHAPE, "byteOffset beyond the tensor buffer");
    er_buffer W{(char *)tensor->buffer.data + tensor->byte_offset,
                tensor->buffer.length - tensor->byte_offset};
    const uint32_t K = (uint32_t)tensor->shape[0], M = (uint32_t)tensor->shape[1];
    switch (tensor->data_type) {
        case ER_TYPE_Q8_0: return encode_gemv(ctx, stream, Fmt::Q8_0, W, input, output, tokens, M, K);
        case ER_TYPE_Q4_K: return encode_gemv(ctx, stream, Fmt::Q4_K, W, input, output, tokens, M, K);
        case ER_TYPE_Q6_K: return encode_gemv(ctx, stream, Fmt::Q6_K, W, input, output, tokens, M, K);
        default:
            return fail(ER_ERR_INVALID_ARGUMENT,
                        "projection data type %u is not supported by the quantized GEMV path",
                        tensor->data_type);
    }
}

}  // extern "C"

#ifdef ER_WITH_PROBES
// ---- measurement kernels (er_hip_probe.h; the measurement library only) ----

// One workgroup per CU for the per-CU rate probes: 96 KB of LDS each, so no
// second workgroup fits beside it.
constexpr uint32_t kProbeCuLds = 96u * 1024u;

er_status er_hip_probe_lds_read(er_hip_ctx *ctx, er_stream stream, uint32_t waves, uint32_t iters, er_buffer sink) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if ((waves != 4 && waves != 8 && waves != 16) || !sink.data || !aligned(sink.data, 4) ||
        sink.length < (uint64_t)ctx->cu_count * 1024u * 4u)
        return fail(ER_ERR_INVALID_ARGUMENT, "lds read probe: waves %u (4, 8 or 16), sink %llu bytes", waves,
                    (unsigned long long)sink.length);
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    uint32_t never = 0x9e3779b9u;
    void *args[] = {&iters, &never, (void *)&sink.data};
    return launch(ctx, K_PROBE_LDS_READ, dim3((uint32_t)ctx->cu_count, 1, 1), dim3(64u * waves, 1, 1), kProbeCuLds,
                  stream, args);
}

er_status er_hip_probe_mfma_valu(er_hip_ctx *ctx, er_stream stream, uint32_t mode, uint32_t iters, er_buffer sink) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (mode > 5u || !sink.data || !aligned(sink.data, 4) || sink.length < (uint64_t)ctx->cu_count * 512u * 4u)
        return fail(ER_ERR_INVALID_ARGUMENT, "mfma/valu probe: mode %u (0..5), sink %llu bytes", mode,
                    (unsigned long long)sink.length);
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    uint32_t never = 0x9e3779b9u;
    void *args[] = {&mode, &iters, &never, (void *)&sink.data};
    return launch(ctx, K_PROBE_MFMA_VALU, dim3((uint32_t)ctx->cu_count, 1, 1), dim3(512, 1, 1), kProbeCuLds, stream,
                  args);
}

er_status er_hip_probe_stream_read(er_hip_ctx *ctx, er_stream stream, er_buffer src, uint64_t bytes,
                                   uint32_t workgroups, er_buffer sink) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (bytes % 16u != 0 || bytes > src.length || workgroups == 0 || sink.length < (uint64_t)workgroups * 256u * 4u)
        return fail(ER_ERR_INVALID_ARGUMENT, "stream read: %llu bytes of a %llu-byte source, %u workgroups, "
                    "sink %llu bytes", (unsigned long long)bytes, (unsigned long long)src.length, workgroups,
                    (unsigned long long)sink.length);
    if (!src.data || !sink.data || !aligned(src.data, 16) || !aligned(sink.data, 4))
        return fail(ER_ERR_INVALID_ARGUMENT, "stream read: null or misaligned buffer");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    uint64_t n16 = bytes / 16u;
    uint32_t never = 0x9e3779b9u;
    void *args[] = {&src.data, &n16, &never, &sink.data};
    return launch(ctx, K_PROBE_STREAM_READ, dim3(workgroups, 1, 1), dim3(256, 1, 1), 0, stream, args);
}

er_status er_hip_probe_gemm_clock(er_hip_ctx *ctx, er_stream stream, er_tensor_type type, er_buffer weight,
                                  er_buffer x_bf16, er_buffer y, uint32_t tokens, uint32_t N, uint32_t K,
                                  er_buffer stamps, uint32_t *items) {
    if (type != ER_TYPE_Q4_K && type != ER_TYPE_Q8_0)
        return fail(ER_ERR_INVALID_ARGUMENT, "GEMM clock probe: type %d is not Q4_K or Q8_0", (int)type);
    if (!items) return fail(ER_ERR_INVALID_ARGUMENT, "GEMM clock probe: null items");
    *items = 0;
    return encode_gemm(ctx, stream, type == ER_TYPE_Q4_K ? Fmt::Q4_K : Fmt::Q8_0, weight, x_bf16, y, tokens, N, K,
                       &stamps, items);
}

er_status er_hip_probe_empty(er_hip_ctx *ctx, er_stream stream) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    return launch(ctx, K_PROBE_EMPTY, dim3(1, 1, 1), dim3(64, 1, 1), 0, stream, nullptr);
}

er_status er_hip_probe_grid_barrier(er_hip_ctx *ctx, er_stream stream, uint32_t workgroups, uint32_t rounds,
                                    uint32_t spin_limit, er_buffer counter, er_buffer out) {
    er_status st = check_ctx(ctx);
    if (st != ER_OK) return st;
    if (workgroups == 0 || workgroups > (uint32_t)ctx->cu_count || spin_limit == 0)
        return fail(ER_ERR_INVALID_ARGUMENT, "grid barrier: %u workgroups (1..%d resident), spin limit %u",
                    workgroups, ctx->cu_count, spin_limit);
    if (!counter.data || !out.data || counter.length < 16u || out.length < 16u || !aligned(counter.data, 16) ||
        !aligned(out.data, 16))
        return fail(ER_ERR_INVALID_ARGUMENT, "grid barrier: counter and out need 16 aligned bytes each");
    st = bind_device(ctx);
    if (st != ER_OK) return st;
    uint64_t one = 1;
    void *za[] = {&counter.data, &one};
    st = launch(ctx, K_FILL_ZERO, dim3(1, 1, 1), dim3(256, 1, 1), 0, stream, za);
    if (st != ER_OK) return st;
    void *args[] = {&counter.data, &rounds, &spin_limit, &out.data};
    return launch(ctx, K_PROBE_GRID_BARRIER, dim3(workgroups, 1, 1), dim3(64, 1, 1), 0, stream, args);
}
#endif  // ER_WITH_PROBES
