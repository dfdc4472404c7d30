// er_gemv_cfg.h -- launch configurations of the integer-dot GEMV kernels,
// shared by the device code (one kernel per entry) and the host dispatcher
// (kernel name table and selection).
//
// Entry X(LPR, NS, R): LPR lanes per row (64/LPR rows groups per wave), NS
// 64-weight slots per lane per row, R rows per lane group.  NS * R <= 8 keeps
// the in-flight weight registers of a lane at <= 96 VGPRs.
#pragma once

#define ER_GEMV_WAVES 4

#define ER_I8_CONFIGS_L(X, LPR) \
    X(LPR, 1, 4) X(LPR, 1, 2) X(LPR, 1, 1) \
    X(LPR, 2, 4) X(LPR, 2, 2) X(LPR, 2, 1) \
    X(LPR, 3, 2) X(LPR, 3, 1) \
    X(LPR, 4, 2) X(LPR, 4, 1) \
    X(LPR, 5, 1) X(LPR, 6, 1) X(LPR, 7, 1) X(LPR, 8, 1)

#define ER_I8_CONFIGS(X) \
    ER_I8_CONFIGS_L(X, 64) ER_I8_CONFIGS_L(X, 32) ER_I8_CONFIGS_L(X, 16) ER_I8_CONFIGS_L(X, 4)

// Multi-matrix / GeGLU Q4_K kernels: R in {2, 4} row computations per lane
// group (GeGLU pairs a gate and an up row, so R is even).
#define ER_I8_MULTI_CONFIGS_L(X, LPR) \
    X(LPR, 1, 4) X(LPR, 1, 2) X(LPR, 2, 4) X(LPR, 2, 2) X(LPR, 3, 2) X(LPR, 4, 2)

#define ER_I8_MULTI_CONFIGS(X) \
    ER_I8_MULTI_CONFIGS_L(X, 64) ER_I8_MULTI_CONFIGS_L(X, 32) ER_I8_MULTI_CONFIGS_L(X, 16) \
    ER_I8_MULTI_CONFIGS_L(X, 4)

// One row computation per lane group, for the multi-matrix kernels whose rows
// stand alone (Q4_K dual / triple, fused Q8_0 QKV; not the paired GeGLU and
// gate/up + SiLU): the most workgroups for a latency-bound launch.
#define ER_I8_MULTI1_CONFIGS_L(X, LPR) X(LPR, 1, 1) X(LPR, 2, 1) X(LPR, 3, 1) X(LPR, 4, 1)
#define ER_I8_MULTI1_CONFIGS(X) \
    ER_I8_MULTI1_CONFIGS_L(X, 64) ER_I8_MULTI1_CONFIGS_L(X, 32) ER_I8_MULTI1_CONFIGS_L(X, 16) \
    ER_I8_MULTI1_CONFIGS_L(X, 4)

// CU-resident Q4_K / Q8_0 / Q6_K kernels (family 3): X(LPR, NS, MAXJ), one 8-wave
// workgroup per CU-sized share of the rows, unrolled kernels for 1..MAXJ row
// steps per wave, and for MAXJ == 8 a rolled one for up to ER_CU_MAX_ROLLED.
// With more slots per lane than MAXJ allows, the unrolled steps keep too many
// slots of x limbs or weights live and the kernels spill.
#ifndef ER_CU_WAVES
#define ER_CU_WAVES 8
#endif
#define ER_CU_MAX_STEPS 8
#define ER_CU_MAX_ROLLED 64  // steps per lane group: one parked sum per lane per register
#define ER_CU_CONFIGS_Q4K(X) \
    X(16, 1, 8) X(16, 2, 8) X(32, 1, 8) X(32, 2, 8) X(64, 1, 8) X(64, 2, 8) X(64, 3, 2) X(64, 4, 2) X(32, 7, 1)
#define ER_CU_CONFIGS_Q8(X) X(16, 1, 8) X(32, 1, 8) X(64, 1, 8)
#define ER_CU_CONFIGS_Q6K(X) X(16, 1, 8) X(32, 1, 8) X(64, 1, 8)

// K-sliced CU-resident Q4_K / Q8_0 kernels for 8192 < K <= 16384 (gemv_cuk):
// one kernel per row-step count 1..ER_CUK_MAX_STEPS (2 rows per step).
#define ER_CUK_MAX_STEPS 16
