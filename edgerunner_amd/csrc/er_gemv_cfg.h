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
