// er_scratch.h -- size of the device scratch array of the allocation-free
// entry points, shared by the kernel code object and the host library.
//
// The array holds the (value, row) partials of the Q6_K greedy top-1 head
// when no caller buffer brings them: one partial per workgroup, at most one
// per 4 rows, so ER_SCRATCH_TOP1_PARTIALS partials serve every head of up to
// 4 * ER_SCRATCH_TOP1_PARTIALS rows (ER_HIP_TOP1_NOALLOC_MAX_ROWS in er_hip.h).
#pragma once

#define ER_SCRATCH_TOP1_PARTIALS 65536u
// values (fp32) in the first half, rows (uint32) in the second
#define ER_SCRATCH_BYTES (ER_SCRATCH_TOP1_PARTIALS * 8u)
