// The input table of a grouped GEMV plan's staging pass, shared by the host runtime and the kernels.
// A large plan stages each distinct input row once per run (brik_gemv_stage_<fmt>: one block per
// entry, writing the block's LDS image of the staged row to the plan's stage buffer at `off`); the
// plan's blocks then copy that image into LDS instead of each computing it.
#pragma once
#include <stdint.h>

typedef struct brik_stage_input {
    const float* x;        // the job's activation row
    const float* gate;     // fused transform of the job (brik_gemv_job_ex), or null
    const float* norm_w;
    float eps;
    int32_t flags;
    int32_t K;
    uint32_t off;          // byte offset of the staged image in the stage buffer (16-byte aligned)
} brik_stage_input;
