// Tables of a grouped GEMV plan, shared by the host runtime and the kernels.
//
// The input table of a plan's staging pass.
// A large plan stages each distinct input row once per run (brik_gemv_stage_<fmt>: one block per
// entry, writing the block's LDS image of the staged row to the plan's stage buffer at `off`); the
// plan's blocks then copy that image into LDS instead of each computing it.
#pragma once
#include <stdint.h>

#include "../../../include/brik.h"   // brik_gemv_job_ex

typedef struct brik_stage_input {
    const float* x;        // the job's activation row
    const float* gate;     // fused transform of the job (brik_gemv_job_ex), or null
    const float* norm_w;
    float eps;
    int32_t flags;
    int32_t K;
    uint32_t off;          // byte offset of the staged image in the stage buffer (16-byte aligned)
} brik_stage_input;

// One block of a grouped GEMV launch: its job, the rows [r0, r1) of that job it computes, the byte
// offset of the job's staged input image in the plan's stage buffer, and how many groups of that image
// a producer wrote (0: all of them; else the block stages the rest itself). Block b reads entry b, so
// everything it needs arrives with one scalar load round trip; a lookup of the job by block index
// (a search over per-job block counts, then the job record) took several dependent ones.
typedef struct brik_gemv_block {
    brik_gemv_job_ex job;
    int32_t r0, r1;
    uint32_t stage_off;
    uint32_t img_groups;
    uint32_t pad[6];       // 128 bytes
} brik_gemv_block;
