// Decode GEMV: y[m, :] = x[m, :] . deq(W)^T for one activation row per grid.y, streaming the
// packed .brik planes once. Replaces the reference's 1-row WGSL kernels matmul_t_q8 / _q4 / _q3
// (src/lib/webgpu/shaders.ts:376-418, 77-114, 323-369), which give each output to one thread
// and walk its weight row serially with 32-bit loads.
//
// Mapping (wave64, 256-thread blocks):
//   * a "team" of TEAM lanes (16, 32 or 64; a DPP row is 16 lanes) owns one weight row at a time;
//     lane l of the team handles the row's groups g = l, l + TEAM, ... so the team's loads of one
//     step are TEAM consecutive groups: TEAM x 16 contiguous bytes for q4 (one 128-bit load per
//     lane per group), fully coalesced.
//   * the activation row is staged once per block in LDS, 16-byte chunks XOR-swizzled inside each
//     32-float group so the lanes of a team (stride of one group) hit distinct banks.
//   * the per-group scale factors out of the dot: y = sum_g s_g * (sum_{k in g} x_k q_k)
//     + m_g * (sum_{k in g} x_k). The group sums of x are computed once at staging.
//   * the TEAM partial sums of a row are reduced with cross-lane shuffles; lane 0 writes y.
#include "common.h"
#include "../../../include/brik.h"   // brik_gemv_job

namespace {

// x chunk c (4 floats) of group g lives at float offset g*32 + ((c ^ (g & 7)) * 4).
__device__ __forceinline__ int xsw(int g, int c) { return g * 32 + ((c ^ (g & 7)) << 2); }

// Stage one activation row (K floats) into LDS and compute its 32-element group sums.
__device__ __forceinline__ void stage_x(const float* __restrict__ xrow, float* xl, float* xsum, int K)
{
    const int nq = K >> 2;               // float4 chunks
    for (int i = threadIdx.x; i < nq; i += blockDim.x) {
        f32x4_t v = *(const f32x4_t*)(xrow + 4 * i);
        const int g = i >> 3, c = i & 7;
        *(f32x4_t*)(xl + xsw(g, c)) = v;
        // group sum: the 8 chunks of a group sit in 8 consecutive lanes (blockDim % 8 == 0)
        float p = (v.x + v.y) + (v.z + v.w);
        p += __shfl_xor(p, 1, 8);
        p += __shfl_xor(p, 2, 8);
        p += __shfl_xor(p, 4, 8);
        if (c == 0) xsum[g] = p;
    }
}

template <int TEAM>
__device__ __forceinline__ float team_sum(float v)
{
#pragma unroll
    for (int off = TEAM / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, TEAM);
    return v;
}

// sum_{k in group} x_k * q_k for one group, per format. xg points at the group's swizzled chunks.
__device__ __forceinline__ float dot_q4(const float* xl, int g, u32x4_t w)
{
    float p = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {          // word j holds elements 8j .. 8j+7
        const uint32_t wj = w[j];
        const uint32_t lo = wj & 0x0f0f0f0fu;          // bytes: elements 8j+0, +2, +4, +6
        const uint32_t hi = (wj >> 4) & 0x0f0f0f0fu;   // bytes: elements 8j+1, +3, +5, +7
        const f32x4_t xa = *(const f32x4_t*)(xl + xsw(g, 2 * j));
        const f32x4_t xb = *(const f32x4_t*)(xl + xsw(g, 2 * j + 1));
        p = __builtin_fmaf(xa.x, (float)byte_of(lo, 0), p);
        p = __builtin_fmaf(xa.y, (float)byte_of(hi, 0), p);
        p = __builtin_fmaf(xa.z, (float)byte_of(lo, 1), p);
        p = __builtin_fmaf(xa.w, (float)byte_of(hi, 1), p);
        p = __builtin_fmaf(xb.x, (float)byte_of(lo, 2), p);
        p = __builtin_fmaf(xb.y, (float)byte_of(hi, 2), p);
        p = __builtin_fmaf(xb.z, (float)byte_of(lo, 3), p);
        p = __builtin_fmaf(xb.w, (float)byte_of(hi, 3), p);
    }
    return p;
}

__device__ __forceinline__ float dot_q8(const float* xl, int g, u32x4_t w0, u32x4_t w1)
{
    float p = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {          // word c holds elements 4c .. 4c+3
        const uint32_t wc = c < 4 ? w0[c] : w1[c - 4];
        const f32x4_t xv = *(const f32x4_t*)(xl + xsw(g, c));
        p = __builtin_fmaf(xv.x, (float)(int8_t)byte_of(wc, 0), p);
        p = __builtin_fmaf(xv.y, (float)(int8_t)byte_of(wc, 1), p);
        p = __builtin_fmaf(xv.z, (float)(int8_t)byte_of(wc, 2), p);
        p = __builtin_fmaf(xv.w, (float)(int8_t)byte_of(wc, 3), p);
    }
    return p;
}

__device__ __forceinline__ float dot_q3(const float* xl, int g, u32x2_t l, uint32_t h)
{
    float p = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {          // chunk c: elements 4c .. 4c+3
        const uint32_t lw = l[c >> 2] >> ((c & 3) * 8);
        const uint32_t hw = h >> (4 * c);
        const f32x4_t xv = *(const f32x4_t*)(xl + xsw(g, c));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t q = ((lw >> (2 * t)) & 3u) | (((hw >> t) & 1u) << 2);
            p = __builtin_fmaf(xv[t], (float)q, p);
        }
    }
    return p;
}

// Rows [r0, r1) of one weight matrix, TEAM lanes per row, x already staged in LDS.
template <int FMT, int TEAM>
__device__ __forceinline__ void gemv_rows(const float* xl, const float* xsum, const uint8_t* __restrict__ p0,
                                          const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc,
                                          const uint16_t* __restrict__ mn, float* __restrict__ yrow,
                                          int G, int r0, int r1, int rstep)
{
    const int lane = threadIdx.x % TEAM;
    const int team = threadIdx.x / TEAM;
    for (int n = r0 + team; n < r1; n += rstep) {
        const size_t gb = (size_t)n * G;      // first flat group of row n
        float acc = 0.f;
        for (int g = lane; g < G; g += TEAM) {
            float p;
            if constexpr (FMT == FMT_Q4) {
                const u32x4_t w = ld_stream((const u32x4_t*)p0 + gb + g);
                p = dot_q4(xl, g, w);
            } else if constexpr (FMT == FMT_Q8) {
                const u32x4_t* wp = (const u32x4_t*)p0 + 2 * (gb + g);
                const u32x4_t w0 = ld_stream(wp), w1 = ld_stream(wp + 1);
                p = dot_q8(xl, g, w0, w1);
            } else {
                const u32x2_t l = ld_stream((const u32x2_t*)p0 + gb + g);
                const uint32_t h = ld_stream((const uint32_t*)p1 + gb + g);
                p = dot_q3(xl, g, l, h);
            }
            const float s = f16_bits_to_f32(sc[gb + g]);
            acc = __builtin_fmaf(s, p, acc);
            if constexpr (FMT != FMT_Q8) {
                const float mm = f16_bits_to_f32(mn[gb + g]);
                acc = __builtin_fmaf(mm, xsum[g], acc);
            }
        }
        acc = team_sum<TEAM>(acc);
        if (lane == 0) yrow[n] = acc;
    }
}

template <int FMT, int TEAM>
__device__ __forceinline__ void gemv_body(const float* __restrict__ x, const uint8_t* __restrict__ p0,
                                          const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc,
                                          const uint16_t* __restrict__ mn, float* __restrict__ y, int K, int N)
{
    extern __shared__ float lds[];
    const int G = K / BRIK_GROUP;
    float* xl = lds;
    float* xsum = lds + K;
    const int m = blockIdx.y;
    stage_x(x + (size_t)m * K, xl, xsum, K);
    __syncthreads();
    constexpr int RPB = 256 / TEAM;      // rows in flight per block
    gemv_rows<FMT, TEAM>(xl, xsum, p0, p1, sc, mn, y + (size_t)m * N, G, blockIdx.x * RPB, N, gridDim.x * RPB);
}

// Grouped GEMV over a job table: block b runs rows [rb * rows_per_block, ...) of job j, where
// block_start[j] <= b < block_start[j + 1] (a prefix over the jobs' block counts).
template <int FMT, int TEAM>
__device__ __forceinline__ void gemv_grouped_body(const brik_gemv_job* __restrict__ jobs,
                                                  const uint32_t* __restrict__ block_start, int njobs,
                                                  int rows_per_block)
{
    extern __shared__ float lds[];
    const uint32_t b = blockIdx.x;
    int lo = 0, hi = njobs - 1;          // last j with block_start[j] <= b
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (block_start[mid] <= b) lo = mid; else hi = mid - 1;
    }
    const brik_gemv_job job = jobs[lo];
    const int K = job.K, G = K / BRIK_GROUP;
    float* xl = lds;
    float* xsum = lds + K;
    stage_x(job.x, xl, xsum, K);
    __syncthreads();
    const int r0 = (int)(b - block_start[lo]) * rows_per_block;
    const int r1 = min(job.N, r0 + rows_per_block);
    constexpr int RPB = 256 / TEAM;
    gemv_rows<FMT, TEAM>(xl, xsum, (const uint8_t*)job.p0, (const uint8_t*)job.p1, job.scales, job.mins,
                         job.y, G, r0, r1, RPB);
}

}  // namespace

#define BRIK_GEMV(NAME, FMT, TEAM)                                                                  \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                         \
        const float* __restrict__ x, const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1, \
        const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, float* __restrict__ y,    \
        int K, int N)                                                                               \
    {                                                                                               \
        gemv_body<FMT, TEAM>(x, p0, p1, sc, mn, y, K, N);                                           \
    }

BRIK_GEMV(brik_gemv_q4_t16, FMT_Q4, 16)
BRIK_GEMV(brik_gemv_q4_t32, FMT_Q4, 32)
BRIK_GEMV(brik_gemv_q4_t64, FMT_Q4, 64)
BRIK_GEMV(brik_gemv_q8_t16, FMT_Q8, 16)
BRIK_GEMV(brik_gemv_q8_t32, FMT_Q8, 32)
BRIK_GEMV(brik_gemv_q8_t64, FMT_Q8, 64)
BRIK_GEMV(brik_gemv_q3_t16, FMT_Q3, 16)
BRIK_GEMV(brik_gemv_q3_t32, FMT_Q3, 32)
BRIK_GEMV(brik_gemv_q3_t64, FMT_Q3, 64)

#define BRIK_GEMV_GROUPED(NAME, FMT, TEAM)                                                          \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                         \
        const brik_gemv_job* __restrict__ jobs, const uint32_t* __restrict__ block_start, int njobs,  \
        int rows_per_block)                                                                         \
    {                                                                                               \
        gemv_grouped_body<FMT, TEAM>(jobs, block_start, njobs, rows_per_block);                     \
    }

BRIK_GEMV_GROUPED(brik_gemv_grouped_q4_t16, FMT_Q4, 16)
BRIK_GEMV_GROUPED(brik_gemv_grouped_q4_t32, FMT_Q4, 32)
BRIK_GEMV_GROUPED(brik_gemv_grouped_q4_t64, FMT_Q4, 64)
BRIK_GEMV_GROUPED(brik_gemv_grouped_q8_t16, FMT_Q8, 16)
BRIK_GEMV_GROUPED(brik_gemv_grouped_q8_t32, FMT_Q8, 32)
BRIK_GEMV_GROUPED(brik_gemv_grouped_q8_t64, FMT_Q8, 64)
BRIK_GEMV_GROUPED(brik_gemv_grouped_q3_t16, FMT_Q3, 16)
BRIK_GEMV_GROUPED(brik_gemv_grouped_q3_t32, FMT_Q3, 32)
BRIK_GEMV_GROUPED(brik_gemv_grouped_q3_t64, FMT_Q3, 64)
