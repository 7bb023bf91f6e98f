// Prefill / grouped GEMM: y[M, N] = x[M, K] . deq(W[N, K])^T on CDNA4 matrix cores.
// Replaces the reference's tiled and shared-memory WGSL kernels (matmul_t_q4_tiled / _shared,
// matmul_t_q8_tiled / _shared, src/lib/webgpu/shaders.ts:120-168, 425-527, 531-577; and
// matmul_t_q3 for M > 1, :323-369), which run scalar f32 FMAs over 16x16 LDS tiles.
//
// Per K step of 32 (exactly one quantization group):
//   * x tile  BM x 32: f32 from HBM -> f16 -> LDS
//   * W tile  BN x 32: packed codes + the group's f16 scale/min -> dequantized f32
//     (fmaf(q, s, m), the reference's value) -> f16 -> LDS
//   * each of the 4 waves runs v_mfma_f32_16x16x32_f16 over its 32 x 32 sub-tile, f32 accumulate.
// f16 (not bf16) operands: 11-bit significands keep the normwise error near 3e-4, inside the
// 1e-3 bar; bf16's 8 bits would not.
//
// Grouped (MoE) mode: row_off != nullptr. Rows of x / y are sorted by expert; expert e owns rows
// [row_off[e], row_off[e+1]) and the weight slice e of a stacked [E, N, K] q-tensor. blockIdx.y
// enumerates (expert, 64-row tile) pairs; blocks past the last pair exit.
#include "common.h"

namespace {

constexpr int BM = 64, BN = 64, BK = 32;
constexpr int LDK = BK + 8;   // LDS row stride in halves (16-byte pad)

// Dequantize 8 consecutive elements (k = 8d .. 8d+7 of group g) of weight row n into halves.
template <int FMT>
__device__ __forceinline__ half8_t deq8(const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,
                                        const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn,
                                        size_t flat_g, int d)
{
    half8_t h;
    const float s = f16_bits_to_f32(sc[flat_g]);
    if constexpr (FMT == FMT_Q8) {
        const u32x2_t w = *((const u32x2_t*)p0 + flat_g * 4 + d);
#pragma unroll
        for (int b = 0; b < 4; ++b) h[b] = (_Float16)((float)(int8_t)byte_of(w.x, b) * s);
#pragma unroll
        for (int b = 0; b < 4; ++b) h[4 + b] = (_Float16)((float)(int8_t)byte_of(w.y, b) * s);
    } else {
        const float m = f16_bits_to_f32(mn[flat_g]);
        if constexpr (FMT == FMT_Q4) {
            const uint32_t w = *((const uint32_t*)p0 + flat_g * 4 + d);
#pragma unroll
            for (int j = 0; j < 8; ++j) h[j] = (_Float16)__builtin_fmaf((float)((w >> (4 * j)) & 15u), s, m);
        } else {
            // elements 8d .. 8d+7: lo word d>>1 at bit 16*(d&1), hi word bits 8d ..
            const uint32_t l = *((const uint32_t*)p0 + flat_g * 2 + (d >> 1)) >> (16 * (d & 1));
            const uint32_t hb = *((const uint32_t*)p1 + flat_g) >> (8 * d);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t q = ((l >> (2 * j)) & 3u) | (((hb >> j) & 1u) << 2);
                h[j] = (_Float16)__builtin_fmaf((float)q, s, m);
            }
        }
    }
    return h;
}

template <int FMT>
__device__ __forceinline__ void gemm_body(const float* __restrict__ x, const uint8_t* __restrict__ p0,
                                          const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc,
                                          const uint16_t* __restrict__ mn, float* __restrict__ y,
                                          int M, int K, int N, const int* __restrict__ row_off, int E)
{
    __shared__ _Float16 As[BM * LDK];
    __shared__ _Float16 Bs[BN * LDK];

    const int G = K / BRIK_GROUP;
    const int n0 = blockIdx.x * BN;
    int m0 = blockIdx.y * BM, m_end = M;
    size_t g_base = 0;          // flat group offset of this block's weight matrix

    if (row_off) {
        // find (expert e, tile t) for this blockIdx.y: tiles are enumerated expert by expert
        int remaining = blockIdx.y, e = 0;
        for (; e < E; ++e) {
            const int cnt = row_off[e + 1] - row_off[e];
            const int tiles = (cnt + BM - 1) / BM;
            if (remaining < tiles) break;
            remaining -= tiles;
        }
        if (e >= E) return;     // uniform across the block, before any barrier
        m0 = row_off[e] + remaining * BM;
        m_end = row_off[e + 1];
        g_base = (size_t)e * N * G;
    }

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    floatx4_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    const int sr = tid >> 2, sd = tid & 3;      // staging: row sr, 8-element chunk sd
    for (int g = 0; g < G; ++g) {
        {   // x tile
            const int m = m0 + sr;
            half8_t h;
            if (m < m_end) {
                const float* xp = x + (size_t)m * K + g * BK + sd * 8;
                const f32x4_t a0 = *(const f32x4_t*)xp, a1 = *(const f32x4_t*)(xp + 4);
#pragma unroll
                for (int t = 0; t < 4; ++t) { h[t] = (_Float16)a0[t]; h[4 + t] = (_Float16)a1[t]; }
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) h[t] = (_Float16)0.f;
            }
            *(half8_t*)(As + sr * LDK + sd * 8) = h;
        }
        {   // W tile
            const int n = n0 + sr;
            half8_t h;
            if (n < N) {
                h = deq8<FMT>(p0, p1, sc, mn, g_base + (size_t)n * G + g, sd);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) h[t] = (_Float16)0.f;
            }
            *(half8_t*)(Bs + sr * LDK + sd * 8) = h;
        }
        __syncthreads();
        half8_t a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = *(const half8_t*)(As + (wm + i * 16 + (lane & 15)) * LDK + (lane >> 4) * 8);
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = *(const half8_t*)(Bs + (wn + j * 16 + (lane & 15)) * LDK + (lane >> 4) * 8);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        __syncthreads();
    }

    // D layout: lane holds column (lane & 15), rows 4 * (lane >> 4) + r
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn + j * 16 + (lane & 15);
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm + i * 16 + 4 * (lane >> 4) + r;
                if (m < m_end) y[(size_t)m * N + n] = acc[i][j][r];
            }
        }
}

}  // namespace

#define BRIK_GEMM(NAME, FMT)                                                                        \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                         \
        const float* __restrict__ x, const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1, \
        const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, float* __restrict__ y,    \
        int M, int K, int N, const int* __restrict__ row_off, int E)                               \
    {                                                                                               \
        gemm_body<FMT>(x, p0, p1, sc, mn, y, M, K, N, row_off, E);                                  \
    }

BRIK_GEMM(brik_gemm_q4, FMT_Q4)
BRIK_GEMM(brik_gemm_q8, FMT_Q8)
BRIK_GEMM(brik_gemm_q3, FMT_Q3)
