// Standalone dequantization of .brik planes to f32: the bit-exactness check of the in-register
// dequant the matmul kernels use. Reference semantics: dequantizeQ8/Q4/Q3
// (src/lib/brik/q8web.ts:74-83, q4web.ts:82-96, q3web.ts:97-110).
//
// Exactness argument: code*s is exact in f32 (<= 8-bit code times an 11-bit half mantissa),
// so fmaf(code, s, m) rounds the exact q*s+m once, as the reference's double expression rounded
// once into a Float32Array does.
#include "common.h"

// One thread per 8 elements (one 32-bit word of nibbles / two of int8 / one byte of q3 slots).
extern "C" __global__ __launch_bounds__(256) void brik_dequant_q8(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ sc, float* __restrict__ out,
    uint64_t n8)
{
    uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n8) return;
    uint64_t e0 = t * 8;
    u32x2_t w = *(const u32x2_t*)(codes + e0);
    float s = f16_bits_to_f32(sc[e0 / BRIK_GROUP]);
    f32x4_t o0, o1;
    for (int b = 0; b < 4; ++b) o0[b] = (float)(int8_t)byte_of(w.x, b) * s;
    for (int b = 0; b < 4; ++b) o1[b] = (float)(int8_t)byte_of(w.y, b) * s;
    *(f32x4_t*)(out + e0) = o0;
    *(f32x4_t*)(out + e0 + 4) = o1;
}

extern "C" __global__ __launch_bounds__(256) void brik_dequant_q4(
    const uint8_t* __restrict__ nib, const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn,
    float* __restrict__ out, uint64_t n8)
{
    uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n8) return;
    uint64_t e0 = t * 8;
    uint32_t w = *(const uint32_t*)(nib + e0 / 2);
    float s = f16_bits_to_f32(sc[e0 / BRIK_GROUP]);
    float m = f16_bits_to_f32(mn[e0 / BRIK_GROUP]);
    f32x4_t o0, o1;
    // nibble j of the word is element e0 + j (low nibble = even index, q4web.ts:48-49)
    for (int j = 0; j < 4; ++j) o0[j] = __builtin_fmaf((float)((w >> (4 * j)) & 15u), s, m);
    for (int j = 0; j < 4; ++j) o1[j] = __builtin_fmaf((float)((w >> (4 * (j + 4))) & 15u), s, m);
    *(f32x4_t*)(out + e0) = o0;
    *(f32x4_t*)(out + e0 + 4) = o1;
}

extern "C" __global__ __launch_bounds__(256) void brik_dequant_q3(
    const uint32_t* __restrict__ lo, const uint32_t* __restrict__ hi, const uint16_t* __restrict__ sc,
    const uint16_t* __restrict__ mn, float* __restrict__ out, uint64_t n8)
{
    uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n8) return;
    uint64_t e0 = t * 8;
    // code i: 2 low bits at lo[i>>4] bit (i&15)*2, high bit at hi[i>>5] bit (i&31) (q3web.ts:55-56)
    uint32_t l = lo[e0 >> 4] >> ((e0 & 15) * 2);
    uint32_t h = hi[e0 >> 5] >> (e0 & 31);
    float s = f16_bits_to_f32(sc[e0 / BRIK_GROUP]);
    float m = f16_bits_to_f32(mn[e0 / BRIK_GROUP]);
    f32x4_t o0, o1;
    for (int j = 0; j < 4; ++j)
        o0[j] = __builtin_fmaf((float)(((l >> (2 * j)) & 3u) | (((h >> j) & 1u) << 2)), s, m);
    for (int j = 4; j < 8; ++j)
        o1[j - 4] = __builtin_fmaf((float)(((l >> (2 * j)) & 3u) | (((h >> j) & 1u) << 2)), s, m);
    *(f32x4_t*)(out + e0) = o0;
    *(f32x4_t*)(out + e0 + 4) = o1;
}

// y[0, n) = 0: the K == 0 matmul (empty sums). A kernel rather than a memset node, so a caller may
// capture it in a graph.
extern "C" __global__ __launch_bounds__(256) void brik_fill_zero(float* __restrict__ y, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) y[i] = 0.f;
}
