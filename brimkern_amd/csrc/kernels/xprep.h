// Activation staging for the decode GEMV: one f32 row x[K] -> LDS as 24-bit block floating point.
//
// Per 32-element group g (the quantization group of the weights), with e_g the binary exponent of
// max|x| over the group (frexp), every element becomes the integer X = rint(x * 2^(22 - e_g)),
// |X| < 2^22, split into three signed bytes X = h * 65536 + m * 256 + l (h, m, l in [-128, 127]).
// The dot products with the integer weight codes then run on v_dot4_i32_i8 (four int8 MACs per lane
// per instruction, exact int32 sums), and the group's result is rescaled by 2^(e_g - 22) in f32.
// Relative to the group's largest element this keeps 22 bits, about f32's 24-bit significand.
//
// LDS layout for K = 32 * G, group-major so a group's limbs are reached with immediate offsets:
//   limbs: group g (0 <= g <= G) occupies bytes [96g, 96g + 96): limb t (0 = h, 1 = m, 2 = l) at
//          96g + 32t, its 32 bytes in the byte order the format's code unpacking produces (code_pos),
//          the two 16-byte halves swapped when bit 3 of g is set (so lanes reading groups g and g + 8
//          in one instruction hit different banks). Group G is all zeros: consumers point groups past
//          the end of a row at it, which zeroes their contribution without a select;
//   xse[g]: {f32 sum of the group's x, int32 e_g - 22}, g <= G, xse[G] = {0, 0};
//   flag:  int32, nonzero if the row holds a non-finite value (the exact f32 path then runs);
//   inv:   f32, the RMSNorm factor of a fused input transform (1 without one), and 4 words of scratch
//          for its block reduction.
//
// Fused input transform (grouped plans, brik_gemv_job_ex): the staged row may be
//   act(gate[k]) * x[k]                  (SwiGLU act = SiLU, GeGLU act = tanh-GELU), then / or
//   v[k] * inv * g[k],  inv = 1 / sqrt(sum v^2 / K + eps),  g = w or 1 + w   (RMSNorm)
// as the reference computes n1 = rmsnorm(x) and g = swiglu(gate, up) before recMM
// (src/lib/webgpu/shaders.ts:580-626; kernels.ts:1701, 1723, 1726).
#pragma once
#include "common.h"
#include "../../../include/brik.h"   // BRIK_JOB_* flags

namespace brik {

// Byte position, inside a group's 32 limb bytes (before the half swap), of group element e.
//   q8: codes are already bytes in element order.
//   q4: code dword j (elements 8j..8j+7) unpacks to two byte dwords: (w & 0x0f0f0f0f) holds elements
//       8j, 8j+2, 8j+4, 8j+6 and ((w >> 4) & 0x0f0f0f0f) holds 8j+1, 8j+3, 8j+5, 8j+7; they are
//       byte dwords 2j and 2j+1.
//   q3: byte dword s (0..7) holds codes s, s+8, s+16, s+24 (see unpack in gemv.hip).
template <int FMT>
__device__ __forceinline__ int code_pos(int e)
{
    if constexpr (FMT == FMT_Q8) return e;
    else if constexpr (FMT == FMT_Q4) return ((2 * (e >> 3) + (e & 1)) << 2) + ((e & 7) >> 1);
    else return ((e & 7) << 2) + (e >> 3);
}

__device__ __forceinline__ int half_swap(int g) { return ((g >> 3) & 1) << 4; }

struct XStage {
    int8_t* limbs;
    float2* xse;      // {sum, bit-cast int exponent}
    int* flag;
    float* inv;       // inv, then 4 reduction slots
    int G;
};

// Bytes of the staged row; the block's partial-sum buffer follows at this offset (4-byte aligned).
__host__ __device__ __forceinline__ size_t xstage_bytes(int K)
{
    return (size_t)104 * (K / BRIK_GROUP + 1) + 32;
}

__device__ __forceinline__ XStage xstage_layout(void* lds, int K)
{
    XStage s;
    s.G = K / BRIK_GROUP;
    s.limbs = (int8_t*)lds;
    s.xse = (float2*)((char*)lds + (size_t)96 * (s.G + 1));
    s.flag = (int*)(s.xse + s.G + 1);
    s.inv = (float*)(s.flag + 1);
    return s;
}

// The fused input transform of a job; all null for a plain matmul.
struct Fuse {
    const float* gate;     // gated activation input, or null
    const float* norm_w;   // RMSNorm gain, or null
    float eps;
    int flags;             // BRIK_JOB_GAIN_ONE_PLUS, BRIK_JOB_ACT_GELU
};

__device__ __forceinline__ float act(float v, int flags)
{
    if (flags & BRIK_JOB_ACT_GELU)          // tanh-approximated GELU, as the reference's geglu
        return 0.5f * v * (1.f + tanhf(0.7978845608f * (v + 0.044715f * v * v * v)));
    return v / (1.f + expf(-v));            // SiLU, as the reference's swiglu
}

// Element k of the transformed row given the RMSNorm factor inv (1 without a norm).
__device__ __forceinline__ float fused_in(const float* __restrict__ x, const Fuse& F, float inv, int k)
{
    float v = x[k];
    if (F.gate) v = act(F.gate[k], F.flags) * v;
    if (F.norm_w) v = v * inv * ((F.flags & BRIK_JOB_GAIN_ONE_PLUS) ? 1.f + F.norm_w[k] : F.norm_w[k]);
    return v;
}

__device__ __forceinline__ f32x4_t fused_in4(f32x4_t v, const Fuse& F, float inv, int k)
{
    if (F.gate) {
        const f32x4_t g = *(const f32x4_t*)(F.gate + k);
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = act(g[t], F.flags) * v[t];
    }
    if (F.norm_w) {
        f32x4_t w = *(const f32x4_t*)(F.norm_w + k);
        if (F.flags & BRIK_JOB_GAIN_ONE_PLUS) w = w + 1.f;
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = v[t] * inv * w[t];
    }
    return v;
}

__device__ __forceinline__ void split_limbs(float v, int sh, bool finite, int& h, int& m, int& l)
{
    const int X = finite ? (int)__builtin_rintf(ldexpf(v, sh)) : 0;
    l = (int)(int8_t)(X & 0xff);
    const int X1 = (X - l) >> 8;
    m = (int)(int8_t)(X1 & 0xff);
    h = (X1 - m) >> 8;
}

// Stage x[0..K) (16-byte aligned, K % 32 == 0). All threads of the block call it; ends with a barrier.
template <int FMT>
__device__ __forceinline__ void xstage(const float* __restrict__ x, const XStage& S, int K, const Fuse& F)
{
    const int G = S.G;
    if (threadIdx.x == 0) {
        *S.flag = 0;
        S.xse[G] = float2{0.f, 0.f};
    }
    if (threadIdx.x < 24) ((uint32_t*)(S.limbs + 96 * G))[threadIdx.x] = 0u;   // the zero group
    const int nq = K >> 2;
    float inv = 1.f;
    if (F.norm_w) {
        // sum of squares of the (gated) row: per thread, per wave, then across the block's waves
        float ss = 0.f;
        for (int i = threadIdx.x; i < nq; i += blockDim.x) {
            const f32x4_t v = fused_in4(*(const f32x4_t*)(x + 4 * i), Fuse{F.gate, nullptr, 0.f, F.flags}, 1.f, 4 * i);
            ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        }
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        if ((threadIdx.x & 63) == 0) S.inv[1 + (threadIdx.x >> 6)] = ss;
        __syncthreads();
        float t = 0.f;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += S.inv[1 + w];
        inv = 1.f / sqrtf(t / (float)K + F.eps);
    }
    if (threadIdx.x == 0) *S.inv = inv;
    __syncthreads();
    // the 8 float4 chunks of a group sit in 8 consecutive lanes (blockDim % 8 == 0, nq % 8 == 0);
    // every loop trip is entered by whole 8-lane groups, so the DPP group reductions see full groups
    for (int i = threadIdx.x; i < nq; i += blockDim.x) {
        const f32x4_t v = fused_in4(*(const f32x4_t*)(x + 4 * i), F, inv, 4 * i);
        const int g = i >> 3, c = i & 7;
        const float p = sum8((v.x + v.y) + (v.z + v.w));
        const float a = max8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        const bool finite = __builtin_isfinite(p) && __builtin_isfinite(a);
        int e = 0;
        (void)frexpf(a, &e);                 // a < 2^e, so |x * 2^(22-e)| < 2^22
        const int sh = 22 - e;
        if (c == 0) S.xse[g] = float2{p, __builtin_bit_cast(float, -sh)};
        if (!finite) *S.flag = 1;
        int hh[4], mm[4], ll[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) split_limbs(v[t], sh, finite, hh[t], mm[t], ll[t]);
        int8_t* base = S.limbs + 96 * g;
        const int hs = half_swap(g);
        if constexpr (FMT == FMT_Q8) {
            // elements 4c..4c+3 are byte dword c of every limb
            const int pos = (4 * c) ^ hs;
            auto pack = [](const int (&b)[4]) {
                return (uint32_t)(b[0] & 0xff) | ((uint32_t)(b[1] & 0xff) << 8) | ((uint32_t)(b[2] & 0xff) << 16) |
                       ((uint32_t)(b[3] & 0xff) << 24);
            };
            *(uint32_t*)(base + pos) = pack(hh);
            *(uint32_t*)(base + 32 + pos) = pack(mm);
            *(uint32_t*)(base + 64 + pos) = pack(ll);
        } else if constexpr (FMT == FMT_Q4) {
            // elements 4c..4c+3 give bytes (c&1)*2 and +1 of byte dwords 2j (even elements) and
            // 2j+1 (odd elements), j = c/2: two 16-bit stores per limb
            const int j = c >> 1, bo = (c & 1) * 2;
            const int pe = ((8 * j) + bo) ^ hs, po = ((8 * j + 4) + bo) ^ hs;
            auto st = [&](int8_t* lb, const int (&b)[4]) {
                *(uint16_t*)(lb + pe) = (uint16_t)((b[0] & 0xff) | ((b[2] & 0xff) << 8));
                *(uint16_t*)(lb + po) = (uint16_t)((b[1] & 0xff) | ((b[3] & 0xff) << 8));
            };
            st(base, hh);
            st(base + 32, mm);
            st(base + 64, ll);
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int pos = code_pos<FMT>(4 * c + t) ^ hs;
                base[pos] = (int8_t)hh[t];
                base[32 + pos] = (int8_t)mm[t];
                base[64 + pos] = (int8_t)ll[t];
            }
        }
    }
    __syncthreads();
}

}  // namespace brik
