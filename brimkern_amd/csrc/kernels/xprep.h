// Activation staging for the decode GEMV: one f32 row x[K] -> LDS as 24-bit block floating point.
//
// Per 32-element group g (the quantization group of the weights), with e_g the binary exponent of
// max|x| over the group (frexp), every element becomes the integer X = rint(x * 2^(22 - e_g)),
// |X| < 2^22, split into three signed bytes X = h * 65536 + m * 256 + l (h, m, l in [-128, 127]).
// The dot products with the integer weight codes then run on v_dot4_i32_i8 (four int8 MACs per lane
// per instruction, exact int32 sums), and the group's result is rescaled by 2^(e_g - 22) in f32.
// Relative to the group's largest element this keeps 22 bits, about f32's 24-bit significand.
// This byte-limb image serves q8 (int8 codes); q4 and q3 use the digit-plane image further below
// (the same X, written as six 4-bit digits for v_dot8_i32_i4).
//
// LDS layout for K = 32 * G, group-major so a group's limbs are reached with immediate offsets:
//   limbs: group g (0 <= g <= G) occupies bytes [96g, 96g + 96): limb t (0 = h, 1 = m, 2 = l) at
//          96g + 32t, its 32 bytes in element order (the order of the q8 code bytes),
//          the two 16-byte halves swapped when bit 3 of g is set (so lanes reading groups g and g + 8
//          in one instruction hit different banks). Group G is all zeros: consumers point groups past
//          the end of a row at it, which zeroes their contribution without a select;
//   xse[g]: {f32 sum of the group's x, int32 e_g - 22}, g <= G, xse[G] = {0, 0};
//   flag:  int32, nonzero if the row holds a non-finite value (the exact f32 path then runs);
//   inv:   f32, the RMSNorm factor of a fused input transform (1 without one), and 16 words of
//          scratch for its block reduction (one per wave; a plan's staging pass runs 16 waves).
//
// Fused input transform (grouped plans, brik_gemv_job_ex): the staged row may be
//   act(gate[k]) * x[k]                  (SwiGLU act = SiLU, GeGLU act = tanh-GELU), then / or
//   v[k] * inv * g[k],  inv = 1 / sqrt(sum v^2 / K + eps),  g = w or 1 + w   (RMSNorm)
// as the reference computes n1 = rmsnorm(x) and g = swiglu(gate, up) before recMM
// (src/lib/webgpu/shaders.ts:580-626; kernels.ts:1701, 1723, 1726). The image holds v[k] * g[k]; the
// scalar inv multiplies each row's result instead (stage_finish).
#pragma once
#include "common.h"
#include "../../../include/brik.h"   // BRIK_JOB_* flags

namespace brik {

__device__ __forceinline__ int half_swap(int g) { return ((g >> 3) & 1) << 4; }

struct XStage {
    int8_t* limbs;
    float2* xse;      // {sum, bit-cast int exponent}
    int* flag;
    float* inv;       // inv, then 16 reduction slots
    int G;
};

// Bytes after the groups: flag, RMSNorm factor, 16 reduction slots, padded to 16 bytes.
#define BRIK_XSTAGE_TAIL 80

// Bytes of the staged row; the block's partial-sum buffer follows at this offset (4-byte aligned).
__host__ __device__ __forceinline__ size_t xstage_bytes(int K)
{
    return (size_t)104 * (K / BRIK_GROUP + 1) + BRIK_XSTAGE_TAIL;
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

// SiLU v / (1 + e^-v), as the reference's swiglu; with BRIK_JOB_ACT_GELU its tanh-GELU
// 0.5 v (1 + tanh u), u = 0.7978845608 (v + 0.044715 v^3), written as v / (1 + e^(-2u)) (the same
// function: 0.5 (1 + tanh u) = 1 / (1 + e^(-2u))). The exponential is v_exp_f32 of the argument times
// log2(e) and the quotient one v_rcp_f32 (about 1 ulp each; for |v| <= 10 the result is within ~1e-6
// relative) instead of libm's expf / tanhf and an IEEE divide: a handful of instructions per element
// instead of ~30 matters because every block of a fused launch transforms the whole row, on one wave
// per SIMD. Limits match the reference's: v -> -inf gives -0, v -> +inf gives v, NaN stays NaN, and
// v = -inf gives NaN (-inf / inf).
__device__ __forceinline__ float act(float v, int flags)
{
    const float t = (flags & BRIK_JOB_ACT_GELU) ? -1.5957691216f * (v + 0.044715f * v * v * v) : -v;
    return v * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(t * 1.4426950409f));
}

// Element k of the transformed row given the RMSNorm factor inv (1 without a norm).
__device__ __forceinline__ float fused_in(const float* __restrict__ x, const Fuse& F, float inv, int k)
{
    float v = x[k];
    if (F.gate) v = act(F.gate[k], F.flags) * v;
    if (F.norm_w) v = v * inv * ((F.flags & BRIK_JOB_GAIN_ONE_PLUS) ? 1.f + F.norm_w[k] : F.norm_w[k]);
    return v;
}

// The loads behind C consecutive float4 chunks of the transformed row: x, and the gate and RMSNorm
// gain where the fusion uses them (the others stay unset).
template <int C>
struct RawIn {
    f32x4_t x[C], g[C], w[C];
};

// Buffer resources over the inputs of a staging pass (x, gate, RMSNorm gain: `bytes` each), built from
// laundered pointers (launder_uniform) so that the loads keep their place in program order:
// batched_in's hook relies on the x loads going out first.
struct InRs {
    brsrc_t x, g, w;
};

__device__ __forceinline__ InRs in_rsrc(const float* __restrict__ x, const Fuse& F, uint32_t bytes)
{
    const float* xl = launder_uniform(x);
    return InRs{make_rsrc(xl, bytes), make_rsrc(F.gate ? launder_uniform(F.gate) : xl, F.gate ? bytes : 0u),
                make_rsrc(F.norm_w ? launder_uniform(F.norm_w) : xl, F.norm_w ? bytes : 0u)};
}

__device__ __forceinline__ f32x4_t ld_f4(const brsrc_t& r, int k)
{
    return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)k * 4u, 0u, 0));
}

template <int C>
__device__ __forceinline__ void load_in(RawIn<C>& r, const InRs& R, const Fuse& F, int k)
{
#pragma unroll
    for (int c = 0; c < C; ++c) r.x[c] = ld_f4(R.x, k + 4 * c);
    if (F.gate) {
#pragma unroll
        for (int c = 0; c < C; ++c) r.g[c] = ld_f4(R.g, k + 4 * c);
    }
    if (F.norm_w) {
#pragma unroll
        for (int c = 0; c < C; ++c) r.w[c] = ld_f4(R.w, k + 4 * c);
    }
}

// Chunk c of the gated row act(gate) * x from its loads (x itself without a gate).
template <int C>
__device__ __forceinline__ f32x4_t apply_in(const RawIn<C>& r, int c, const Fuse& F)
{
    f32x4_t v = r.x[c];
    if (F.gate) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = act(r.g[c][t], F.flags) * v[t];
    }
    return v;
}

// v times the RMSNorm gain of chunk c (w, or 1 + w).
template <int C>
__device__ __forceinline__ f32x4_t gain_in(const RawIn<C>& r, int c, const Fuse& F, f32x4_t v)
{
    f32x4_t w = r.w[c];
    if (F.flags & BRIK_JOB_GAIN_ONE_PLUS) w = w + 1.f;
    return v * w;
}

__device__ __forceinline__ float sumsq4(f32x4_t v) { return (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w); }

// A staging call's hook for other loads (none by default).
struct NoLoads {
    __device__ __forceinline__ void operator()() const {}
};

// body(i, loads) for i = threadIdx.x, + NT, ... < n over chunks of 4C floats, in that order (NT: the
// block's threads, a compile-time constant: blockDim.x can cost a memory round trip to read).
// The loads of SB consecutive trips are issued together before any is used, so a thread pays one
// memory round trip per SB trips instead of one per trip (a K = 9728 row takes five trips of a
// 256-thread block). Indices past n are clamped for the loads, which then stay in range, and their
// trips run no body. Whole aligned lane groups enter each body together when n and NT are
// multiples of the group size, as the DPP group reductions need.
// after_first() runs once, right after the first batch's loads are issued (every thread calls it):
// the GEMV issues its first weight loads there. Vector-memory loads complete in issue order, so the
// first batch's bodies then wait for x only, with the weights still in flight behind it; issued
// before x, the weights would have to arrive before staging could start.
template <int SB, int C, int NT, class Body, class After = NoLoads>
__device__ __forceinline__ void batched_in(const float* __restrict__ x, const Fuse& F, int n, Body body,
                                           After after_first = After())
{
    constexpr int bd = NT;
    const int tid = (int)threadIdx.x;
    const InRs R = in_rsrc(x, F, (uint32_t)n * 16u * C);
    auto load = [&](RawIn<C> (&r)[SB], int b) {
#pragma unroll
        for (int u = 0; u < SB; ++u) {
            const int i = min(b + u * bd + tid, n - 1);
            load_in<C>(r[u], R, F, 4 * C * i);
        }
    };
    auto run = [&](const RawIn<C> (&r)[SB], int b) {
#pragma unroll
        for (int u = 0; u < SB; ++u) {
            if (b + u * bd >= n) break;           // the same for every thread of the block
            const int i = b + u * bd + tid;
            if (i < n) body(i, r[u]);
        }
    };
    // The first batch is straight-line code (n > 0 always: K >= 32), so the compiler's wait before its
    // bodies counts the hook's loads as still in flight; inside the loop under a condition, the
    // branch-merged count had it wait for them.
    {
        RawIn<C> r[SB];
        load(r, 0);
        // keep the order: x loads, then the hook's loads (the empty asm orders memory operations in the
        // compiler's IR, the scheduling barrier in the machine scheduler)
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        after_first();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        run(r, 0);
    }
    for (int b = SB * bd; b < n; b += SB * bd) {
        RawIn<C> r[SB];
        load(r, b);
        run(r, b);
    }
}

// RMSNorm in staging: the factor inv = 1 / sqrt(sum v^2 / K + eps) (v the gated row) is one scalar
// per row, and a row's result is linear in its input (sum X q and the min term sum x alike), so the
// image holds v * gain without inv and the row's result is multiplied by inv afterwards. One pass over
// x then yields both the image and the sum of squares.
//
// End of a staging pass: the flag (nonzero if any thread saw a non-finite value, `bad`) and inv from
// the threads' partial sums of squares `ss` (1 without a norm). A zero, infinite or NaN factor raises
// the flag too: the exact path applies it per element, as the reference does. thread 0 wrote flag = 0
// before the pass; the 1s are written after the first barrier, so they cannot race it. Ends with a
// barrier after which flag and inv hold their final values.
template <int NT>
__device__ __forceinline__ void stage_finish(int* flag, float* inv, const Fuse& F, int K, float ss, int bad)
{
    if (F.norm_w) {
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        if ((threadIdx.x & 63) == 0) inv[1 + (threadIdx.x >> 6)] = ss;
    }
    const bool wave_bad = __any(bad);
    __syncthreads();
    if (wave_bad && (threadIdx.x & 63) == 0) *flag = 1;
    if (threadIdx.x == 0) {
        float f = 1.f;
        if (F.norm_w) {
            float t = 0.f;
            for (int w = 0; w < NT / 64; ++w) t += inv[1 + w];
            f = 1.f / sqrtf(t / (float)K + F.eps);
            if (!(f > 0.f && f < __builtin_inff())) *flag = 1;
        }
        *inv = f;
    }
    __syncthreads();
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
// SB: loop trips whose loads a thread issues together (batched_in); more trips hold more registers.
template <int FMT, int SB, int NT, class After = NoLoads>
__device__ __forceinline__ void xstage(const float* __restrict__ x, const XStage& S, int K, const Fuse& F,
                                       After after_first = After())
{
    static_assert(FMT == FMT_Q8, "q4 and q3 stage digit planes (xstage_d)");
    const int G = S.G;
    if (threadIdx.x == 0) {
        *S.flag = 0;
        S.xse[G] = float2{0.f, 0.f};
    }
    if (threadIdx.x < 24) ((uint32_t*)(S.limbs + 96 * G))[threadIdx.x] = 0u;   // the zero group
    const int nq = K >> 2;
    float ss = 0.f;
    int bad = 0;
    // the 8 float4 chunks of a group sit in 8 consecutive lanes (NT % 8 == 0, nq % 8 == 0);
    // every body is entered by whole 8-lane groups, so the DPP group reductions see full groups
    batched_in<SB, 1, NT>(x, F, nq, [&](int i, const RawIn<1>& r) {
        f32x4_t v = apply_in<1>(r, 0, F);
        if (F.norm_w) {
            ss += sumsq4(v);
            v = gain_in<1>(r, 0, F, v);
        }
        const int g = i >> 3, c = i & 7;
        const float p = sum8((v.x + v.y) + (v.z + v.w));
        const float a = max8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        const bool finite = __builtin_isfinite(p) && __builtin_isfinite(a);
        int e = 0;
        (void)frexpf(a, &e);                 // a < 2^e, so |x * 2^(22-e)| < 2^22
        const int sh = 22 - e;
        if (c == 0) S.xse[g] = float2{p, __builtin_bit_cast(float, -sh)};
        bad |= !finite;
        int hh[4], mm[4], ll[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) split_limbs(v[t], sh, finite, hh[t], mm[t], ll[t]);
        int8_t* base = S.limbs + 96 * g;
        const int hs = half_swap(g);
        // elements 4c..4c+3 are byte dword c of every limb
        const int pos = (4 * c) ^ hs;
        auto pack = [](const int (&b)[4]) {
            return (uint32_t)(b[0] & 0xff) | ((uint32_t)(b[1] & 0xff) << 8) | ((uint32_t)(b[2] & 0xff) << 16) |
                   ((uint32_t)(b[3] & 0xff) << 24);
        };
        *(uint32_t*)(base + pos) = pack(hh);
        *(uint32_t*)(base + 32 + pos) = pack(mm);
        *(uint32_t*)(base + 64 + pos) = pack(ll);
    }, after_first);
    stage_finish<NT>(S.flag, S.inv, F, K, ss, bad);
}

// ---- q4: x as six signed 4-bit digit planes ---------------------------------------------------
// The q4 GEMV multiplies x with the nibble codes directly on v_dot8_i32_i4 (eight 4-bit MACs per
// instruction), so no code is ever unpacked. x is staged with the same per-group scaling as above,
// X = rint(x * 2^(22 - e_g)), |X| < 2^22, written as six balanced base-16 digits
//   X = sum_n d_n 16^n, d_n in [-8, 7].
// (X + 0x888888) holds the digits offset by 8 in its six nibbles, so XOR 0x888888 of it leaves each
// d_n as a signed nibble: two instructions per element. Digit plane n of a group is 16 bytes, eight
// nibbles per dword, in the element order of the format's code nibbles (digit_elem):
//   q4: nibble i of dword j is element 8j + i, the order of the q4 codes themselves (element 2i is the
//       low nibble of byte i). The codes enter the dot products as signed nibbles q - 8 (XOR 0x8 per
//       nibble); the group term is sum X q = sum_n 16^n (d_n . (q - 8)) + 8 sum X, every step an exact
//       int32 (|sum X q| < 15 * 2^27).
//   q3: nibble i of dword j is element 16 (j >> 1) + 2i + (j & 1): the order in which the 2-bit plane's
//       fields fall into nibbles when a lo word is masked with 0x33333333 (even elements) or shifted
//       right by 2 first (odd elements); the hi bit of each is inserted at bit 2 of its nibble (gemv.hip).
//       The codes 0..7 are nonnegative signed nibbles as they are: sum X q = sum_n 16^n (d_n . q)
//       (|sum X q| < 7 * 2^27).
//
// LDS layout, group-major so every read uses an immediate offset: group g (0 <= g <= G) occupies
// bytes [112g, 112g + 112): digit plane n at 112g + 16n (n < 6), then {f32 sum of the group's x,
// int32 e_g - 22, int32 8 * sum X, int32 1 if the group holds a value that is not finite, else 0} at
// 112g + 96. Group G is all zeros (the zero group). A team's
// lanes read consecutive groups 112 bytes apart, which spreads any 8 of them over distinct banks.
// Then the flag, the RMSNorm factor and its reduction slots as in the byte-limb layout.
struct XStageD {
    unsigned char* base;
    int* flag;
    float* inv;
    int G;
};

__host__ __device__ __forceinline__ size_t xstage_d_bytes(int K)
{
    return (size_t)112 * (K / BRIK_GROUP + 1) + BRIK_XSTAGE_TAIL;
}

__device__ __forceinline__ XStageD xstage_d_layout(void* lds, int K)
{
    XStageD s;
    s.G = K / BRIK_GROUP;
    s.base = (unsigned char*)lds;
    s.flag = (int*)(s.base + (size_t)112 * (s.G + 1));
    s.inv = (float*)(s.flag + 1);
    return s;
}

// max / sum over aligned groups of 4 lanes (one quantization group: 4 lanes x 8 elements)
__device__ __forceinline__ float max4(float v)
{
    v = BRIK_DPP_MAX(v, DPP_QUAD_1032);
    return BRIK_DPP_MAX(v, DPP_QUAD_2301);
}
__device__ __forceinline__ float sum4(float v)
{
    v = BRIK_DPP_ADD(v, DPP_QUAD_1032);
    return BRIK_DPP_ADD(v, DPP_QUAD_2301);
}
__device__ __forceinline__ int sum4i(int v)
{
    v += __builtin_amdgcn_mov_dpp(v, DPP_QUAD_1032, 0xF, 0xF, false);
    return v + __builtin_amdgcn_mov_dpp(v, DPP_QUAD_2301, 0xF, 0xF, false);
}

// Transpose 8 x 8 nibbles: out[n] nibble i = in[i] nibble n (three stages: 16-bit halves between
// words 4 apart, bytes between words 2 apart, nibbles between neighbours).
__device__ __forceinline__ void nibble_transpose8(const uint32_t (&a)[8], uint32_t (&w)[8])
{
    uint32_t t[8], u[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        t[i] = __builtin_amdgcn_perm(a[i + 4], a[i], 0x05040100u);       // a_i.h0  a_{i+4}.h0
        t[i + 4] = __builtin_amdgcn_perm(a[i + 4], a[i], 0x07060302u);   // a_i.h1  a_{i+4}.h1
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = q < 2 ? q : q + 2;
        u[i] = __builtin_amdgcn_perm(t[i + 2], t[i], 0x06020400u);       // t_i.b0 t_{i+2}.b0 t_i.b2 t_{i+2}.b2
        u[i + 2] = __builtin_amdgcn_perm(t[i + 2], t[i], 0x07030501u);   // t_i.b1 t_{i+2}.b1 t_i.b3 t_{i+2}.b3
    }
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        w[i] = (u[i] & 0x0F0F0F0Fu) | ((u[i + 1] << 4) & 0xF0F0F0F0u);
        w[i + 1] = ((u[i] >> 4) & 0x0F0F0F0Fu) | (u[i + 1] & 0xF0F0F0F0u);
    }
}

// Element of a group at nibble i of digit-plane dword j (see above).
template <int FMT>
__host__ __device__ __forceinline__ int digit_elem(int j, int i)
{
    return FMT == FMT_Q3 ? 16 * (j >> 1) + 2 * i + (j & 1) : 8 * j + i;
}

// One group's digit planes from its 32 values: the thread at quad position j (lane & 3) holds elements
// 8j .. 8j+7 in v0, v1; all four lanes of an aligned quad call it together (the group's sum, max and
// sum X are DPP quad reductions). gb: the group's 112 bytes (LDS, or a staged image in global memory).
// Writes the planes and {sum x, e - 22, 8 sum X, 1 if a value is not finite else 0}; returns
// whether the values are all finite (the planes of a group that is not are all zeros).
template <int FMT>
__device__ __forceinline__ bool stage_group_d(f32x4_t v0, f32x4_t v1, int j, unsigned char* gb)
{
    // The sums below start from the values as rounded: with -ffp-contract=fast the compiler could
    // otherwise fold a caller's product (act(gate) * up, v * gain) into them as an FMA, and decide
    // that differently in each kernel that inlines this one, while a GLU pair launch must write the
    // image its consumer would stage itself.
    asm volatile("" : "+v"(v0), "+v"(v1));
    const float p = sum4(((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w)));
    const float a = max4(fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                               fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w)))));
    const bool finite = __builtin_isfinite(p) && __builtin_isfinite(a);
    int e = 0;
    (void)frexpf(a, &e);                 // a < 2^e, so |x * 2^(22-e)| < 2^22
    const int sh = 22 - e;
    uint32_t dg[8];
    int sx = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int X = finite ? (int)__builtin_rintf(ldexpf(t < 4 ? v0[t] : v1[t - 4], sh)) : 0;
        sx += X;
        dg[t] = (uint32_t)(X + 0x888888) ^ 0x888888u;   // digit n of X in nibble n, as a signed nibble
    }
    sx = sum4i(sx);
    uint32_t w[8];
    if constexpr (FMT == FMT_Q3) {
        // thread j holds elements 8j .. 8j+7: the even ones are nibbles 4(j&1) .. +3 of dword 2(j>>1),
        // the odd ones the same nibbles of dword 2(j>>1)+1; transposed in the order 0 2 4 6 1 3 5 7
        // every digit plane word splits into those two 16-bit halves
        const uint32_t eo[8] = {dg[0], dg[2], dg[4], dg[6], dg[1], dg[3], dg[5], dg[7]};
        nibble_transpose8(eo, w);
        const int de = 8 * (j >> 1) + 2 * (j & 1), dodd = de + 4;   // byte offsets in a plane
#pragma unroll
        for (int n = 0; n < 6; ++n) {
            *(uint16_t*)(gb + 16 * n + de) = (uint16_t)w[n];
            *(uint16_t*)(gb + 16 * n + dodd) = (uint16_t)(w[n] >> 16);
        }
    } else {
        nibble_transpose8(dg, w);
#pragma unroll
        for (int n = 0; n < 6; ++n) *(uint32_t*)(gb + 16 * n + 4 * j) = w[n];
    }
    if (j == 0) *(i32x4_t*)(gb + 96) = i32x4_t{__builtin_bit_cast(int, p), -sh, sx * 8, finite ? 0 : 1};
    return finite;
}

// Stage x[0..K) (16-byte aligned, K % 32 == 0) as digit planes: one thread per 8 consecutive elements,
// a quad of lanes per group. All threads of the block call it; ends with a barrier. after_first: as in
// batched_in.
template <int FMT, int SB, int NT, class After = NoLoads>
__device__ __forceinline__ void xstage_d(const float* __restrict__ x, const XStageD& S, int K, const Fuse& F,
                                         After after_first = After())
{
    const int G = S.G;
    if (threadIdx.x == 0) *S.flag = 0;
    if (threadIdx.x < 7) *(u32x4_t*)(S.base + 112 * G + 16 * threadIdx.x) = u32x4_t{0u, 0u, 0u, 0u};
    float ss = 0.f;
    int bad = 0;
    // every body is entered by whole quads (NT % 4 == 0, K/8 % 4 == 0), so the DPP group
    // reductions see full groups
    const int n8 = K >> 3;
    batched_in<(SB > 1 ? SB - 1 : 1), 2, NT>(x, F, n8, [&](int i, const RawIn<2>& r) {
        f32x4_t v0 = apply_in<2>(r, 0, F), v1 = apply_in<2>(r, 1, F);
        if (F.norm_w) {
            ss += sumsq4(v0) + sumsq4(v1);
            v0 = gain_in<2>(r, 0, F, v0);
            v1 = gain_in<2>(r, 1, F, v1);
        }
        bad |= !stage_group_d<FMT>(v0, v1, i & 3, S.base + 112 * (i >> 2));
    }, after_first);
    stage_finish<NT>(S.flag, S.inv, F, K, ss, bad);
}

// Groups [g0, G) of an input row for a block whose LDS already receives groups [0, g0) from a
// producer's image (a GLU pair launch that wrote only those): `src` holds the row's values from
// element 32 g0 on, as the producer wrote them (act(gate) * up, rounded), and they are staged by the
// same group code as xstage_d's, with the zero group after them. The flag is set to -1 (the caller
// then reads every group's own non-finite marker) and the RMSNorm factor to 1: such an input has no
// RMSNorm. No barrier: the caller's follows. after_first: as in batched_in.
template <int FMT, int SB, int NT, class After = NoLoads>
__device__ __forceinline__ void xstage_d_tail(const float* __restrict__ src, const XStageD& S, int g0,
                                              After after_first = After())
{
    const int G = S.G;
    if (threadIdx.x == 0) {
        *S.flag = -1;
        *S.inv = 1.f;
    }
    if (threadIdx.x < 7) *(u32x4_t*)(S.base + 112 * G + 16 * threadIdx.x) = u32x4_t{0u, 0u, 0u, 0u};
    const Fuse none{nullptr, nullptr, 0.f, 0};
    batched_in<(SB > 1 ? SB - 1 : 1), 2, NT>(src, none, 4 * (G - g0), [&](int i, const RawIn<2>& r) {
        (void)stage_group_d<FMT>(r.x[0], r.x[1], i & 3, S.base + 112 * (g0 + (i >> 2)));
    }, after_first);
}

// The same group image from lanes 0-31 of one wave (all active), lane e holding element e: for a
// producer that writes a single group at the end of its block, with the group reductions as DPP steps
// and two lane reads instead of the 8-element-per-lane work of stage_group_d. Every value is
// bit-identical to stage_group_d's: the group sum follows the same tree, ((e0 + e1) + (e2 + e3)) +
// ((e4 + e5) + (e6 + e7)) within each 8, then (c0 + c1) + (c2 + c3) (each exchange meets an add's
// operands in one order or the other, and an IEEE sum is commutative); max and the integer sums are
// exact in any order.
template <int FMT>
__device__ __forceinline__ void stage_group_lanes(float v, unsigned char* gb)
{
    asm volatile("" : "+v"(v));   // as in stage_group_d
    const int e = (int)(threadIdx.x & 63);
    float p = sum8(v);                                   // c_j in the 8 lanes of chunk j
    p = BRIK_DPP_ADD(p, DPP_ROW_ROR8);                   // c0 + c1 in lanes 0-15, c2 + c3 in 16-31
    p = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), 0)) +
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), 16));
    float a = max8(fabsf(v));
    a = BRIK_DPP_MAX(a, DPP_ROW_ROR8);
    a = fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 0)),
              __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 16)));
    const bool finite = __builtin_isfinite(p) && __builtin_isfinite(a);
    int ex = 0;
    (void)frexpf(a, &ex);
    const int sh = 22 - ex;
    const int X = finite ? (int)__builtin_rintf(ldexpf(v, sh)) : 0;
    int sx = X;
    sx += __builtin_amdgcn_mov_dpp(sx, DPP_QUAD_1032, 0xF, 0xF, false);
    sx += __builtin_amdgcn_mov_dpp(sx, DPP_QUAD_2301, 0xF, 0xF, false);
    sx += __builtin_amdgcn_mov_dpp(sx, DPP_ROW_HALF_MIRROR, 0xF, 0xF, false);
    sx += __builtin_amdgcn_mov_dpp(sx, DPP_ROW_ROR8, 0xF, 0xF, false);
    sx = __builtin_amdgcn_readlane(sx, 0) + __builtin_amdgcn_readlane(sx, 16);
    const uint32_t dg = (uint32_t)(X + 0x888888) ^ 0x888888u;
    // nibble i of plane dword j holds element digit_elem(j, i): q4 j = e >> 3, i = e & 7 (the 8 lanes of
    // a dword are adjacent); q3 j = 2 (e >> 4) + (e & 1), i = (e & 15) >> 1 (the lanes of one parity in
    // a 16-lane row)
    const int sl = FMT == FMT_Q3 ? 4 * ((e & 15) >> 1) : 4 * (e & 7);
    const bool writer = FMT == FMT_Q3 ? (e & 14) == 0 : (e & 7) == 0;
    const int dw = FMT == FMT_Q3 ? 2 * (e >> 4) + (e & 1) : e >> 3;
#pragma unroll
    for (int n = 0; n < 6; ++n) {
        uint32_t w = ((dg >> (4 * n)) & 0xFu) << sl;
        if constexpr (FMT == FMT_Q3) {
            w |= __builtin_amdgcn_mov_dpp(w, 0x122, 0xF, 0xF, false);    // row_ror:2
            w |= __builtin_amdgcn_mov_dpp(w, DPP_ROW_ROR4, 0xF, 0xF, false);
            w |= __builtin_amdgcn_mov_dpp(w, DPP_ROW_ROR8, 0xF, 0xF, false);
        } else {
            w |= __builtin_amdgcn_mov_dpp(w, DPP_QUAD_1032, 0xF, 0xF, false);
            w |= __builtin_amdgcn_mov_dpp(w, DPP_QUAD_2301, 0xF, 0xF, false);
            w |= __builtin_amdgcn_mov_dpp(w, DPP_ROW_HALF_MIRROR, 0xF, 0xF, false);
        }
        if (writer) *(uint32_t*)(gb + 16 * n + 4 * dw) = w;
    }
    if (e == 0) *(i32x4_t*)(gb + 96) = i32x4_t{__builtin_bit_cast(int, p), -sh, sx * 8, finite ? 0 : 1};
}

// Whether any of the G groups of a digit-plane image holds a value that is not finite (the marker
// stage_group_d writes). Called by every thread of the block after the image is in LDS; the
// block-wide OR ends with a barrier.
template <int NT>
__device__ __forceinline__ int image_bad(const XStageD& S)
{
    int bad = 0;
    for (int g = (int)threadIdx.x; g < S.G; g += NT) bad |= *(const int*)(S.base + 112 * g + 108);
    return __syncthreads_or(bad);
}

}  // namespace brik
