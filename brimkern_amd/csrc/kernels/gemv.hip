// Decode GEMV: y[m, :] = x[m, :] . deq(W)^T for one activation row per grid.y, streaming the packed
// .brik planes once. Replaces the reference's 1-row WGSL kernels matmul_t_q8 / _q4 / _q3
// (src/lib/webgpu/shaders.ts:376-418, 77-114, 323-369), which give each output to one thread and
// walk its weight row serially with 32-bit loads.
//
// Arithmetic. The group scale factors out of the dot product:
//   y_n = sum_g [ s_ng * sum_{k in g} x_k q_nk + m_ng * sum_{k in g} x_k ].
// x is staged once per block as 24-bit block floating point (xprep.h), so sum x_k q_nk is an exact
// int32 dot product, rescaled once per group: for q8 of int8 limbs with the int8 codes as loaded
// (v_dot4_i32_i8); for q4 and q3 of signed 4-bit digits with the codes as signed nibbles
// (v_dot8_i32_i4): the q4 nibbles as loaded, the q3 ones assembled from its 2-bit and 1-bit planes.
// A one-hot x reproduces deq(W) bit-exactly: the single product s*q*2^21 and its rescale are exact
// and the final fmaf(m, 1, s*q) rounds q*s + m once, as the reference's dequantize does.
//
// Mapping (wave64, 256-thread blocks):
//   * a team of TEAM lanes (16, 32 or 64) owns R adjacent weight rows; lane l handles groups
//     g = l, l + TEAM, ... so one step of a team loads U * TEAM consecutive groups per row: for q4,
//     U x TEAM x 16 contiguous bytes, one 128-bit load per lane per group. With U * TEAM = K / 32 a
//     step is whole rows, and the block streams one contiguous stretch of the code plane per step,
//     the pattern HBM serves fastest;
//   * each lane reads a group's x limbs from LDS once and applies them to its R rows;
//   * software pipeline: a lane's work is a sequence of steps of U groups x R rows; the loads of
//     step i + D - 1 are issued before step i is consumed, and the first D - 1 steps' loads right after
//     the loads of x, so staging x overlaps their latency;
//   * each lane stores its running partial sum of a row to LDS every step (branch-free loop body); after
//     the loop, the TEAM partials of a row are loaded by TEAM lanes at once and added with DPP steps
//     within 16-lane rows and lane exchanges across rows (row_sums), and the row's first lane writes y.
#include "common.h"
#include "xprep.h"
#include "stage_abi.h"
#include "../../../include/brik.h"   // brik_gemv_job

namespace {

using brik::XStage;
using brik::Fuse;

// Raw data of one (row, group) as loaded from the planes.
template <int FMT> struct Grp;
// Scale and min stay raw 16-bit values (v_cvt_f32_f16 reads the low half of the register), so no
// zero-extension consumes a load before the step that uses it.
template <> struct Grp<FMT_Q4> { u32x4_t w; uint16_t s, m; };
template <> struct Grp<FMT_Q8> { u32x4_t w0, w1; uint16_t s; };
template <> struct Grp<FMT_Q3> { u32x2_t l; uint32_t h; uint16_t s, m; };

// Vector-memory load instructions load_grp issues per (row, group).
template <int FMT> struct LoadsPerGroup { static constexpr int v = FMT == FMT_Q3 ? 4 : 3; };

// Bytes per group in the code plane (p0).
template <int FMT> struct CodeBytes { static constexpr int v = FMT == FMT_Q4 ? 16 : FMT == FMT_Q8 ? 32 : 8; };

struct Planes {
    const uint8_t* p0;
    const uint8_t* p1;
    const uint16_t* sc;
    const uint16_t* mn;
};

// Buffer resources over the planes of an N x K matrix (G groups per row).
struct Rs {
    brsrc_t code, hi, sc, mn;
};

template <int FMT>
__device__ __forceinline__ Rs make_rs(const Planes& P, int N, int G)
{
    const uint32_t groups = (uint32_t)N * (uint32_t)G;
    Rs r;
    r.code = make_rsrc(P.p0, groups * CodeBytes<FMT>::v);
    r.hi = make_rsrc(FMT == FMT_Q3 ? (const void*)P.p1 : (const void*)P.p0, FMT == FMT_Q3 ? groups * 4 : 0);
    r.sc = make_rsrc(P.sc, groups * 2);
    r.mn = make_rsrc(FMT == FMT_Q8 ? (const void*)P.sc : (const void*)P.mn, FMT == FMT_Q8 ? 0 : groups * 2);
    return r;
}

// Load group (gi + goff) where gi is per lane (VGPR) and goff = step offset (uniform) + gconst.
template <int FMT>
__device__ __forceinline__ void load_grp(Grp<FMT>& d, const Rs& rs, uint32_t gi, uint32_t gstep, uint32_t gconst)
{
    constexpr int CB = CodeBytes<FMT>::v;
    if constexpr (FMT == FMT_Q4) {
        d.w = __builtin_amdgcn_raw_buffer_load_b128(rs.code, (gi + gconst) * CB, gstep * CB, BRIK_AUX_STREAM);
        d.m = __builtin_amdgcn_raw_buffer_load_b16(rs.mn, (gi + gconst) * 2, gstep * 2, 0);
    } else if constexpr (FMT == FMT_Q8) {
        d.w0 = __builtin_amdgcn_raw_buffer_load_b128(rs.code, (gi + gconst) * CB, gstep * CB, BRIK_AUX_STREAM);
        d.w1 = __builtin_amdgcn_raw_buffer_load_b128(rs.code, (gi + gconst) * CB + 16, gstep * CB, BRIK_AUX_STREAM);
    } else {
        d.l = __builtin_amdgcn_raw_buffer_load_b64(rs.code, (gi + gconst) * CB, gstep * CB, BRIK_AUX_STREAM);
        d.h = __builtin_amdgcn_raw_buffer_load_b32(rs.hi, (gi + gconst) * 4, gstep * 4, BRIK_AUX_STREAM);
        d.m = __builtin_amdgcn_raw_buffer_load_b16(rs.mn, (gi + gconst) * 2, gstep * 2, 0);
    }
    d.s = __builtin_amdgcn_raw_buffer_load_b16(rs.sc, (gi + gconst) * 2, gstep * 2, 0);
}

// The group's 32 q8 codes as 8 dwords of bytes, in element order (the staged limbs' order).
template <int FMT>
__device__ __forceinline__ void unpack(const Grp<FMT>& d, uint32_t (&b)[8])
{
    static_assert(FMT == FMT_Q8, "q4 and q3 run on code nibbles (code_nibbles)");
#pragma unroll
    for (int j = 0; j < 4; ++j) { b[j] = d.w0[j]; b[4 + j] = d.w1[j]; }
}

// sum_{k in g} x_k q_k * 2^-(e_g - 22) as exact int32 limb dot products, combined in f32.
__device__ __forceinline__ float limb_dot(const uint32_t (&b)[8], const u32x4_t (&xl)[3][2])
{
    int a[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        int v = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) v = __builtin_amdgcn_sdot4((int)b[j], (int)xl[t][0][j], v, false);
#pragma unroll
        for (int j = 0; j < 4; ++j) v = __builtin_amdgcn_sdot4((int)b[4 + j], (int)xl[t][1][j], v, false);
        a[t] = v;
    }
    const int hm = (a[0] << 8) + a[1];                   // |a0| <= 2^19, so no int32 overflow
    return __builtin_fmaf((float)hm, 256.f, (float)a[2]);
}

// acc += s * sum(x q) + m * sum(x) for one (row, group). A group past the end of the row reads the
// zero group of the staged x, so both terms vanish without a select.
template <int FMT>
__device__ __forceinline__ float use_grp(const Grp<FMT>& d, const u32x4_t (&xl)[3][2], float2 xse, float acc)
{
    uint32_t b[8];
    unpack<FMT>(d, b);
    const float p = ldexpf(limb_dot(b, xl), __builtin_bit_cast(int, xse.y));   // exact rescale
    acc = __builtin_fmaf(f16_bits_to_f32(d.s), p, acc);
    if constexpr (FMT != FMT_Q8) acc = __builtin_fmaf(f16_bits_to_f32(d.m), xse.x, acc);
    return acc;
}

// Exact f32 fallback for a row holding Inf/NaN: per-element dequant, f32 FMA.
template <int FMT>
__device__ __forceinline__ float deq_elem(const Planes& P, size_t e)
{
    const size_t fg = e / BRIK_GROUP;
    const float s = f16_bits_to_f32(P.sc[fg]);
    if constexpr (FMT == FMT_Q8) {
        return (float)(int8_t)P.p0[e] * s;
    } else {
        uint32_t q;
        if constexpr (FMT == FMT_Q4) {
            q = (P.p0[e >> 1] >> (4 * (e & 1))) & 15u;
        } else {
            const uint32_t lw = ((const uint32_t*)P.p0)[e >> 4], hw = ((const uint32_t*)P.p1)[e >> 5];
            q = ((lw >> ((e & 15) * 2)) & 3u) | (((hw >> (e & 31)) & 1u) << 2);
        }
        return __builtin_fmaf((float)q, s, f16_bits_to_f32(P.mn[fg]));
    }
}

template <int TEAM>
__device__ __forceinline__ float team_sum(float v)
{
    v = sum16(v);
    if constexpr (TEAM >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (TEAM >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Per-team schedule over one matrix. The block owns row sets p = 0 .. nsets-1; team t computes rows
// n0(p) + [0, R) with n0(p) = r0 + t * R + p * rstep. A row set takes B steps; step b covers groups
// lane + TEAM * (U*b + u), u < U. The S = nsets * B steps of a team run as one software pipeline of
// depth D: the loads of step i + D - 1 are issued before step i is consumed.
//
// The pipelined loop body is straight-line code (no branches), which is what lets the compiler keep
// the loads of the steps ahead in flight (s_waitcnt vmcnt(N) rather than vmcnt(0)): step indices
// advance by scalar selects, rows past r1 and groups past G are clamped for loading and masked for
// accumulation, and each lane stores its running partial sums to LDS every step (the value after a
// row set's last step is the lane's final partial). The cross-lane sums and the y writes happen
// once, after the loop.
// Loop trips of the in-block x staging whose loads a thread issues together (xprep.h batched_in).
// The whole-row two-row variant keeps one: its blocks hold the most weight registers, and the launches
// it serves (large plans, large single matrices) copy a pre-staged image instead; for the others the
// extra registers cost no occupancy that their launches (at most a few blocks per CU) use.
constexpr int stage_trips(int R, int U) { return U >= 5 && R >= 2 ? 1 : 4; }

template <int FMT, int TEAM, int R, int U>
struct Work {
    static constexpr int NT = 256;                 // threads per block
    static constexpr int RPI = (NT / TEAM) * R;    // rows per block iteration
    static constexpr int PARTS = TEAM;             // partial sums per row
    static constexpr int NACC = R;                 // accumulators per lane
    static constexpr int UG = U;                   // groups per lane per step
    typedef Grp<FMT> Data[U][R];                   // loads of one step
    Rs rs;
    int G, r0, r1, rstep, B, lane, team;
    float* part;       // LDS [nsets][RPI][TEAM] lane partials (see gemv_matrix)

    // activation staging: int8 limbs (xprep.h)
    static constexpr int STAGE_TRIPS = stage_trips(R, U);
    using XS = XStage;
    static __device__ __forceinline__ XS xs_layout(void* lds, int K) { return brik::xstage_layout(lds, K); }
    static __device__ __forceinline__ size_t xs_bytes(int K) { return brik::xstage_bytes(K); }
    // NTH: the threads of the block that stages (a staging kernel runs more than a GEMV block)
    template <int NTH = NT, class After = brik::NoLoads>
    static __device__ __forceinline__ void stage(const float* __restrict__ x, const XS& S, int K, const Fuse& F,
                                                 After after_first = After())
    {
        brik::xstage<FMT, STAGE_TRIPS, NTH>(x, S, K, F, after_first);
    }

    __device__ __forceinline__ void init()
    {
        lane = threadIdx.x % TEAM;
        team = threadIdx.x / TEAM;
        B = (G + U * TEAM - 1) / (U * TEAM);
    }
    __device__ __forceinline__ bool even() const { return G % (U * TEAM) == 0; }

    __device__ __forceinline__ int n0(int p) const { return r0 + team * R + p * rstep; }

    // Loads of step (p, b), branch-free. Rows past r1 are clamped to r1 - 1 (their results are never
    // written). EVEN (G a multiple of U * TEAM): every group of every step exists, so the step's group
    // offset goes in the uniform soffset. Otherwise each lane's group index is clamped to G - 1 (the
    // consumer reads the zero group for those).
    template <bool EVEN>
    __device__ __forceinline__ void issue(Grp<FMT> (&d)[U][R], int p, int b) const
    {
        const int n = n0(p);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = (uint32_t)min(n + r, r1 - 1) * (uint32_t)G;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if constexpr (EVEN) {
                    load_grp<FMT>(d[u][r], rs, row + (uint32_t)lane, (uint32_t)(TEAM * U * b), (uint32_t)(u * TEAM));
                } else {
                    const uint32_t g = (uint32_t)min(lane + TEAM * (U * b + u), G - 1);
                    load_grp<FMT>(d[u][r], rs, row + g, 0u, 0u);
                }
            }
        }
    }

    // Consume step (p, b) into acc (reset first when b == 0) and store the lane partials.
    template <bool EVEN>
    __device__ __forceinline__ void consume(const Grp<FMT> (&d)[U][R], const XStage& S, int p, int b,
                                            float (&acc)[R]) const
    {
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = b == 0 ? 0.f : acc[r];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int gl = min(lane + TEAM * (U * b + u), G);      // G: the zero group
            const int hs = brik::half_swap(gl);
            const int8_t* b0 = S.limbs + 96 * gl + hs;              // half 0 of limb t at b0 + 32t
            const int8_t* b1 = S.limbs + 96 * gl + (16 - hs);       // half 1 of limb t at b1 + 32t
            u32x4_t xl[3][2];
#pragma unroll
            for (int t = 0; t < 3; ++t) {
                xl[t][0] = *(const u32x4_t*)(b0 + 32 * t);
                xl[t][1] = *(const u32x4_t*)(b1 + 32 * t);
            }
            const float2 xse = S.xse[gl];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = use_grp<FMT>(d[u][r], xl, xse, acc[r]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) part[(p * RPI + team * R + r) * TEAM + lane] = acc[r];
    }
};

// Bit k of the two bytes of h that `sel` picks (v_perm selector: bytes at 0 and 2, zeros between) to
// bit 2k: the 16-bit Morton spread, its first step done by the byte permute.
__device__ __forceinline__ uint32_t spread16(uint32_t h, uint32_t sel)
{
    uint32_t t = __builtin_amdgcn_perm(0u, h, sel);
    t = (t | (t << 4)) & 0x0F0F0F0Fu;
    t = (t | (t << 2)) & 0x33333333u;
    return (t | (t << 1)) & 0x55555555u;
}

__device__ __forceinline__ uint32_t bit_insert(uint32_t mask, uint32_t a, uint32_t b)
{
    return (a & mask) | (b & ~mask);     // v_bfi_b32
}

// A group's codes as four words of signed nibbles in the digit-plane order of the format (xprep.h
// digit_elem). q4: the code words as loaded, XOR 0x8 per nibble (q - 8; the staged 8 sum X undoes it).
// q3: lo word L (elements 16h .. 16h+15, 2 bits each) masked with 0x33333333 leaves the even elements
// in nibbles, L >> 2 the odd ones; the hi word spread to every other bit (element e's bit at 2e within
// its half) puts an even element's hi bit at nibble bit 2 after a shift by 2, an odd element's where it
// is. 14 instructions for the two spreads, 8 for the four words, instead of merging the planes into
// eight byte words (~35).
template <int FMT>
__device__ __forceinline__ void code_nibbles(const Grp<FMT>& d, uint32_t (&c)[4])
{
    if constexpr (FMT == FMT_Q4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = d.w[j] ^ 0x88888888u;
    } else {
        const uint32_t s0 = spread16(d.h, 0x0c010c00u), s1 = spread16(d.h, 0x0c030c02u);
        c[0] = bit_insert(0x33333333u, d.l.x, s0 << 2);
        c[1] = bit_insert(0x33333333u, d.l.x >> 2, s0);
        c[2] = bit_insert(0x33333333u, d.l.y, s1 << 2);
        c[3] = bit_insert(0x33333333u, d.l.y >> 2, s1);
    }
}

// q4 and q3 on v_dot8_i32_i4: x as signed 4-bit digit planes (xprep.h, xstage_d), codes as signed
// nibbles (code_nibbles). Per (row, group): 24 dot8 over the six digit planes d_5 .. d_0 in Horner
// chains, then one conversion, one exact rescale and two FMAs. With DigitChains<FMT> = C chains,
// chain k takes planes 5 - k, 5 - k - C, ... (most significant first, shifting by 4C bits between
// them), and sum X q = sum_k chain_k * 16^(C - 1 - k) (+ for q4 the staged 8 * sum X that undoes the
// -8), an exact int32 in wrapping arithmetic (no chain's partial sum can overflow: each is below
// 2048 * (1 + 2^(4C) + ...) < 2^28). The chains of a group's R rows are independent, so 3 chains
// give 3R dot8 sequences to interleave where one serial chain of 24 waits for each result: q4 decode
// launches of one or two waves per SIMD (Qwen3-4B, graph-replayed) q 4.35 -> 4.10 us, gate 6.40 ->
// 6.20, down 8.44 -> 8.20, k/v 3.45 -> 3.34, the fused decoder layer 30.9 -> 30.2 us, the 36-layer
// set 296.4 -> 295.5 us per step. The q3 LM head, whose code assembly already supplies independent
// work and which runs 4 waves per SIMD, measured 37.3 us with one chain against 37.6 with three, so
// q3 keeps one. The dot products use the clamping form: no partial sum overflows, so the value is
// the same, and the compiler keeps each chain as written instead of splitting it into sums.
//
// P = 2 (GLU pairs): two matrices of equal shape on the same staged x. A team's R rows are then
// RH = R / 2 rows of the first matrix (rs) followed by the same rows of the second (rs2): row r of
// the team is row n0(p) + r % RH of matrix r / RH. NTB: threads per block.
template <int FMT> struct DigitChains { static constexpr int v = FMT == FMT_Q4 ? 3 : 1; };
static_assert(6 % DigitChains<FMT_Q4>::v == 0 && 6 % DigitChains<FMT_Q3>::v == 0, "whole chains");

template <int FMT, int TEAM, int R, int U, int P = 1, int NTB = 256>
struct WorkD {
    static_assert(P == 1 || (P == 2 && R % 2 == 0), "pair rows");
    static constexpr int NT = NTB;                 // threads per block
    static constexpr int RPI = (NT / TEAM) * R;    // rows per block iteration, both matrices together
    static constexpr int RH = R / P;               // rows per team and matrix
    static constexpr int PARTS = TEAM;
    static constexpr int NACC = R;
    static constexpr int UG = U;
    typedef Grp<FMT> Data[U][R];
    Rs rs, rs2;
    int G, r0, r1, rstep, B, lane, team;
    float* part;

    static constexpr int STAGE_TRIPS = stage_trips(R, U);
    using XS = brik::XStageD;
    static __device__ __forceinline__ XS xs_layout(void* lds, int K) { return brik::xstage_d_layout(lds, K); }
    static __device__ __forceinline__ size_t xs_bytes(int K) { return brik::xstage_d_bytes(K); }
    template <int NTH = NT, class After = brik::NoLoads>
    static __device__ __forceinline__ void stage(const float* __restrict__ x, const XS& S, int K, const Fuse& F,
                                                 After after_first = After())
    {
        brik::xstage_d<FMT, STAGE_TRIPS, NTH>(x, S, K, F, after_first);
    }

    __device__ __forceinline__ void init()
    {
        lane = threadIdx.x % TEAM;
        team = threadIdx.x / TEAM;
        B = (G + U * TEAM - 1) / (U * TEAM);
    }
    __device__ __forceinline__ bool even() const { return G % (U * TEAM) == 0; }
    __device__ __forceinline__ int n0(int p) const { return r0 + team * RH + p * rstep; }

    template <bool EVEN>
    __device__ __forceinline__ void issue(Grp<FMT> (&d)[U][R], int p, int b) const
    {
        const int n = n0(p);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = (uint32_t)min(n + r % RH, r1 - 1) * (uint32_t)G;
            const Rs& q = r < RH ? rs : rs2;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if constexpr (EVEN) {
                    load_grp<FMT>(d[u][r], q, row + (uint32_t)lane, (uint32_t)(TEAM * U * b), (uint32_t)(u * TEAM));
                } else {
                    const uint32_t g = (uint32_t)min(lane + TEAM * (U * b + u), G - 1);
                    load_grp<FMT>(d[u][r], q, row + g, 0u, 0u);
                }
            }
        }
    }

    template <bool EVEN>
    __device__ __forceinline__ void consume(const Grp<FMT> (&d)[U][R], const XS& S, int p, int b,
                                            float (&acc)[R]) const
    {
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = b == 0 ? 0.f : acc[r];
        // EVEN: group lane + TEAM (U b + u) sits at 112 (lane + TEAM U b) + 112 TEAM u (an immediate)
        const unsigned char* a0 = S.base + 112 * (lane + TEAM * U * b);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const unsigned char* a;
            if constexpr (EVEN) a = a0 + 112 * TEAM * u;
            else a = S.base + 112 * min(lane + TEAM * (U * b + u), G);    // G: the zero group
            u32x4_t L[6];
#pragma unroll
            for (int n = 0; n < 6; ++n) L[n] = *(const u32x4_t*)(a + 16 * n);
            const i32x4_t xs = *(const i32x4_t*)(a + 96);                   // {sum x, e - 22, 8 sum X, 0}
            // The six plane reads issue together, so one LDS round trip per group is waited for (left to
            // itself the compiler reads each plane just before its dot products, six waits per group),
            // on the q4 variants of one group per lane step whose teams are 16 or 64 lanes: the fused
            // decoder layer 30.3 -> 29.9 us per layer in alternating processes on one box. The others
            // keep the compiler's order: there the batched reads cost registers and time (the 36-layer
            // set 296.2 -> 297.4 us, the single q and gate launches +1 %, down on 32-lane teams 8.23 ->
            // 8.38 us, the q3 LM head 84 -> 152 VGPRs, 4 -> 3 waves per SIMD, 38.2 -> 39.4 us).
            if constexpr (FMT == FMT_Q4 && U == 1 && TEAM != 32) __builtin_amdgcn_sched_barrier(0);
            uint32_t c[R][4];
#pragma unroll
            for (int r = 0; r < R; ++r) code_nibbles<FMT>(d[u][r], c[r]);
            constexpr int CH = DigitChains<FMT>::v;
            int ch[CH][R];
#pragma unroll
            for (int t = 0; t < 6 / CH; ++t) {
#pragma unroll
                for (int k = 0; k < CH; ++k)
#pragma unroll
                    for (int r = 0; r < R; ++r) ch[k][r] = t == 0 ? 0 : ch[k][r] << (4 * CH);
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int k = 0; k < CH; ++k)
#pragma unroll
                        for (int r = 0; r < R; ++r)
                            ch[k][r] = __builtin_amdgcn_sdot8((int)c[r][j], (int)L[5 - k - CH * t][j], ch[k][r], true);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t vu = FMT == FMT_Q4 ? (uint32_t)xs.z : 0u;
#pragma unroll
                for (int k = 0; k < CH; ++k) vu += (uint32_t)ch[k][r] << (4 * (CH - 1 - k));
                const float pr = ldexpf((float)(int)vu, xs.y);                // exact rescale
                acc[r] = __builtin_fmaf(f16_bits_to_f32(d[u][r].s), pr, acc[r]);
                acc[r] = __builtin_fmaf(f16_bits_to_f32(d[u][r].m), __builtin_bit_cast(float, xs.x), acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) part[(p * RPI + team * R + r) * TEAM + lane] = acc[r];
    }
};

template <int TEAM, int R, int U>
struct Work<FMT_Q4, TEAM, R, U> : WorkD<FMT_Q4, TEAM, R, U> {};
template <int TEAM, int R, int U>
struct Work<FMT_Q3, TEAM, R, U> : WorkD<FMT_Q3, TEAM, R, U> {};
// GLU pair work (digit-plane formats only)
template <int FMT, int TEAM, int R, int U, int NT>
using PairWork = WorkD<FMT, TEAM, R, U, 2, NT>;

// Exact path for a row holding Inf/NaN: teams of 16 lanes (16 in a 256-thread block); in every row set
// (rows base + [0, RPI), base = r0, r0 + rstep, ...) team t takes rows t, t + teams, ... (any RPI).
template <int FMT, int RPI, int NT>
__device__ __forceinline__ void gemv_rows_exact(const float* __restrict__ x, const Fuse& F, float inv,
                                                const Planes& P, float* __restrict__ yrow,
                                                const float* __restrict__ res, int K, int r0, int r1, int rstep)
{
    const int lane = threadIdx.x % 16;
    const int team = threadIdx.x / 16;
    constexpr int nteams = NT / 16;
    for (int base = r0; base < r1; base += rstep) {
        for (int i = team; i < RPI; i += nteams) {
            const int n = base + i;         // uniform across the team's 16 lanes
            if (n >= r1) break;
            float acc = 0.f;
            for (int k = lane; k < K; k += 16)
                acc = __builtin_fmaf(brik::fused_in(x, F, inv, k), deq_elem<FMT>(P, (size_t)n * K + k), acc);
            acc = team_sum<16>(acc);
            if (lane == 0) yrow[n] = res ? res[n] + acc : acc;
        }
    }
}

// Copy a staged x image of `bytes` bytes (a multiple of 8) from global memory into LDS at `lds`:
// direct global->LDS loads, 1 KiB per wave instruction, 16 bytes per lane.
template <int NT>
__device__ __forceinline__ void stage_copy(const unsigned char* __restrict__ src, unsigned char* lds, uint32_t bytes)
{
    const brsrc_t r = make_rsrc(src, bytes);
    const uint32_t lane = threadIdx.x & 63;
    for (uint32_t c0 = (threadIdx.x >> 6) * 1024u; c0 < bytes; c0 += NT * 16u)
        if (c0 + 16u * lane < bytes)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (brik::lds_void_t*)(lds + c0), 16, c0 + 16u * lane, 0, 0, 0);
}

// The software pipeline of one team: D - 1 steps issued while x is staged, then a straight-line
// loop (unrolled by D so buffer indices are static) issuing step i + D - 1 and consuming step i.
// Vector-memory loads complete in issue order, so whatever x comes from is loaded first and the D - 1
// weight steps are issued behind it: staging then waits for x alone and runs while the weights are in
// flight (issued first, they had to arrive before staging could start, and the two latencies added
// up). In-block staging issues the weights after its first batch of x loads (xprep.h batched_in); with a
// pre-staged image (`staged`, written by brik_gemv_stage_<fmt> or by a GLU pair launch) the block
// copies it into LDS, then issues the weights. An image that holds only groups [0, img_groups) (a GLU
// pair launch that wrote those; 0: the whole image) is copied as far as it goes and the block stages the
// remaining groups itself, issuing the weights after the first batch of those loads. Returns true,
// before any step is consumed, if the row holds a value that is not finite: the caller then runs the
// exact path.
template <int FMT, class W, int D, bool EVEN>
__device__ __forceinline__ bool pipeline(W& w, const typename W::XS& X, const float* __restrict__ x, const Fuse& F,
                                         int K, int S, const unsigned char* __restrict__ staged, unsigned char* lds,
                                         int img_groups = 0)
{
    typename W::Data d[D];
    int ip = 0, bp = 0;                      // (p, b) of the next step to issue
    auto issue_ahead = [&] {
#pragma unroll
        for (int k = 0; k < D - 1; ++k) {
            w.template issue<EVEN>(d[k], ip, bp);
            const bool wrap = bp + 1 == w.B;
            bp = wrap ? 0 : bp + 1;
            ip += wrap;
        }
    };
    int flag;
    if (staged) {
        bool part = false;
        if constexpr (FMT != FMT_Q8) part = img_groups > 0 && img_groups < X.G;
        if (part) {
            // the tail's loads first, then the copy and the weights: the LDS writes of the tail's groups
            // come after every load is issued (the compiler waits for a direct global->LDS load before
            // any later LDS write, so a copy issued first would hold back the tail's loads)
            // the producer's values of the remaining groups follow its image in the same buffer
            if constexpr (FMT != FMT_Q8)
                brik::xstage_d_tail<FMT, W::STAGE_TRIPS, W::NT>(
                    (const float*)(staged + ((W::xs_bytes(K) + 15) & ~(size_t)15)), X, img_groups, [&] {
                    stage_copy<W::NT>(staged, lds, 112u * (uint32_t)img_groups);
                    __builtin_amdgcn_sched_barrier(0);
                    issue_ahead();
                });
        } else {
            stage_copy<W::NT>(staged, lds, (uint32_t)((W::xs_bytes(K) + 15) & ~(size_t)15));
            __builtin_amdgcn_sched_barrier(0);
            issue_ahead();
        }
        // every load issued after the copy (and the staged tail's loads) is one of the D - 1 weight
        // steps above
        brik::wait_vmcnt<(D - 1) * W::NACC * W::UG * LoadsPerGroup<FMT>::v>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        flag = *X.flag;
        // a GLU pair launch writes the groups of an image but not its flag, which stays -1: each group
        // then carries its own marker (a stager writes the flag, 0 or 1)
        if constexpr (FMT != FMT_Q8)
            if (flag < 0) flag = brik::image_bad<W::NT>(X);
    } else {
        W::stage(x, X, K, F, issue_ahead);
        flag = *X.flag;
    }
    if (flag) return true;
    float acc[W::NACC] = {};
    int pc = 0, bc = 0;                      // (p, b) of the next step to consume
    int i = 0;
    for (; i + D <= S; i += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            w.template issue<EVEN>(d[(k + D - 1) % D], ip, bp);
            {
                const bool wrap = bp + 1 == w.B;
                bp = wrap ? 0 : bp + 1;
                ip += wrap;
            }
            w.template consume<EVEN>(d[k], X, pc, bc, acc);
            const bool wrap = bc + 1 == w.B;
            bc = wrap ? 0 : bc + 1;
            pc += wrap;
        }
    }
    // the remaining S - i < D steps are already issued
#pragma unroll
    for (int k = 0; k < D - 1; ++k) {
        if (i + k < S) {
            w.template consume<EVEN>(d[k], X, pc, bc, acc);
            const bool wrap = bc + 1 == w.B;
            bc = wrap ? 0 : bc + 1;
            pc += wrap;
        }
    }
    return false;
}

// The sums of `rows` rows of PARTS lane partials each (LDS, row-major: partial l of row q at
// part[q * PARTS + l]): PARTS consecutive threads load one row's partials together and add them with
// DPP steps within 16-lane rows and __shfl_xor exchanges across them (team_sum), and the row's first
// lane calls out(q, sum). Every row sums in the same order, whichever thread holds it. Called by every thread of
// the block (NT threads, a multiple of PARTS); the partials must be complete (after a barrier).
template <int PARTS, int NT, class Out>
__device__ __forceinline__ void row_sums(const float* __restrict__ part, int rows, Out out)
{
    constexpr int per = NT / PARTS;                   // rows per pass
    const int l = (int)threadIdx.x % PARTS;
    for (int q0 = 0; q0 < rows; q0 += per) {          // the same trips for every thread: the DPP steps
        const int q = q0 + (int)threadIdx.x / PARTS;  // see whole teams
        const float v = team_sum<PARTS>(q < rows ? part[q * PARTS + l] : 0.f);
        if (l == 0 && q < rows) out(q, v);
    }
}

// The sampling pre-work of an LM head (topk.hip, brik_topk_prep) applied to the head's own output
// rows as they are written: softcap, then the repetition penalty for rows listed in `recent`, and the
// maximum order key of every 16 consecutive logits into maxima[n / 16] (the layout brik_topk_select
// reads), so the logits are not read back by a separate pass.
struct HeadEpi {
    float cap;                 // softcap when > 0
    int pen;                   // penalty applies
    float penalty;
    const int32_t* recent;     // n_recent ids
    int n_recent;
    uint32_t* maxima;          // one per 16 logits
};

// Rows of the block (q = p RPI + i: row r0 + p rstep + i) given their sums v[q] in LDS: the head's
// transforms, the logits written, the 16-row maxima. RPI and the set starts are multiples of 16, so 16
// consecutive q are one chunk of 16 consecutive rows. marks: a bitmap of the block's rows (LDS, zeroed
// by the caller's earlier pass). Every thread of the block calls it.
template <int RPI, int NT>
__device__ __forceinline__ void head_finish(const HeadEpi& h, const float* __restrict__ v, uint32_t* marks,
                                            float* __restrict__ yrow, int N, int r0, int rstep, int nsets)
{
    static_assert(RPI % 16 == 0 && NT % 16 == 0, "16-row chunks");
    const int rows = nsets * RPI;
    if (h.pen) {
        // ids outside [0, N) are skipped, as brik_topk_prep does
        for (int r = (int)threadIdx.x; r < h.n_recent; r += NT) {
            const int id = h.recent[r];
            const int d = id - r0;
            if (id >= 0 && id < N && d >= 0) {
                const int p = d / rstep, i = d % rstep;
                if (p < nsets && i < RPI) atomicOr(&marks[(p * RPI + i) >> 5], 1u << ((p * RPI + i) & 31));
            }
        }
        __syncthreads();
    }
    for (int q0 = 0; q0 < rows; q0 += NT) {              // the same trips for every thread (DPP below)
        const int q = q0 + (int)threadIdx.x;
        const int n = r0 + (q / RPI) * rstep + q % RPI;
        uint32_t key = 0u;
        if (q < rows && n < N) {
            float t = v[q];
            const bool p = h.pen && ((marks[q >> 5] >> (q & 31)) & 1u);
            if (h.cap > 0.f) t = h.cap * tanhf(t / h.cap);
            if (p) t = t > 0.f ? t / h.penalty : t * h.penalty;
            yrow[n] = t;
            key = order_key(t);
        }
        key = max16u(key);
        if ((q & 15) == 0 && q < rows && n < N) h.maxima[n >> 4] = key;
    }
}

// Rows [r0, r1) of one N x K matrix in steps of rstep: first loads, x staging, the pipelined steps,
// then the cross-lane sums of the LDS partials are written to y. The block owns row sets
// p = 0 .. nsets-1 with rows r0 + p * rstep + [0, RPI). With a head epilogue (HEAD, he), the sums go
// through head_finish instead: its LDS (the sums, the penalty bitmap) follows the partials.
template <int FMT, class W, int D, bool HEAD = false>
__device__ __forceinline__ void gemv_matrix(const float* __restrict__ x, const Fuse& F, const Planes& P,
                                            float* __restrict__ yrow, const float* __restrict__ res,
                                            int N, int K, int r0, int r1, int rstep, unsigned char* lds,
                                            const unsigned char* __restrict__ staged, int img_groups = 0,
                                            const HeadEpi* he = nullptr)
{
    W w;
    w.G = K / BRIK_GROUP;
    w.rs = make_rs<FMT>(P, N, w.G);
    w.r0 = r0; w.r1 = r1; w.rstep = rstep;
    w.init();
    const int nsets = r0 < r1 ? (r1 - r0 + rstep - 1) / rstep : 0;     // block-uniform
    const int S = nsets * w.B;                                            // steps per lane
    const typename W::XS X = W::xs_layout(lds, K);
    w.part = (float*)(lds + W::xs_bytes(K));
    const bool exact = w.even() ? pipeline<FMT, W, D, true>(w, X, x, F, K, S, staged, lds, img_groups)
                                : pipeline<FMT, W, D, false>(w, X, x, F, K, S, staged, lds, img_groups);
    float* hv = w.part + (size_t)nsets * W::RPI * W::PARTS;           // HEAD: the row sums
    uint32_t* marks = (uint32_t*)(hv + nsets * W::RPI);               // HEAD: the penalty bitmap
    if constexpr (HEAD)
        for (int i = (int)threadIdx.x; i < (nsets * W::RPI + 31) / 32; i += W::NT) marks[i] = 0u;
    if (exact) {
        // teams of 16 lanes over RPI rows per iteration
        gemv_rows_exact<FMT, W::RPI, W::NT>(x, F, *X.inv, P, yrow, res, K, r0, r1, rstep);
        if constexpr (HEAD) {
            __syncthreads();       // the rows just written are visible to the block
            for (int q = (int)threadIdx.x; q < nsets * W::RPI; q += W::NT) {
                const int n = r0 + (q / W::RPI) * rstep + q % W::RPI;
                hv[q] = n < r1 ? yrow[n] : 0.f;
            }
            __syncthreads();
            head_finish<W::RPI, W::NT>(*he, hv, marks, yrow, r1, r0, rstep, nsets);
        }
        return;
    }
    __syncthreads();
    // cross-lane sums (row_sums), times the RMSNorm factor of a fused input (1 otherwise: exact), which
    // the staged image leaves out; rows past r1 are skipped
    const float inv = *X.inv;
    row_sums<W::PARTS, W::NT>(w.part, nsets * W::RPI, [&](int q, float v) {
        const int n = r0 + (q / W::RPI) * rstep + q % W::RPI;
        if (n < r1) {
            v *= inv;
            v = res ? res[n] + v : v;
            if constexpr (HEAD) hv[q] = v;
            else yrow[n] = v;
        }
    });
    if constexpr (HEAD) {
        __syncthreads();
        head_finish<W::RPI, W::NT>(*he, hv, marks, yrow, r1, r0, rstep, nsets);
    }
}

// One matrix, one activation row per grid.y. `staged` (M = 1 only): the row's LDS image, written by
// brik_gemv_stage1_<fmt>, which every block copies instead of staging x itself.
template <int FMT, class W, int D>
__device__ __forceinline__ void gemv_body(const float* __restrict__ x, const uint8_t* __restrict__ p0,
                                          const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc,
                                          const uint16_t* __restrict__ mn, float* __restrict__ y, int K, int N,
                                          const unsigned char* __restrict__ staged)
{
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int RPI = W::RPI;     // rows per block iteration
    const Planes P{p0, p1, sc, mn};
    gemv_matrix<FMT, W, D>(x + (size_t)blockIdx.y * K, Fuse{nullptr, nullptr, 0.f, 0}, P, y + (size_t)blockIdx.y * N,
                           nullptr, N, K, blockIdx.x * RPI, N, gridDim.x * RPI, lds, staged);
}

// Grouped GEMV over a plan's block table: block b runs rows [r0, r1) of the job in blocks[b], in row
// sets of RPI rows. With a stage buffer (non-null stage_base) the job's x image is at
// stage_base + stage_off, whole or (img_groups > 0) its first img_groups groups.
template <int FMT, class W, int D>
__device__ __forceinline__ void gemv_grouped_body(const brik_gemv_block* __restrict__ blocks,
                                                  const unsigned char* __restrict__ stage_base)
{
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int RPI = W::RPI;
    const brik_gemv_block bd = blocks[blockIdx.x];
    const brik_gemv_job_ex& je = bd.job;
    const brik_gemv_job& job = je.job;
    const Planes P{(const uint8_t*)job.p0, (const uint8_t*)job.p1, job.scales, job.mins};
    gemv_matrix<FMT, W, D>(job.x, Fuse{je.gate, je.norm_w, je.eps, je.flags}, P, job.y, je.res, job.N, job.K, bd.r0,
                           bd.r1, RPI, lds, stage_base ? stage_base + bd.stage_off : nullptr, (int)bd.img_groups);
}

// GLU pair (brik_gemv_plan_create_glu): rows [r0, r0 + H) of gate (jobs jg) and up (ju), H = RPI / 2,
// both N x K on one staged x (their common input and fusion), in one row set; then the staged image
// of act(gate) * up over these rows, which are whole quantization groups of the consumer's K' = N
// input (H and r0 are multiples of 32): written to img + 112 g for each group g they cover, in the
// digit-plane layout of xprep.h, bit-identical to what the consumer would stage (stage_group_lanes,
// the 32-lane form of the code that stages a row in LDS). Each row sum
// uses the same lane partials, summed in the same order (a rotation by the row index), as the
// single-matrix path with the same TEAM and U, so gate and up, and with them the image, are
// bit-identical to those of unpaired plans.
// IMG = false: the pair launch's blocks past the whole groups it writes images for (H any whole number
// of team rows): gate.y, up.y and act(gate) * up of rows n >= tail0 at index n - tail0 of the values
// that follow the image in the same buffer, which the consumer stages itself.
template <int FMT, class W, int D, bool IMG = true>
__device__ __forceinline__ void gemv_glu_pair(const brik_gemv_job_ex& jg, const brik_gemv_job_ex& ju, int r0,
                                              unsigned char* __restrict__ img, int act_flags, unsigned char* lds,
                                              int tail0 = 0)
{
    constexpr int H = W::RPI / 2, RH = W::RH, R = W::NACC, PARTS = W::PARTS;
    static_assert((!IMG || H % BRIK_GROUP == 0) && R == 2 * RH, "whole groups per block");
    const int K = jg.job.K, N = jg.job.N;
    const Fuse F{jg.gate, jg.norm_w, jg.eps, jg.flags};
    const Planes Pg{(const uint8_t*)jg.job.p0, (const uint8_t*)jg.job.p1, jg.job.scales, jg.job.mins};
    const Planes Pu{(const uint8_t*)ju.job.p0, (const uint8_t*)ju.job.p1, ju.job.scales, ju.job.mins};
    W w;
    w.G = K / BRIK_GROUP;
    w.rs = make_rs<FMT>(Pg, N, w.G);
    w.rs2 = make_rs<FMT>(Pu, N, w.G);
    w.r0 = r0; w.r1 = min(N, r0 + H); w.rstep = H;
    w.init();
    const typename W::XS X = W::xs_layout(lds, K);
    w.part = (float*)(lds + W::xs_bytes(K));
    const bool exact = w.even() ? pipeline<FMT, W, D, true>(w, X, jg.job.x, F, K, w.B, nullptr, lds)
                                : pipeline<FMT, W, D, false>(w, X, jg.job.x, F, K, w.B, nullptr, lds);
    float* vals = (float*)lds;     // gate then up values of the set; the x image is not read any more
    if (exact) {
        gemv_rows_exact<FMT, H, W::NT>(jg.job.x, F, *X.inv, Pg, jg.job.y, jg.res, K, w.r0, w.r1, H);
        gemv_rows_exact<FMT, H, W::NT>(ju.job.x, F, *X.inv, Pu, ju.job.y, ju.res, K, w.r0, w.r1, H);
        __syncthreads();           // the rows just written are visible to the block
        for (int q = threadIdx.x; q < 2 * H; q += W::NT) {
            const int n = r0 + q % H;
            vals[q] = n < N ? (q < H ? jg.job.y : ju.job.y)[n] : 0.f;
        }
    } else {
        __syncthreads();
        // read by every thread before the values overwrite LDS: a tiny row's image tail, inv included,
        // lies under them (the partials do not: they start past the image, at 304 bytes or more)
        const float inv = *X.inv;
        __syncthreads();
        // partial row q = team * R + r is row i = team * RH + r % RH of matrix r / RH; summed as the
        // unpaired plans sum theirs (row_sums), so gate and up are bit-identical to those
        row_sums<PARTS, W::NT>(w.part, W::RPI, [&](int q, float s) {
            const int r = q % R, m = r / RH, i = q / R * RH + r % RH;
            s *= inv;
            const int n = r0 + i;
            if (n < N) {
                const float* res = m ? ju.res : jg.res;
                s = res ? res[n] + s : s;
                (m ? ju.job.y : jg.job.y)[n] = s;
            }
            vals[m * H + i] = s;
        });
    }
    __syncthreads();
    if constexpr (!IMG) {
        float* tail = (float*)(img + ((W::xs_bytes(N) + 15) & ~(size_t)15));
        const int q = (int)threadIdx.x;
        if (q < H && r0 + q < N) tail[r0 + q - tail0] = brik::act(vals[q], act_flags) * vals[H + q];
        return;
    }
    // group g on lanes 0-31 of wave g, lane e holding element e
    const int g = threadIdx.x >> 6, e = threadIdx.x & 63;
    if (g < H / BRIK_GROUP && e < BRIK_GROUP) {
        const float v = brik::act(vals[BRIK_GROUP * g + e], act_flags) * vals[H + BRIK_GROUP * g + e];
        brik::stage_group_lanes<FMT>(v, img + 112 * (r0 / BRIK_GROUP + g));
    }
}

}  // namespace

#define BRIK_GEMV(FMTN, FMT, TEAM, RR, UU, DD)                                                      \
    extern "C" __global__ __launch_bounds__(256) void brik_gemv_##FMTN##_t##TEAM##_r##RR##_u##UU##_d##DD( \
        const float* __restrict__ x, const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1, \
        const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, float* __restrict__ y,    \
        int K, int N, const unsigned char* __restrict__ staged)                                     \
    {                                                                                               \
        gemv_body<FMT, Work<FMT, TEAM, RR, UU>, DD>(x, p0, p1, sc, mn, y, K, N, staged);            \
    }                                                                                               \
    extern "C" __global__ __launch_bounds__(256) void brik_gemvg_##FMTN##_t##TEAM##_r##RR##_u##UU##_d##DD( \
        const brik_gemv_block* __restrict__ blocks, const unsigned char* __restrict__ stage_base)    \
    {                                                                                               \
        gemv_grouped_body<FMT, Work<FMT, TEAM, RR, UU>, DD>(blocks, stage_base);                    \
    }

// The variant table of the runtime (brik_runtime.cpp, kGemvVariants) lists these in this order.
#define BRIK_GEMV_FMT(FMTN, FMT)     \
    BRIK_GEMV(FMTN, FMT, 16, 2, 1, 2) \
    BRIK_GEMV(FMTN, FMT, 16, 2, 1, 3) \
    BRIK_GEMV(FMTN, FMT, 16, 2, 1, 4) \
    BRIK_GEMV(FMTN, FMT, 16, 4, 1, 2) \
    BRIK_GEMV(FMTN, FMT, 16, 2, 2, 2) \
    BRIK_GEMV(FMTN, FMT, 32, 2, 1, 3) \
    BRIK_GEMV(FMTN, FMT, 64, 1, 1, 3) \
    BRIK_GEMV(FMTN, FMT, 16, 2, 5, 2) \
    BRIK_GEMV(FMTN, FMT, 16, 1, 5, 2) \
    BRIK_GEMV(FMTN, FMT, 16, 1, 2, 2) \
    BRIK_GEMV(FMTN, FMT, 32, 1, 1, 2)

BRIK_GEMV_FMT(q4, FMT_Q4)
BRIK_GEMV_FMT(q8, FMT_Q8)
BRIK_GEMV_FMT(q3, FMT_Q3)

// An LM head with the sampling pre-work in its epilogue (HeadEpi, head_finish): the q4 / q3 variant of
// single matrices whose x image is staged once per call (whole rows, two rows per team). The runtime
// (brik_runtime.cpp, lm_head_topk) then runs brik_topk_select on the maxima it writes.
#define BRIK_GEMV_HEAD(FMTN, FMT, TEAM, RR, UU, DD)                                                      \
    extern "C" __global__ __launch_bounds__(256) void brik_gemvh_##FMTN##_t##TEAM##_r##RR##_u##UU##_d##DD( \
        const float* __restrict__ x, const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,      \
        const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, float* __restrict__ y, int K,   \
        int N, const unsigned char* __restrict__ staged, float cap, int pen, float penalty,              \
        const int32_t* __restrict__ recent, int n_recent, uint32_t* __restrict__ maxima)                 \
    {                                                                                                    \
        extern __shared__ __align__(16) unsigned char lds[];                                             \
        using W_ = Work<FMT, TEAM, RR, UU>;                                                              \
        const HeadEpi he{cap, pen, penalty, recent, n_recent, maxima};                                  \
        gemv_matrix<FMT, W_, DD, true>(x, Fuse{nullptr, nullptr, 0.f, 0}, Planes{p0, p1, sc, mn}, y,     \
                                       nullptr, N, K, (int)blockIdx.x * W_::RPI, N,                      \
                                       (int)gridDim.x * W_::RPI, lds, staged, 0, &he);                   \
    }
BRIK_GEMV_HEAD(q4, FMT_Q4, 16, 2, 5, 2)
BRIK_GEMV_HEAD(q3, FMT_Q3, 16, 2, 5, 2)

// GLU pair launch: jobs[0] = gate, jobs[1] = up. Block b < nfull (NT threads, teams of TEAM lanes)
// runs rows [H b, H b + H) of both, H = RPI / 2 = 32 (one quantization group of down's input), and
// writes that group of the image of act(gate) * up to img (act_flags: BRIK_JOB_ACT_GELU or 0). Blocks
// past nfull run 8 rows of both each (teams of 64 lanes) from row 32 nfull on and write gate.y, up.y
// and act(gate) * up of their rows after the image: the runtime keeps nfull at a whole number of
// blocks per CU when the groups exceed the CUs by a small remainder, and the consumer stages those
// last groups itself from those values, so no CU runs two of the 64-row blocks while others run one.
// The runtime table (brik_runtime.cpp, kGluVariant) names this shape.
#define BRIK_GEMV_PAIR(FMTN, FMT, TEAM, RR, UU, DD, NT)                                                   \
    extern "C" __global__ __launch_bounds__(NT) void brik_gemvp_##FMTN##_t##TEAM##_r##RR##_u##UU##_d##DD##_n##NT( \
        const brik_gemv_job_ex* __restrict__ jobs, unsigned char* __restrict__ img, int act_flags, int nfull) \
    {                                                                                                   \
        extern __shared__ __align__(16) unsigned char lds[];                                            \
        using W_ = PairWork<FMT, TEAM, RR, UU, NT>;                                                     \
        using WB_ = PairWork<FMT, 64, RR, 1, NT>;                                                       \
        const int b = (int)blockIdx.x;                                                                  \
        if (b < nfull)                                                                                  \
            gemv_glu_pair<FMT, W_, DD>(jobs[0], jobs[1], b * (W_::RPI / 2), img, act_flags, lds);       \
        else                                                                                            \
            gemv_glu_pair<FMT, WB_, DD, false>(jobs[0], jobs[1],                                        \
                                               nfull * (W_::RPI / 2) + (b - nfull) * (WB_::RPI / 2), img, \
                                               act_flags, lds, nfull * (W_::RPI / 2));                  \
    }
BRIK_GEMV_PAIR(q4, FMT_Q4, 16, 2, 1, 2, 512)
BRIK_GEMV_PAIR(q3, FMT_Q3, 16, 2, 1, 2, 512)

// Staging pass of a large grouped plan: block i (1024 threads) writes the LDS image of input i (x, or
// its fused transform) to out + in[i].off in the layout a plan block stages (it depends only on the
// format). An RMSNorm factor's f32 sum of squares runs over 16 waves here, so it may round
// differently from a 4-wave block's.
namespace {
template <int FMT>
__device__ __forceinline__ void stage_input(const brik_stage_input* __restrict__ in, unsigned char* __restrict__ out)
{
    using W = Work<FMT, 16, 2, 1>;
    const brik_stage_input e = in[blockIdx.x];
    const typename W::XS S = W::xs_layout(out + e.off, e.K);
    W::template stage<1024>(e.x, S, e.K, Fuse{e.gate, e.norm_w, e.eps, e.flags});
}
}  // namespace

// Staging of one plain activation row for a single-matrix M = 1 call (brik_matmul_t_<fmt>): one block.
namespace {
template <int FMT>
__device__ __forceinline__ void stage_row(const float* __restrict__ x, int K, unsigned char* __restrict__ out)
{
    using W = Work<FMT, 16, 2, 1>;
    W::template stage<1024>(x, W::xs_layout(out, K), K, Fuse{nullptr, nullptr, 0.f, 0});
}
}  // namespace

extern "C" __global__ __launch_bounds__(1024) void brik_gemv_stage1_q4(const float* __restrict__ x, int K,
                                                                      unsigned char* __restrict__ out)
{
    stage_row<FMT_Q4>(x, K, out);
}
extern "C" __global__ __launch_bounds__(1024) void brik_gemv_stage1_q3(const float* __restrict__ x, int K,
                                                                      unsigned char* __restrict__ out)
{
    stage_row<FMT_Q3>(x, K, out);
}

extern "C" __global__ __launch_bounds__(1024) void brik_gemv_stage_q8(const brik_stage_input* __restrict__ in,
                                                                     unsigned char* __restrict__ out)
{
    stage_input<FMT_Q8>(in, out);
}
extern "C" __global__ __launch_bounds__(1024) void brik_gemv_stage_q4(const brik_stage_input* __restrict__ in,
                                                                     unsigned char* __restrict__ out)
{
    stage_input<FMT_Q4>(in, out);
}
extern "C" __global__ __launch_bounds__(1024) void brik_gemv_stage_q3(const brik_stage_input* __restrict__ in,
                                                                     unsigned char* __restrict__ out)
{
    stage_input<FMT_Q3>(in, out);
}
