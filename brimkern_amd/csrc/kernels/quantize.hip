// f32 -> packed .brik planes on the GPU, byte-identical to the reference's CPU encoders quantizeQ8 /
// quantizeQ4 / quantizeQ3 + packQ* (src/lib/brik/q8web.ts:28-50, q4web.ts:28-53, q3web.ts:34-60),
// which the loader and the GGUF->BRIK converter produce and the matmuls consume. The reference's own
// GPU quantizers (quantize_q8 / quantize_q4, src/lib/webgpu/shaders.ts:1285-1356) round ties to even
// and compute in f32; these follow the CPU encoders instead, whose arithmetic is JavaScript doubles:
//   q8: s = f16(amax / 127 || 1e-8);                 q = clamp(round_half_up(x / s), -127, 127)
//   q4: s = f16((max - min) / 15 || 1e-8), m = f16(min); q = clamp(round_half_up((x - m) / s), 0, 15)
//   q3: as q4 with 7 levels
// with f16() = f32ToF16Bits (src/lib/brik/f16.ts:8-22) and the decoded value of the f16 bits used for
// the codes (|| 1e-8 again when it decodes to 0). The arithmetic that has to round as JavaScript's does
// (differences, quotients, the f16 round trip) runs in f64 on the GPU, where each of these operations is
// correctly rounded, and none of it has a product feeding a sum, so fused multiply-add contraction
// cannot change it; code_fast below decides the rounding of each code in f32 with a proven margin and
// hands the rare close cases to the f64 path.
//
// Layout: two lanes per 32-element group, 16 elements each. A wave takes 32 consecutive groups (4 KiB
// of f32): its lanes load them with consecutive 16-byte loads (1 KiB per instruction), stage them in
// the wave's own LDS rows with a 16-byte pad per group (36 floats), and each pair of lanes then encodes
// its group from LDS. The scan order, the min / max ties and the stores follow the reference's loop:
// each lane scans its half in order and the pair combines the halves keeping the first half's value on
// ties. Staging 32 groups per wave (18 KiB of LDS per block) lets a CU hold 32 waves, twice what
// one lane per group (64 groups per wave) allowed.
#include "common.h"

namespace {

// f32ToF16Bits: the value rounded to f32, then sign | exponent | 10-bit mantissa rounded half up on
// the first dropped bit; exponents below the normal range give +-0, above it +-65504 (0x7bff), and a
// mantissa carry out of exponent 30 gives the infinity bits, as the reference's conversion does.
// Branch-free: the rounded mantissa is added to the shifted exponent, so a carry out of the mantissa
// (r = 0x400) increments the exponent and clears the mantissa bits.
__device__ __forceinline__ uint32_t f16_encode(double v)
{
    const uint32_t x = __builtin_bit_cast(uint32_t, (float)v);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int exp = (int)((x >> 23) & 0xffu) - 127 + 15;
    const uint32_t mant = x & 0x7fffffu;
    const uint32_t body = ((uint32_t)exp << 10) + (mant >> 13) + ((mant >> 12) & 1u);
    return sign | (exp <= 0 ? 0u : exp >= 31 ? 0x7bffu : body);
}

// f16BitsToF32 for the bits f16_encode produces (no subnormals, no NaN; the infinity bits decode to
// infinity): the exact value, through the hardware conversion (every f16 value is an f32 value).
__device__ __forceinline__ float f16_decode(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// JavaScript's `v || 1e-8` for a number: 0 and NaN are falsy.
__device__ __forceinline__ double or_tiny(double v) { return (v == 0.0 || v != v) ? 1e-8 : v; }

// Math.round: the nearest integer, ties toward +infinity (exact for every double: v - floor(v) is
// exact below 2^52 and v is integral above). NaN stays NaN.
__device__ __forceinline__ double js_round(double v)
{
    const double f = floor(v);
    return v - f >= 0.5 ? f + 1.0 : f;
}

// The integer a clamped code becomes when stored into a typed array (NaN -> 0).
__device__ __forceinline__ int code_of(double q, double lo, double hi)
{
    if (q != q) return 0;
    q = q < lo ? lo : q > hi ? hi : q;
    return (int)q;
}

// The code of one value exactly as the reference computes it: Math.round(d / s) with the f64
// division, clamped to [lo, hi].
__device__ __forceinline__ int code_exact(double d, double s, double lo, double hi)
{
    return code_of(js_round(d / s), lo, hi);
}

// v_cvt_i32_f32: the integer part, saturating, with NaN -> 0 (the hardware conversion; a C cast of
// NaN would be undefined).
__device__ __forceinline__ int cvt_i32(float v)
{
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// The same code in f32, without a division. Per group: r = 1 / s to within 2^-23 relative (v_rcp_f32),
// c = 1/2 - m r (two f32 roundings). Per value, u = x r + c with one rounding: against the exact
// U = (x - m) / s + 1/2, |u - U| <= 5 * 2^-24 (|x| + |m|) / s + 2^-24 (the r error on both products,
// the roundings of m r, of c and of u, and |U| <= (|x| + |m|) / s + 1/2). JavaScript's f64 quotient,
// rounded half up, is floor of a value within 2^-52 (|x| + |m|) / s + 2^-53 of U. The margin
// e = (|x| + |m|) r 2^-20, about 16 * 2^-24 (|x| + |m|) / s, covers both whenever u lies near an
// integer (then |x - m| / s >= 1/2, so the absolute terms are at most 4 * 2^-24 (|x| + |m|) / s);
// far from one, when (|x| + |m|) / s < 1/11, u is within 0.1 of 1/2. So when u is farther than e
// from every integer, floor(u) is JavaScript's Math.round. Otherwise `unsure` is set and the caller
// redoes the group with code_exact (rare for weights: exact ties, values within about 2^-20 of one,
// or groups far from zero relative to their spread).
// NaN gives 0 and infinities saturate before the clamp, as the reference's stores and clamp do. For
// lo = 0 the truncating conversion gives the clamped floor (they differ only below 0), so no floor
// is taken. Per group: `c`, `er` = r 2^-20 and `h0` = 1/2 - |m| er; then 1/2 - e = h0 - |x| er.
template <int LO, int HI>
__device__ __forceinline__ int code_fast(float x, float r, float c, float er, float h0, bool& unsure)
{
    const float u = fmaf(x, r, c);
    const float h = fmaf(-fabsf(x), er, h0);
    int q;
    if constexpr (LO == 0) {
        unsure |= fabsf(__builtin_amdgcn_fractf(u) - 0.5f) >= h;
        q = cvt_i32(u);
    } else {
        const float fu = floorf(u);
        unsure |= fabsf((u - fu) - 0.5f) >= h;
        q = cvt_i32(fu);
    }
    return q < LO ? LO : q > HI ? HI : q;
}

constexpr int ENC_GROUPS = 32;           // groups per wave iteration (two lanes each)
constexpr int ENC_ROW = 36;              // floats per staged group: 32 + a 16-byte pad
constexpr int ENC_LOADS = ENC_GROUPS * 8 / 64;   // 16-byte loads per lane per wave iteration
constexpr int ENC_BLOCKS_PER_CU = 8;     // 18 KiB of LDS each: eight blocks (32 waves) per CU

// The wave's groups [g0, g0 + 32) of src, as lane-interleaved float4s: t[i] of lane l is float4
// 64 i + l of the range, so each load of the wave reads 1 KiB of consecutive f32. Past the end of
// src the last float4 is read again (in bounds; those rows are never encoded).
__device__ __forceinline__ void load_rows(const f32x4_t* __restrict__ src, size_t g0, size_t groups,
                                          f32x4_t (&t)[ENC_LOADS])
{
    const int lane = threadIdx.x & 63;
    const size_t limit = (groups - g0) * 8;           // float4s from g0 to the end of src
#pragma unroll
    for (int i = 0; i < ENC_LOADS; ++i) {
        const size_t f = (size_t)i * 64 + lane;
        t[i] = src[g0 * 8 + (f < limit ? f : limit - 1)];
    }
}

// Write loaded rows into the wave's own LDS rows (row j = group g0 + j, 16-byte pad per row). Only
// the wave itself touches its rows, so waiting for its own LDS writes orders them before its reads
// (no block barrier).
__device__ __forceinline__ void store_rows(const f32x4_t (&t)[ENC_LOADS], float* __restrict__ rows)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < ENC_LOADS; ++i) {
        const int f = i * 64 + lane;
        *reinterpret_cast<f32x4_t*>(rows + (f >> 3) * ENC_ROW + (f & 7) * 4) = t[i];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

__device__ __forceinline__ f32x4_t row4(const float* row, int i) { return *reinterpret_cast<const f32x4_t*>(row + 4 * i); }

// The value of the other lane of this lane's pair (lane ^ 1): DPP quad_perm [1, 0, 3, 2]. Both lanes of
// a pair always run together (they hold the same group).
__device__ __forceinline__ uint32_t pair_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ float pair_f32(float v) { return __builtin_bit_cast(float, pair_u32(__builtin_bit_cast(uint32_t, v))); }

// Combine the two halves' results of a scan that keeps the first of equal values: the second half's
// value replaces the first half's only when `beyond` it. `second`: this lane holds the second half.
__device__ __forceinline__ float first_min(float own, bool second)
{
    const float other = pair_f32(own);
    const float a = second ? other : own, b = second ? own : other;
    return b < a ? b : a;
}
__device__ __forceinline__ float first_max(float own, bool second)
{
    const float other = pair_f32(own);
    const float a = second ? other : own, b = second ? own : other;
    return b > a ? b : a;
}

// min and max of the group as the reference's loop finds them: NaN never replaces a value, and of
// equal values (+0 and -0) the first stays. Each lane scans its 16 elements in order; the pair then
// keeps the first half's value unless the second half's is strictly beyond it, which is what the
// scan over all 32 gives. The first pass takes v_min / v_max of the quieted values (NaN never
// replaces a value there either), which may pick either zero of a +0 / -0 tie: a group whose minimum
// or maximum is zero is scanned again with the reference's compares (both lanes of the pair see the
// same combined values, so they take that branch together).
__device__ __forceinline__ void min_max(const float* half, bool second, float& mn, float& mx)
{
    mn = __builtin_inff();
    mx = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const f32x4_t w = row4(half, i);
        const float e[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float c = __builtin_canonicalizef(e[j]);
            mn = fminf(mn, c);
            mx = fmaxf(mx, c);
        }
    }
    mn = first_min(mn, second);
    mx = first_max(mx, second);
    if (mn == 0.f || mx == 0.f) {
        mn = __builtin_inff();
        mx = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4_t w = row4(half, i);
            const float e[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (e[j] < mn) mn = e[j];
                if (e[j] > mx) mx = e[j];
            }
        }
        mn = first_min(mn, second);
        mx = first_max(mx, second);
    }
}

// The asymmetric (q4 / q3) group header: f16 scale (max - min) / L || 1e-8 and min, their decoded
// values s (|| 1e-8) and m, and 1 / s. Both lanes of the pair compute it (the same inputs, the same
// result).
template <int L>
__device__ __forceinline__ void asym_header(const float* half, bool second, uint32_t& sh, uint32_t& mh, double& s,
                                            double& m)
{
    float mn, mx;
    min_max(half, second, mn, mx);
    sh = f16_encode(or_tiny(((double)mx - (double)mn) / (double)L));
    mh = f16_encode((double)mn);
    s = or_tiny((double)f16_decode(sh));
    m = (double)f16_decode(mh);
}

// The per-group constants of code_fast for scale s and min m. A non-finite c (m infinite) marks the
// group unsure.
struct FastConst {
    float r, c, er, h0;
};
__device__ __forceinline__ FastConst fast_const(double s, double m, bool& unsure)
{
    FastConst k;
    const float mf = (float)m;
    k.r = __builtin_amdgcn_rcpf((float)s);
    k.c = 0.5f - mf * k.r;
    k.er = k.r * 0x1p-20f;
    k.h0 = 0.5f - fabsf(mf) * k.er;
    unsure = !(fabsf(k.c) <= 3.4028235e38f);
    return k;
}

// The wave's staging and loop, shared by the encoders: `encode(g, half, second)` encodes the half of
// group g starting at `half` in LDS (elements 16 second .. 16 second + 15 of the group).
template <class F>
__device__ __forceinline__ void encode_groups(const f32x4_t* __restrict__ src, size_t groups, float* lds, F&& encode)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float* rows = lds + wave * ENC_GROUPS * ENC_ROW;
    const bool second = lane & 1;
    const float* half = rows + (lane >> 1) * ENC_ROW + (second ? 16 : 0);
    const size_t stride = (size_t)gridDim.x * 4 * ENC_GROUPS;
    size_t g0 = ((size_t)blockIdx.x * 4 + wave) * ENC_GROUPS;
    f32x4_t t[ENC_LOADS];
    if (g0 < groups) load_rows(src, g0, groups, t);
    for (; g0 < groups; g0 += stride) {
        store_rows(t, rows);
        if (g0 + stride < groups) load_rows(src, g0 + stride, groups, t);     // the next rows, in flight meanwhile
        const size_t g = g0 + (lane >> 1);
        if (g < groups) encode(g, half, second);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");     // this lane's row reads are done
    }
}

}  // namespace

// In every encoder a wave iteration stages 32 groups and each pair of lanes encodes one group, a half
// each: the codes with code_fast, word by word, and, in the rare case that a value of the group was
// unsure, the half again with code_exact (the later stores overwrite the earlier words). The loads of
// the wave's next 32 groups are issued before the encoding, so they overlap it.
extern "C" __global__ __launch_bounds__(256) void brik_encode_q8(const f32x4_t* __restrict__ src,
                                                                 uint32_t* __restrict__ codes,
                                                                 uint16_t* __restrict__ scales, size_t groups)
{
    __shared__ __attribute__((aligned(16))) float lds[4 * ENC_GROUPS * ENC_ROW];
    encode_groups(src, groups, lds, [&](size_t g, const float* half, bool second) {
        // v_max of the quieted magnitudes: NaN never replaces a value, and equal magnitudes have one
        // bit pattern (|-0| = +0), so the order of the scan does not matter
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4_t w = row4(half, i);
            const float e[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fabsf(__builtin_canonicalizef(e[j])));
        }
        amax = first_max(amax, second);
        const uint32_t sh = f16_encode(or_tiny((double)amax / 127.0));
        if (!second) scales[g] = (uint16_t)sh;
        const double s = or_tiny((double)f16_decode(sh));
        bool unsure;
        const FastConst fk = fast_const(s, 0.0, unsure);
        uint32_t* out = codes + g * 8 + (second ? 4 : 0);
#pragma unroll 1
        for (int k = 0; k < 4; ++k) {
            const f32x4_t w = row4(half, k);
            const float e[4] = {w.x, w.y, w.z, w.w};
            uint32_t word = 0u;
#pragma unroll
            for (int b = 0; b < 4; ++b)
                word |= ((uint32_t)code_fast<-127, 127>(e[b], fk.r, fk.c, fk.er, fk.h0, unsure) & 0xffu) << (8 * b);
            out[k] = word;
        }
        if (unsure || pair_u32(unsure)) {
#pragma unroll 1
            for (int k = 0; k < 4; ++k) {
                uint32_t word = 0u;
                for (int b = 0; b < 4; ++b)
                    word |= ((uint32_t)code_exact((double)half[4 * k + b], s, -127.0, 127.0) & 0xffu) << (8 * b);
                out[k] = word;
            }
        }
    });
}

extern "C" __global__ __launch_bounds__(256) void brik_encode_q4(const f32x4_t* __restrict__ src,
                                                                 uint32_t* __restrict__ nibbles,
                                                                 uint16_t* __restrict__ scales,
                                                                 uint16_t* __restrict__ mins, size_t groups)
{
    __shared__ __attribute__((aligned(16))) float lds[4 * ENC_GROUPS * ENC_ROW];
    encode_groups(src, groups, lds, [&](size_t g, const float* half, bool second) {
        uint32_t sh, mh;
        double s, m;
        asym_header<15>(half, second, sh, mh, s, m);
        if (!second) {
            scales[g] = (uint16_t)sh;
            mins[g] = (uint16_t)mh;
        }
        bool unsure;
        const FastConst fk = fast_const(s, m, unsure);
        uint32_t* out = nibbles + g * 4 + (second ? 2 : 0);
#pragma unroll 1
        for (int k = 0; k < 2; ++k) {         // element 8 k + b of the half is nibble b of word k (low nibble = even)
            const f32x4_t a = row4(half, 2 * k), c = row4(half, 2 * k + 1);
            const float e[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
            uint32_t word = 0u;
#pragma unroll
            for (int b = 0; b < 8; ++b) word |= (uint32_t)code_fast<0, 15>(e[b], fk.r, fk.c, fk.er, fk.h0, unsure) << (4 * b);
            out[k] = word;
        }
        if (unsure || pair_u32(unsure)) {
#pragma unroll 1
            for (int k = 0; k < 2; ++k) {
                uint32_t word = 0u;
                for (int b = 0; b < 8; ++b)
                    word |= (uint32_t)code_exact((double)half[8 * k + b] - m, s, 0.0, 15.0) << (4 * b);
                out[k] = word;
            }
        }
    });
}

extern "C" __global__ __launch_bounds__(256) void brik_encode_q3(const f32x4_t* __restrict__ src,
                                                                 uint32_t* __restrict__ lo, uint32_t* __restrict__ hi,
                                                                 uint16_t* __restrict__ scales,
                                                                 uint16_t* __restrict__ mins, size_t groups)
{
    __shared__ __attribute__((aligned(16))) float lds[4 * ENC_GROUPS * ENC_ROW];
    encode_groups(src, groups, lds, [&](size_t g, const float* half, bool second) {
        uint32_t sh, mh;
        double s, m;
        asym_header<7>(half, second, sh, mh, s, m);
        if (!second) {
            scales[g] = (uint16_t)sh;
            mins[g] = (uint16_t)mh;
        }
        bool unsure;
        const FastConst fk = fast_const(s, m, unsure);
        // this half: lo word `second` (2 low bits each) and hi bits [16 second, 16 second + 16)
        uint32_t l = 0u, hb = 0u;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const f32x4_t w = row4(half, c);
            const float e[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t q = (uint32_t)code_fast<0, 7>(e[b], fk.r, fk.c, fk.er, fk.h0, unsure);
                l |= (q & 3u) << (2 * (4 * c + b));
                hb |= (q >> 2) << (4 * c + b);
            }
        }
        if (unsure || pair_u32(unsure)) {
            l = 0u;
            hb = 0u;
            for (int i = 0; i < 16; ++i) {
                const uint32_t q = (uint32_t)code_exact((double)half[i] - m, s, 0.0, 7.0);
                l |= (q & 3u) << (2 * i);
                hb |= (q >> 2) << i;
            }
        }
        lo[g * 2 + (second ? 1 : 0)] = l;
        const uint32_t other = pair_u32(hb);
        if (!second) hi[g] = hb | (other << 16);
    });
}

// f16 bits -> f32 as the reference's conversion path decodes an F16 tensor before quantizing it
// (f16ToF32, src/lib/webgpu/kernels.ts:3213-3222, applied by dequantizeToGpu at kernels.ts:798-803):
// the IEEE half value, subnormals included, except that exponent 31 (infinity and NaN) decodes to
// +-65504. Thread t converts elements [8 t, 8 t + 8); src and out are 16-byte aligned.
extern "C" __global__ __launch_bounds__(256) void brik_f16_decode(const uint16_t* __restrict__ src,
                                                                  float* __restrict__ out, size_t n)
{
    const size_t n8 = (n + 7) / 8;
    for (size_t t = (size_t)blockIdx.x * 256 + threadIdx.x; t < n8; t += (size_t)gridDim.x * 256) {
        const size_t i0 = t * 8;
        uint32_t h[8];
        if (i0 + 8 <= n) {
            const u32x4_t w = *reinterpret_cast<const u32x4_t*>(src + i0);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                h[2 * j] = ws[j] & 0xffffu;
                h[2 * j + 1] = ws[j] >> 16;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) h[j] = i0 + j < n ? src[i0 + j] : 0u;
        }
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool top = ((h[j] >> 10) & 0x1fu) == 0x1fu;
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)h[j]);
            v[j] = top ? ((h[j] & 0x8000u) ? -65504.f : 65504.f) : d;
        }
        if (i0 + 8 <= n) {
            f32x4_t* o = reinterpret_cast<f32x4_t*>(out + i0);
            o[0] = f32x4_t{v[0], v[1], v[2], v[3]};
            o[1] = f32x4_t{v[4], v[5], v[6], v[7]};
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (i0 + j < n) out[i0 + j] = v[j];
        }
    }
}
