// Prefill / grouped GEMM: y[M, N] = x[M, K] . deq(W[N, K])^T on CDNA4 matrix cores.
// Replaces the reference's tiled and shared-memory WGSL kernels (matmul_t_q4_tiled / _shared,
// matmul_t_q8_tiled / _shared, src/lib/webgpu/shaders.ts:120-168, 425-527, 531-577; and
// matmul_t_q3 for M > 1, :323-369), which run scalar f32 FMAs over 16x16 LDS tiles.
//
// Two launches:
//   1. brik_xprep_f16: each row of x is scaled by a power of two 2^(15 - e) (e = the binary exponent
//      of the row's largest |x|, so the scaled row fits binary16 whatever its magnitude), rounded to
//      f16 and written to a workspace row of Kp = roundup(K, 128) halves (zero padded), with the 8
//      elements of every aligned 8-group in the order [0 4 1 5 2 6 3 7]; rscale[m] = 2^(e - 15).
//   2. brik_gemm_<fmt>_<BM>x<TN>: 4 waves, block tile BM x 64 TN; each wave owns 16 TN columns over
//      all BM rows and runs v_mfma_f32_16x16x32_f16 (f32 accumulation). A K step is 128 (four
//      quantization groups). x goes through LDS (double buffered, shared by the 4 waves); W goes
//      straight from global memory into the MFMA B operand: each lane loads one whole group of one
//      column per fragment (16 bytes of q4), and dequantizes it in registers 8 codes at a time, just
//      before the MFMA that consumes them. The dequant is packed f16: a code q placed in the mantissa
//      of 1024.0h reads as 1024 + q (or 1024 + 16 q one nibble higher, which the scale s / 16
//      undoes), and one packed subtract and one packed FMA give the dequantized pair (q s + m); the
//      code pairs (j, j + 4) this produces from 8 packed codes fix the [0 4 1 5 2 6 3 7] order. The
//      epilogue multiplies by rscale[m] (exact) and stores y.
// f16 (not bf16) operands: 11-bit significands keep the normwise error near 3e-4, inside the 1e-3
// bar; bf16's 8 bits would not. The row scaling removes f16's range limit on activations.
//
// Dense mode (row_off == nullptr): a 1-D grid ordered so the M tiles of one N tile go to the same
// XCD (blocks are dealt to the 8 XCDs round-robin) and share its L2 for the weight tile. Grouped
// (MoE) mode: rows of x / y are sorted by expert; expert e owns rows [row_off[e], row_off[e+1]) and
// weight slice e of a stacked [E, N, K] q-tensor; blockIdx.y enumerates (expert, BM-row tile)
// pairs and blocks past the last pair exit.
#include "common.h"

namespace {

constexpr int XPREP_MAXC = 20;  // 8-float chunks per lane held in registers by the one-pass x staging

__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ uint32_t as_u32(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ float wave_max(float v)
{
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ float absmax8(f32x4_t a, f32x4_t b)
{
    // fmaxf drops NaN; rows whose largest magnitude is Inf keep scale 1
    return fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                 fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
}

__device__ __forceinline__ half8_t to_h8(f32x4_t a, f32x4_t b, float up)
{
    half8_t h;
    h[0] = (_Float16)(a.x * up); h[1] = (_Float16)(b.x * up);
    h[2] = (_Float16)(a.y * up); h[3] = (_Float16)(b.y * up);
    h[4] = (_Float16)(a.z * up); h[5] = (_Float16)(b.z * up);
    h[6] = (_Float16)(a.w * up); h[7] = (_Float16)(b.w * up);
    return h;
}

}  // namespace

// ---- 1. activation staging ----------------------------------------------------------------------

// One wave per row, four rows per block. Rows of up to 64 * XPREP_MAXC 8-float chunks are read once
// into registers; longer rows are read twice.
extern "C" __global__ __launch_bounds__(256) void brik_xprep_f16(const float* __restrict__ x,
                                                                 uint16_t* __restrict__ xh,
                                                                 float* __restrict__ rscale, int M, int K,
                                                                 int Kp)
{
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;     // a whole wave; no block-level synchronisation follows
    const int lane = threadIdx.x & 63;
    const float* xr = x + (size_t)m * K;
    uint16_t* hr = xh + (size_t)m * Kp;
    const int nch = K / 8, nchp = Kp / 8;
    auto scale_of = [&](float mx, float& up) {
        int e = 15;                                                    // zero / non-finite rows: scale 1
        if (mx > 0.f && mx <= 3.4028235e38f) (void)frexpf(mx, &e);    // mx = f * 2^e, f in [0.5, 1)
        up = ldexpf(1.f, 15 - e);
        if (lane == 0) rscale[m] = ldexpf(1.f, e - 15);
    };
    if (nchp <= 64 * XPREP_MAXC) {
        f32x4_t a[XPREP_MAXC], b[XPREP_MAXC];
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < XPREP_MAXC; ++i) {
            const int c = lane + 64 * i;
            a[i] = b[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if (c < nch) {
                a[i] = *(const f32x4_t*)(xr + c * 8);
                b[i] = *(const f32x4_t*)(xr + c * 8 + 4);
            }
        }
#pragma unroll
        for (int i = 0; i < XPREP_MAXC; ++i) mx = fmaxf(mx, absmax8(a[i], b[i]));
        float up;
        scale_of(wave_max(mx), up);
#pragma unroll
        for (int i = 0; i < XPREP_MAXC; ++i) {
            const int c = lane + 64 * i;
            if (c < nchp) *(half8_t*)(hr + c * 8) = to_h8(a[i], b[i], up);
        }
        return;
    }
    float mx = 0.f;
    for (int c = lane; c < nch; c += 64)
        mx = fmaxf(mx, absmax8(*(const f32x4_t*)(xr + c * 8), *(const f32x4_t*)(xr + c * 8 + 4)));
    float up;
    scale_of(wave_max(mx), up);
    for (int c = lane; c < nchp; c += 64) {
        f32x4_t a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
        if (c < nch) {
            a = *(const f32x4_t*)(xr + c * 8);
            b = *(const f32x4_t*)(xr + c * 8 + 4);
        }
        *(half8_t*)(hr + c * 8) = to_h8(a, b, up);
    }
}

// ---- 2. GEMM ------------------------------------------------------------------------------------

namespace {

constexpr int GK = 128;              // K per pipeline step: four quantization groups
constexpr int ALD = GK + 8;          // LDS row stride of the x tile in halves (272 bytes)

// Block tile: BM rows x 64 TN columns, 4 waves; wave c owns columns [16 TN c, 16 TN (c + 1)) of every
// BM row, so each W element of the block is loaded and dequantized by exactly one lane.
template <int BM_, int TN_>
struct Tile {
    static constexpr int BM = BM_, TN = TN_, TM = BM_ / 16;
    static constexpr int BN = 64 * TN_;
    static constexpr int NT = 256;
    static constexpr int XC = BM_ / 16;                   // 16-byte x chunks per thread per step
    static constexpr int A_BYTES = 2 * BM_ * ALD * 2;     // double-buffered x tile
    static constexpr int CLD = BN + 4;                    // epilogue staging row stride (floats)
    static constexpr int C_BYTES = 16 * CLD * 4;          // one 16-row fragment
    static constexpr int RF = (A_BYTES / C_BYTES) >= TM ? TM : (A_BYTES / C_BYTES) >= 4 ? 4
                            : (A_BYTES / C_BYTES) >= 2 ? 2 : 1;   // row fragments per epilogue round
    static constexpr int SMEM = A_BYTES > RF * C_BYTES ? A_BYTES : RF * C_BYTES;
    static_assert(BM_ % 16 == 0 && TN_ >= 1 && TM % RF == 0, "tile shape");
};

// Per lane and 16-column fragment: the codes of one group of one column.
// Words: q4 4 nibble dwords; q8 8 code dwords; q3 2 dwords of 2-bit fields + 1 dword of high bits.
template <int FMT>
struct WCodes {
    uint32_t w[FMT == FMT_Q8 ? 8 : FMT == FMT_Q4 ? 4 : 3];
};

// B-operand mapping (MFMA v_mfma_f32_16x16x32_f16, lane l: column l & 15, k slots 8 (l >> 4) + i):
// in step t, k-slice kk (0..3) and lane quarter q = l >> 4 hold the true K index
// 128 t + 32 q + 8 kk + i, so lane quarter q owns group 4 t + q whole: one load of its codes. The
// A operand (x, from LDS) uses the same mapping.
template <int FMT, int TN>
__device__ __forceinline__ void w_load(WCodes<FMT> (&f)[TN], const brsrc_t& p0, const brsrc_t& p1,
                                       const uint32_t (&colg)[TN], int step, int q, int G)
{
    // groups past the end are clamped in-bounds here and zeroed at the dequant
    const uint32_t g = (uint32_t)min(4 * step + q, G - 1);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const uint32_t gi = colg[j] + g;
        if constexpr (FMT == FMT_Q4) {
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(p0, gi * 16, 0, 0);
            f[j].w[0] = v.x; f[j].w[1] = v.y; f[j].w[2] = v.z; f[j].w[3] = v.w;
        } else if constexpr (FMT == FMT_Q8) {
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(p0, gi * 32, 0, 0);
            const u32x4_t u = __builtin_amdgcn_raw_buffer_load_b128(p0, gi * 32 + 16, 0, 0);
            f[j].w[0] = v.x; f[j].w[1] = v.y; f[j].w[2] = v.z; f[j].w[3] = v.w;
            f[j].w[4] = u.x; f[j].w[5] = u.y; f[j].w[6] = u.z; f[j].w[7] = u.w;
        } else {
            const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(p0, gi * 8, 0, 0);
            f[j].w[0] = v.x; f[j].w[1] = v.y;
            f[j].w[2] = __builtin_amdgcn_raw_buffer_load_b32(p1, gi * 4, 0, 0);
        }
    }
}

// Scales (and mins) of two steps: the 8 groups 8 u .. 8 u + 7 of each of the lane's columns, one
// 16-byte load per column shared by its four quarter lanes (one cache line per column every two
// steps instead of one per step). The window starts at any even byte offset (unaligned buffer
// loads are exact on this hardware) and is moved back to end inside the plane, `lim` being the
// last valid window start (plane groups - 8); sm_pick re-indexes. Groups past the row end are
// zeroed at the dequant.
template <int TN>
__device__ __forceinline__ void sm_load(u32x4_t (&v)[TN], const brsrc_t& r, const uint32_t (&colg)[TN], int u,
                                        uint32_t lim)
{
#pragma unroll
    for (int j = 0; j < TN; ++j)
        v[j] = __builtin_amdgcn_raw_buffer_load_b128(r, min(colg[j] + 8 * u, lim) * 2, 0, 0);
}

// f16 bits of group 8 u + 4 e + q of column group base cg from the window of pair u (e = 0 / 1: which
// step of the pair). For a live group the index into the window is 0..7.
__device__ __forceinline__ uint32_t sm_pick(const u32x4_t& v, uint32_t cg, int u, int e, int q, uint32_t lim)
{
    const uint32_t g = cg + 8 * u;
    const uint32_t k = g - min(g, lim) + 4 * e + q;
    const uint32_t d = k < 2 ? v.x : k < 4 ? v.y : k < 6 ? v.z : v.w;
    return (d >> (16 * (k & 1))) & 0xffffu;
}

// Dequantize 8 codes to 4 packed f16 pairs (codes j and j + 4 in pair j).
// q4: the low nibble of each byte lands on the mantissa units, the high nibble 16 units up.
__device__ __forceinline__ u32x4_t deq8_q4(uint32_t w, half2_t s2, half2_t s2_16, half2_t m2)
{
    const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
    const uint32_t w8 = w >> 8;
    u32x4_t r;
    r[0] = as_u32(__builtin_elementwise_fma(as_h2((w & 0x000F000Fu) | 0x64006400u) - k1024, s2, m2));
    r[1] = as_u32(__builtin_elementwise_fma(as_h2((w & 0x00F000F0u) | 0x64006400u) - k1024, s2_16, m2));
    r[2] = as_u32(__builtin_elementwise_fma(as_h2((w8 & 0x000F000Fu) | 0x64006400u) - k1024, s2, m2));
    r[3] = as_u32(__builtin_elementwise_fma(as_h2((w8 & 0x00F000F0u) | 0x64006400u) - k1024, s2_16, m2));
    return r;
}

// q3: `lo16` 8 two-bit fields, `hi8` their high bits.
__device__ __forceinline__ u32x4_t deq8_q3(uint32_t lo16, uint32_t hi8, half2_t s2, half2_t m2)
{
    const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
    // code j sits at bits 2j of L and code j + 4 at bits 16 + 2j; high bits likewise at 2 + j, 18 + j of H
    const uint32_t L = lo16 | (lo16 << 8), H = (hi8 << 2) | (hi8 << 14);
    u32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = ((L >> (2 * j)) & 0x00030003u) | ((H >> j) & 0x00040004u) | 0x64006400u;
        r[j] = as_u32(__builtin_elementwise_fma(as_h2(c) - k1024, s2, m2));
    }
    return r;
}

// q8: bytes of w (codes 0..3) and w2 (codes 4..7).
__device__ __forceinline__ u32x4_t deq8_q8(uint32_t w, uint32_t w2, half2_t s2)
{
    const half2_t k1152 = {(_Float16)1152.f, (_Float16)1152.f};
    w ^= 0x80808080u;        // int8 -> int8 + 128
    w2 ^= 0x80808080u;
    u32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // byte j of w -> low half, byte j of w2 -> high half, zero bytes above each
        const uint32_t c = __builtin_amdgcn_perm(w2, w, (0x0cu << 24) | ((4u + j) << 16) | (0x0cu << 8) | j);
        r[j] = as_u32((as_h2(c | 0x64006400u) - k1152) * s2);
    }
    return r;
}

// B operand of k-slice kk from one lane's group: codes 8 kk .. 8 kk + 7, scale / min bits s, m.
template <int FMT>
__device__ __forceinline__ half8_t b_frag(const WCodes<FMT>& f, int kk, _Float16 s, _Float16 m)
{
    const half2_t s2 = {s, s}, m2 = {m, m};
    u32x4_t o;
    if constexpr (FMT == FMT_Q4) {
        const _Float16 s16 = s * (_Float16)0.0625f;     // exact for normal scales >= 2^-10
        o = deq8_q4(f.w[kk], s2, half2_t{s16, s16}, m2);
    } else if constexpr (FMT == FMT_Q8) {
        o = deq8_q8(f.w[2 * kk], f.w[2 * kk + 1], s2);
    } else {
        o = deq8_q3((f.w[kk >> 1] >> (16 * (kk & 1))) & 0xffffu, (f.w[2] >> (8 * kk)) & 0xffu, s2, m2);
    }
    return __builtin_bit_cast(half8_t, o);
}

// LDS-only barrier: orders LDS traffic across the block without waiting for global loads in flight.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int FMT, class T>
__device__ __forceinline__ void mma_step(const _Float16* A, const WCodes<FMT> (&wc)[T::TN],
                                         const u32x4_t (&sv)[T::TN], const u32x4_t (&mv)[T::TN],
                                         const uint32_t (&sg)[T::TN], uint32_t lim, floatx4_t (&acc)[T::TM][T::TN],
                                         int t, int lane, int q, int G)
{
    constexpr int TM = T::TM, TN = T::TN;
    const bool live = 4 * t + q < G;
    _Float16 s[TN], m[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const uint32_t sb = sm_pick(sv[j], sg[j], t >> 1, t & 1, q, lim);
        const uint32_t mb = FMT != FMT_Q8 ? sm_pick(mv[j], sg[j], t >> 1, t & 1, q, lim) : 0u;
        s[j] = live ? __builtin_bit_cast(_Float16, (uint16_t)sb) : (_Float16)0.f;
        m[j] = (FMT != FMT_Q8 && live) ? __builtin_bit_cast(_Float16, (uint16_t)mb) : (_Float16)0.f;
    }
    // k-slice kk + 1 is dequantized while the MFMAs of k-slice kk run: the scheduling groups below
    // interleave one MFMA with two VALU instructions
    half8_t b[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) b[j] = b_frag<FMT>(wc[j], 0, s[j], m[j]);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        half8_t a[TM], bn[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            a[i] = *(const half8_t*)(A + (i * 16 + (lane & 15)) * ALD + 32 * q + 8 * kk);
        if (kk < 3) {
#pragma unroll
            for (int j = 0; j < TN; ++j) bn[j] = b_frag<FMT>(wc[j], kk + 1, s[j], m[j]);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, TM, 0);       // the A fragment reads first
#pragma unroll
        for (int g = 0; g < TM * TN; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);    // two VALU
        }
        if (kk < 3) {
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = bn[j];
        }
    }
}

template <int FMT, class T>
__device__ __forceinline__ void gemm_body(const uint16_t* __restrict__ xh, const float* __restrict__ rscale,
                                          const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,
                                          const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn,
                                          float* __restrict__ y, int M, int K, int N,
                                          const int* __restrict__ row_off, int E)
{
    constexpr int BM = T::BM, BN = T::BN, TM = T::TM, TN = T::TN, XC = T::XC, NT = T::NT;
    __shared__ __attribute__((aligned(16))) unsigned char smem[T::SMEM];
    _Float16* const As0 = reinterpret_cast<_Float16*>(smem);
    _Float16* const As1 = As0 + BM * ALD;

    const int G = K / BRIK_GROUP;
    const int Kp = (K + 2 * GK - 1) / (2 * GK) * (2 * GK);
    const int steps = Kp / GK;                 // even, >= 2
    int m0, m_end = M, n0, e = 0;

    if (row_off) {
        n0 = blockIdx.x * BN;
        int remaining = blockIdx.y;
        for (; e < E; ++e) {
            const int cnt = row_off[e + 1] - row_off[e];
            const int tiles = (cnt + BM - 1) / BM;
            if (remaining < tiles) break;
            remaining -= tiles;
        }
        if (e >= E) return;     // uniform across the block, before any barrier
        m0 = row_off[e] + remaining * BM;
        m_end = min(row_off[e + 1], M);     // a malformed table cannot push stores past row M
        if (m0 < 0 || m0 >= m_end) return;
    } else {
        const int nMT = (M + BM - 1) / BM, nNT = (N + BN - 1) / BN;
        const int b = blockIdx.x, gsz = 8 * nMT;
        const int grp = b / gsz, full = nNT / 8;
        int mt, nt;
        if (grp < full) {
            const int w = b - grp * gsz;
            nt = grp * 8 + (w & 7);
            mt = w >> 3;
        } else {
            const int w = b - full * gsz;
            nt = full * 8 + w / nMT;
            mt = w % nMT;
        }
        m0 = mt * BM;
        n0 = nt * BN;
    }

    // buffer resources: the staged x rows of this launch; the W planes of this matrix (expert slice)
    const size_t wel = (size_t)N * K;          // elements of one weight matrix
    const size_t gbase = (size_t)e * N * G;    // flat group offset of the expert slice
    const brsrc_t rx = make_rsrc(xh, (uint32_t)((size_t)M * Kp * 2));
    brsrc_t r0, r1 = rx, rsc, rmn = rx;
    if constexpr (FMT == FMT_Q8) {
        r0 = make_rsrc(p0 + (size_t)e * wel, (uint32_t)wel);
    } else if constexpr (FMT == FMT_Q4) {
        r0 = make_rsrc(p0 + (size_t)e * wel / 2, (uint32_t)(wel / 2));
    } else {
        r0 = make_rsrc(p0 + (size_t)e * wel / 4, (uint32_t)(wel / 4));
        r1 = make_rsrc(p1 + (size_t)e * wel / 8, (uint32_t)(wel / 8));
    }
    // scales and mins: one resource over the whole (stacked) plane, so scale windows of one expert
    // may extend into the next; lim = last window start that ends inside the plane (the host routes
    // planes of fewer than 8 groups elsewhere)
    const uint32_t sgroups = (uint32_t)((size_t)(row_off ? E : 1) * N * G);
    const uint32_t lim = sgroups - 8;
    rsc = make_rsrc(sc, sgroups * 2);
    if constexpr (FMT != FMT_Q8) rmn = make_rsrc(mn, sgroups * 2);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, q = lane >> 4;
    // x staging: chunk c = tid + 256 i is row c / 16, 16-byte part c % 16 of the step's 256-byte row slice
    uint32_t xoff[XC];
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const int c = tid + NT * i;
        const int m = min(m0 + (c >> 4), m_end - 1);      // rows past the tile's end repeat a live row
        xoff[i] = (uint32_t)(m * Kp + (c & 15) * 8) * 2;
    }
    // W: flat group index of this lane's column in fragment j, at group 0
    const int wn = wave * 16 * TN;
    uint32_t colg[TN], sg[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        colg[j] = (uint32_t)(min(n0 + wn + 16 * j + (lane & 15), N - 1) * G);
        sg[j] = (uint32_t)gbase + colg[j];         // the same group in the whole scale plane
    }

    floatx4_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    // Prologue: step 0 of x into LDS buffer 0, step 0 of W and the scales of steps 0 and 1 into
    // registers.
    u32x4_t xs[XC];
    WCodes<FMT> wc[TN], wn_[TN];
    u32x4_t sv[TN], mv[TN] = {};
#pragma unroll
    for (int i = 0; i < XC; ++i) xs[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, xoff[i], 0, 0);
    w_load<FMT, TN>(wc, r0, r1, colg, 0, q, G);
    sm_load<TN>(sv, rsc, sg, 0, lim);
    if constexpr (FMT != FMT_Q8) sm_load<TN>(mv, rmn, sg, 0, lim);
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const int c = tid + NT * i;
        *(u32x4_t*)(As0 + (c >> 4) * ALD + (c & 15) * 8) = xs[i];
    }
    lds_barrier();

    // Steps in pairs (t, t + 1). Step t: issue the loads of step t + 1 (x to registers, W to the next
    // fragment set), multiply step t (x from LDS buffer t & 1, W dequantized from registers one
    // k-slice at a time), then store x of step t + 1 to the other LDS buffer. The scales of a pair
    // arrive with the first step's loads of the previous pair. The last step's extra loads are
    // clamped.
    u32x4_t svn[TN], mvn[TN] = {};
    for (int t = 0; t < steps; t += 2) {
        // -- step t
#pragma unroll
        for (int i = 0; i < XC; ++i) xs[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, xoff[i], (t + 1) * (GK * 2), 0);
        w_load<FMT, TN>(wn_, r0, r1, colg, t + 1, q, G);
        const int un = min(t / 2 + 1, steps / 2 - 1);
        sm_load<TN>(svn, rsc, sg, un, lim);
        if constexpr (FMT != FMT_Q8) sm_load<TN>(mvn, rmn, sg, un, lim);
        __builtin_amdgcn_sched_barrier(0);     // keep the loads ahead of the multiplies
        mma_step<FMT, T>(As0, wc, sv, mv, sg, lim, acc, t, lane, q, G);
#pragma unroll
        for (int i = 0; i < XC; ++i) {
            const int c = tid + NT * i;
            *(u32x4_t*)(As1 + (c >> 4) * ALD + (c & 15) * 8) = xs[i];
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) wc[j] = wn_[j];
        lds_barrier();

        // -- step t + 1
        const int tn = min(t + 2, steps - 1);
#pragma unroll
        for (int i = 0; i < XC; ++i) xs[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, xoff[i], tn * (GK * 2), 0);
        w_load<FMT, TN>(wn_, r0, r1, colg, tn, q, G);
        __builtin_amdgcn_sched_barrier(0);
        mma_step<FMT, T>(As1, wc, sv, mv, sg, lim, acc, t + 1, lane, q, G);
#pragma unroll
        for (int i = 0; i < XC; ++i) {
            const int c = tid + NT * i;
            *(u32x4_t*)(As0 + (c >> 4) * ALD + (c & 15) * 8) = xs[i];
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            wc[j] = wn_[j];
            sv[j] = svn[j];
            mv[j] = mvn[j];
        }
        lds_barrier();
    }

    // Epilogue, RF row fragments per round: the accumulators are staged in LDS (D layout of a 16x16
    // tile: lane holds column lane & 15, rows 4 q + r), then every thread scales 4 consecutive
    // columns of one row by rscale and stores them with one 16-byte store (N % 4 == 0) or four
    // 4-byte stores.
    float* const Cs = reinterpret_cast<float*>(smem);
    constexpr int CH = BN / 4;                      // 4-column chunks per row
#pragma unroll
    for (int i0 = 0; i0 < TM; i0 += T::RF) {
        if (i0) lds_barrier();                      // the previous round's reads are done
#pragma unroll
        for (int ii = 0; ii < T::RF; ++ii)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    Cs[(ii * 16 + 4 * q + r) * T::CLD + wn + 16 * j + (lane & 15)] = acc[i0 + ii][j][r];
        lds_barrier();
        for (int c = tid; c < T::RF * 16 * CH; c += NT) {
            const int row = c / CH, col = (c % CH) * 4;
            const int m = m0 + i0 * 16 + row, n = n0 + col;
            if (m >= m_end || n >= N) continue;
            const f32x4_t v = *(const f32x4_t*)(Cs + row * T::CLD + col) * rscale[m];
            float* dst = y + (size_t)m * N + n;
            if ((N & 3) == 0) {
                *(f32x4_t*)dst = v;
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (n + k < N) dst[k] = v[k];
            }
        }
    }
}

}  // namespace

// Kernel names: brik_gemm_<fmt>_<BM>x<TN> (block tile BM x 64 TN), 256 threads (4 waves) each; the
// runtime picks the tile.
#define BRIK_GEMM(FMTN, FMT, BM_, TN_)                                                                    \
    extern "C" __global__ __launch_bounds__(256) void brik_gemm_##FMTN##_##BM_##x##TN_(                   \
        const uint16_t* __restrict__ xh, const float* __restrict__ rscale, const uint8_t* __restrict__ p0, \
        const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, \
        float* __restrict__ y, int M, int K, int N, const int* __restrict__ row_off, int E)               \
    {                                                                                                     \
        gemm_body<FMT, Tile<BM_, TN_>>(xh, rscale, p0, p1, sc, mn, y, M, K, N, row_off, E);               \
    }

// Tiles in the order of the runtime's table: (BM, TN).
#define BRIK_GEMM_FMT(FMTN, FMT)                                                       \
    BRIK_GEMM(FMTN, FMT, 128, 3) BRIK_GEMM(FMTN, FMT, 128, 2) BRIK_GEMM(FMTN, FMT, 128, 4) \
    BRIK_GEMM(FMTN, FMT, 64, 3) BRIK_GEMM(FMTN, FMT, 64, 2) BRIK_GEMM(FMTN, FMT, 64, 4)    \
    BRIK_GEMM(FMTN, FMT, 32, 3) BRIK_GEMM(FMTN, FMT, 32, 2) BRIK_GEMM(FMTN, FMT, 32, 4)

BRIK_GEMM_FMT(q4, FMT_Q4)
BRIK_GEMM_FMT(q8, FMT_Q8)
BRIK_GEMM_FMT(q3, FMT_Q3)
