// Prefill / grouped GEMM: y[M, N] = x[M, K] . deq(W[N, K])^T on CDNA4 matrix cores.
// Replaces the reference's tiled and shared-memory WGSL kernels (matmul_t_q4_tiled / _shared,
// matmul_t_q8_tiled / _shared, src/lib/webgpu/shaders.ts:120-168, 425-527, 531-577; and
// matmul_t_q3 for M > 1, :323-369), which run scalar f32 FMAs over 16x16 LDS tiles.
//
// Two launches:
//   1. brik_xprep_f16: each row of x is scaled by a power of two 2^(15 - e) (e = the binary exponent
//      of the row's largest |x|, so the scaled row fits binary16 whatever its magnitude), rounded to
//      f16 and written to a workspace row of Kp = roundup(K, 256) halves (zero padded), with the 8
//      elements of every aligned 8-group in the order [0 4 1 5 2 6 3 7]; rscale[m] = 2^(e - 15).
//   2. brik_gemm_<fmt>_<BM>x<TN>[w8]: 4 (or 8) waves, block tile BM x 32 TN NW; each wave owns 32 TN
//      columns over all BM rows and runs v_mfma_f32_32x32x16_f16 (f32 accumulation), which issues at
//      full rate from one wave per SIMD and hides about six VALU instructions of the same wave beside
//      each MFMA; with 8 waves two share each SIMD. A K
//      step is 128 (four quantization groups, 8 MFMA slices of 16). x goes through LDS: PF + 2
//      buffers filled PF + 1 steps ahead by direct global->LDS loads, XOR-swizzled so that the
//      A-fragment reads are free of bank conflicts. W goes straight from global memory into the MFMA B
//      operand: each lane loads two whole groups of one column per step, PF steps ahead (PF = 1 for the
//      dense tiles, more for the latency-bound few-row tiles), and dequantizes them in registers 8
//      codes at a time, one slice ahead of the MFMAs that consume them. The dequant is packed f16: a
//      low nibble q placed in the mantissa of 1024.0h reads as 1024 + q, and a high nibble left in
//      place (bits 4-7) in the mantissa of 64.0h reads as 64 + q; one packed subtract and one packed
//      FMA then give the dequantized pair (q s + m), rounded once to f16 whatever the scale; the
//      code pairs (j, j + 4) this produces from 8 packed codes fix the
//      [0 4 1 5 2 6 3 7] order. Scales and mins are staged in LDS a few steps at a time by coalesced
//      loads. The epilogue multiplies by rscale[m] (exact, staged in LDS at the prologue) and stores y
//      straight from the accumulator registers (the transposed convolution store goes through LDS).
// f16 (not bf16) operands: 11-bit significands keep the normwise error near 3e-4, inside the 1e-3
// bar; with bf16's 8 bits the same products measure 2e-3 to 3e-3 (tests/test_operand_precision.py).
// The row scaling removes f16's range limit on activations.
//
// Dense kernels (brik_gemm_*): a 1-D grid ordered so the M tiles of one N tile go to the same XCD
// (blocks are dealt to the 8 XCDs round-robin) and share its L2 for the weight tile. Grouped (MoE)
// kernels (brik_gemmg_q4_*): rows of x / y are sorted by expert; expert e owns rows
// [row_off[e], row_off[e+1]) and weight slice e of a stacked [E, N, K] q-tensor; blockIdx.y enumerates
// (expert, BM-row tile) pairs, blocks past the last pair exit, and blockIdx.z picks one of two weight
// tensors multiplied by the same rows.
#include "common.h"

namespace {


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

// One 256-thread block per row, a grid of at most 65536 blocks looping over the rows (a launch of few
// rows still fills the CUs: the 512 rows of the prefill shape are 512 blocks, against 128 of one wave
// per row, which ran 6.2 us for 7.9 MB). Rows of up to 256 * XPREP_BCH 8-float chunks are read once
// into registers; longer rows are read twice. Rows of at most XPREP_WAVE_KP staged elements run one
// wave per row instead (four rows per block, CH = 2 or 4 chunks per lane, the maximum a wave
// reduction with no barrier): a 256-thread block on a 768-element row left 160 threads idle (MoE
// step 83.7-84.0 -> 81.2-82.8 us with the gate / up and down rows staged this way). The runtime
// sizes the grid by the same rule. The row maximum is exact in any order, so the output does not
// depend on how the row is split.
constexpr int XPREP_BCH = 4;
constexpr int XPREP_WAVE_KP = 2048;

// The power-of-two scale that fits a row of largest magnitude mx into f16: up = 2^(15 - e) multiplies
// the row, the row's rscale 2^(e - 15) undoes it (zero and non-finite maxima: scale 1).
__device__ __forceinline__ float xprep_up(float mx, float& down)
{
    int e = 15;
    if (mx > 0.f && mx <= 3.4028235e38f) (void)frexpf(mx, &e);    // mx = f * 2^e, f in [0.5, 1)
    down = ldexpf(1.f, e - 15);
    return ldexpf(1.f, 15 - e);
}

template <int CH>
__device__ __forceinline__ void xprep_row_wave(const float* __restrict__ x, uint16_t* __restrict__ xh,
                                               float* __restrict__ rscale, int m, int K, int Kp)
{
    const int lane = threadIdx.x & 63;
    const float* xr = x + (size_t)m * K;
    uint16_t* hr = xh + (size_t)m * Kp;
    const int nch = K / 8, nchp = Kp / 8;
    f32x4_t a[CH], b[CH];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int c = lane + 64 * i;
        a[i] = b[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if (c < nch) {
            a[i] = *(const f32x4_t*)(xr + c * 8);
            b[i] = *(const f32x4_t*)(xr + c * 8 + 4);
        }
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) mx = fmaxf(mx, absmax8(a[i], b[i]));
    mx = wave_max(mx);
    float down;
    const float up = xprep_up(mx, down);
    if (lane == 0) rscale[m] = down;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int c = lane + 64 * i;
        if (c < nchp) *(half8_t*)(hr + c * 8) = to_h8(a[i], b[i], up);
    }
}

__device__ __forceinline__ void xprep_row(const float* __restrict__ x, uint16_t* __restrict__ xh,
                                          float* __restrict__ rscale, int m, int K, int Kp, float* wmax)
{
    const int tid = threadIdx.x;
    const float* xr = x + (size_t)m * K;
    uint16_t* hr = xh + (size_t)m * Kp;
    const int nch = K / 8, nchp = Kp / 8;
    // the block's maximum of the threads' mx, then the power-of-two scale that fits the row into f16
    // (the barrier after the reads of wmax keeps the next row's writes behind them)
    auto scale_of = [&](float mx, float& up) {
        mx = wave_max(mx);
        if ((tid & 63) == 0) wmax[tid >> 6] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
        __syncthreads();
        float down;
        up = xprep_up(mx, down);
        if (tid == 0) rscale[m] = down;
    };
    if (nchp <= 256 * XPREP_BCH) {
        f32x4_t a[XPREP_BCH], b[XPREP_BCH];
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < XPREP_BCH; ++i) {
            const int c = tid + 256 * i;
            a[i] = b[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if (c < nch) {
                a[i] = *(const f32x4_t*)(xr + c * 8);
                b[i] = *(const f32x4_t*)(xr + c * 8 + 4);
            }
        }
#pragma unroll
        for (int i = 0; i < XPREP_BCH; ++i) mx = fmaxf(mx, absmax8(a[i], b[i]));
        float up;
        scale_of(mx, up);
#pragma unroll
        for (int i = 0; i < XPREP_BCH; ++i) {
            const int c = tid + 256 * i;
            if (c < nchp) *(half8_t*)(hr + c * 8) = to_h8(a[i], b[i], up);
        }
        return;
    }
    float mx = 0.f;
    for (int c = tid; c < nch; c += 256)
        mx = fmaxf(mx, absmax8(*(const f32x4_t*)(xr + c * 8), *(const f32x4_t*)(xr + c * 8 + 4)));
    float up;
    scale_of(mx, up);
    for (int c = tid; c < nchp; c += 256) {
        f32x4_t a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
        if (c < nch) {
            a = *(const f32x4_t*)(xr + c * 8);
            b = *(const f32x4_t*)(xr + c * 8 + 4);
        }
        *(half8_t*)(hr + c * 8) = to_h8(a, b, up);
    }
}

extern "C" __global__ __launch_bounds__(256) void brik_xprep_f16(const float* __restrict__ x,
                                                                 uint16_t* __restrict__ xh,
                                                                 float* __restrict__ rscale, int M, int K,
                                                                 int Kp)
{
    __shared__ float wmax[4];
    if (Kp <= 1024) {
        for (int m = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6); m < M; m += (int)gridDim.x * 4)
            xprep_row_wave<2>(x, xh, rscale, m, K, Kp);
        return;
    }
    if (Kp <= XPREP_WAVE_KP) {
        for (int m = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6); m < M; m += (int)gridDim.x * 4)
            xprep_row_wave<4>(x, xh, rscale, m, K, Kp);
        return;
    }
    for (int m = blockIdx.x; m < M; m += gridDim.x)     // the same for the whole block
        xprep_row(x, xh, rscale, m, K, Kp, wmax);
}

// ---- 2. GEMM ------------------------------------------------------------------------------------

namespace {

constexpr int GK = 128;              // K per pipeline step: four quantization groups
constexpr int XROW = GK * 2;         // bytes of one x row per step in LDS (16 chunks of 16 bytes)

// The expert and rows of pair y of an expert-grouped launch, whose pairs are the BM-row tiles of
// experts 0, 1, ... in order. Wave 0 reads row_off 64 experts at a time (one per lane, vector loads),
// scans the tile counts across the wave and publishes the expert that holds pair y through LDS: a few
// dozen instructions and one memory round trip, where walking the experts one by one costs a dependent
// scalar load per expert. Every thread of the block calls it (it ends with a barrier). Returns false,
// for the whole block, when y is past the last pair; offsets that decrease count as empty experts and
// rows are clipped to M, so a malformed table cannot send stores past row M.
template <int BM>
__device__ __forceinline__ bool find_expert_tile(const int* __restrict__ row_off, int E, int y, int M, int& e,
                                                 int& m0, int& m_end)
{
    __shared__ int res[3];
    if (threadIdx.x < 64) {
        const int lane = (int)threadIdx.x;
        int carry = 0, found = -1, fm0 = 0, fend = 0;
        for (int base = 0; base < E && found < 0; base += 64) {     // uniform across wave 0
            const int ex = base + lane;
            int lo = 0, hi = 0, tiles = 0;
            if (ex < E) {
                lo = row_off[ex];
                hi = row_off[ex + 1];
                tiles = hi > lo ? (hi - lo + BM - 1) / BM : 0;
            }
            int incl = tiles;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int v = __shfl_up(incl, o, 64);
                if (lane >= o) incl += v;
            }
            incl += carry;
            const int excl = incl - tiles;
            const unsigned long long own = __ballot(ex < E && y >= excl && y < incl);
            if (own) {
                const int src = __ffsll((long long)own) - 1;
                found = __shfl(ex, src, 64);
                fm0 = __shfl(lo + (y - excl) * BM, src, 64);
                fend = __shfl(min(hi, M), src, 64);
            }
            carry = __shfl(incl, 63, 64);
        }
        if (lane == 0) {
            res[0] = found;
            res[1] = fm0;
            res[2] = fend;
        }
    }
    __syncthreads();
    // block-uniform values read from LDS land in VGPRs: move them to scalar registers, or every buffer
    // resource built from them would be a per-lane value (a waterfall loop around each buffer load)
    e = __builtin_amdgcn_readfirstlane(res[0]);
    m0 = __builtin_amdgcn_readfirstlane(res[1]);
    m_end = __builtin_amdgcn_readfirstlane(res[2]);
    return e >= 0 && m0 >= 0 && m0 < m_end;
}

// Block tile: BM rows x 32 TN NW columns, NW waves (4: one per SIMD, 8: two per SIMD); wave w owns
// columns [32 TN w, 32 TN (w + 1)) of all BM rows as TM = BM / 32 row blocks x TN column blocks of
// v_mfma_f32_32x32x16_f16, so each W element of the block is loaded and dequantized by exactly one
// lane, and the dequantization of one 16-k slice of a column block feeds TM MFMAs. The 32x32x16 MFMA
// (32 cycles) issues at full rate from a single wave and leaves room for about six VALU instructions
// of the same wave beside each one, which is what the dequantization needs at TM = 4.
// x steps go through PF + 2 LDS buffers of BM rows x 256 bytes, filled by direct global->LDS loads
// PF + 1 steps ahead (PF below). The 16-byte chunk c of row r sits at position c ^ (r & 15) of the row, so the 16 rows
// that one 16-lane phase of an A-fragment read touches hit 16 different bank groups.
// Scales and mins go through LDS too, a chunk of SCH steps (SG groups, 2 SG bytes of each column) at
// a time, double buffered: the block loads them with coalesced 16-byte-per-lane global->LDS loads
// instead of every lane fetching its own 2-byte values from a different cache line.
// PF: how many steps ahead the W codes are loaded (a register ring of PF + 1 steps); the x buffers
// then number PF + 2, filled PF + 1 steps ahead. Loads complete in issue order, so waiting for the x
// of the next step also waits for every W load issued before it: W runs PF steps ahead only when x
// runs further ahead still. A launch of few blocks (few rows per expert, small M) is bound by the
// memory latency of each step, and PF > 1 keeps several steps of W in flight; a launch of many blocks
// per CU (the dense prefill) hides the latency across blocks and keeps PF = 1.
template <int FMT, int BM_, int TN_, int NW_ = 4, int PF_ = 1>
struct Tile {
    static constexpr int BM = BM_, TN = TN_, TM = BM_ / 32, NW = NW_, PF = PF_;
    static constexpr int BN = 32 * TN_ * NW_;
    static constexpr int NT = 64 * NW_;
    static constexpr int XI = BM_ / (4 * NW_);           // 16-byte x chunks per thread per step
    static constexpr int XBUF = BM_ * XROW;               // one x buffer
    static constexpr int XQ = PF_ + 2;                    // x buffers
    static constexpr int A_BYTES = XQ * XBUF;
    static constexpr int PLANES = FMT == FMT_Q8 ? 1 : FMT == FMT_F16 ? 0 : 2;  // scales (and mins); f16 has none
    // scale chunks: SG groups (SCH = SG / 4 steps) of every column of the block, SG * 2 bytes per column
    // and plane; loaded 16 bytes per lane, LPC lanes per column. A chunk loaded at the first step of the
    // previous chunk must have landed when the last step of that chunk reads it, SCH - 1 steps later:
    // the wait of a step covers the loads issued PF steps before it, so SCH >= PF + 1. Small chunks
    // keep the LDS of a block small (two blocks of the 64-row 8-wave tile fit a CU with SG = 8).
    // The chunk is also a whole number of 1024-byte load instructions per wave.
    static constexpr bool sg_fits(int sg) { return sg / 4 >= PF_ + 1 && (PLANES * BN * sg * 2) % (NW_ * 1024) == 0; }
    static constexpr int SG = sg_fits(8) ? 8 : sg_fits(16) ? 16 : 32, SCH = SG / 4, LPC = SG / 8;
    static constexpr int SPLANE = BN * SG * 2;            // one plane of one scale chunk
    static constexpr int SBUF = PLANES * SPLANE;          // one scale chunk
    static constexpr int NSD = PLANES * SPLANE / 1024 / NW_;   // scale-chunk load instructions per wave
    static constexpr int S_OFF = A_BYTES;                 // scale chunks follow the x buffers
    static constexpr int CLD = BN + 4;                    // transposed-store staging row stride (floats)
    static constexpr int C_BYTES = 32 * CLD * 4;          // one 32-row block
    static constexpr int RF = (A_BYTES / C_BYTES) >= TM ? TM : (A_BYTES / C_BYTES) >= 2 && TM % 2 == 0 ? 2 : 1;
    static constexpr int MAIN = A_BYTES + 2 * SBUF + 64;  // + a pad for reads of dead groups
    static constexpr int RS_OFF = MAIN;                   // the tile's row scales (BM floats)
    static constexpr int SMEM = MAIN + 4 * BM_ > RF * C_BYTES ? MAIN + 4 * BM_ : RF * C_BYTES;
    // vector-memory loads per step: W codes, then the x chunks
    static constexpr int W_OPS = (FMT == FMT_Q4 ? 2 : FMT == FMT_F16 ? 8 : 4) * TN_;
    // loads a wave may still have in flight once the x of the next step has landed: the W and x of the
    // PF - 1 steps issued after it, and the W of the current step
    static constexpr int VM_NEXT_X = (PF_ - 1) * (W_OPS + XI) + W_OPS;
    static_assert(BM_ % 32 == 0 && TN_ >= 1 && (NW_ == 4 || NW_ == 8) && BM_ % (4 * NW_) == 0 && TM % RF == 0 &&
                  SCH >= PF_ + 1 && NSD * NW_ * 1024 == PLANES * SPLANE &&
                  SMEM <= 160 * 1024 && PF_ >= 1 && VM_NEXT_X < 64 && XI + (PF_ - 1) * (W_OPS + XI) < 64,
                  "tile shape");
};

// K mapping of a step (128 k = 8 slices of 16, one MFMA each): lane half h = lane >> 5, slice s and
// element i hold the true K index 128 t + 64 h + 8 s + i. A lane half therefore owns groups 4 t + 2 h
// and 4 t + 2 h + 1 of its column whole (slices 0-3 and 4-7), and one load brings each group's codes.
// A (x from LDS) and B (W) use the same mapping, so the order of the contraction does not matter.
// f16 weights use 128 t + 16 s + 8 h + i instead: their loads are not per group, and this mapping
// makes the two lane halves of a load read adjacent pieces of a weight row.

// Per lane and 32-column block: the codes of two groups of one column, and their f16 scale and min
// bits (one group per register, low half). Words: q4 2 x 4 nibble dwords; q8 2 x 8 code dwords; q3
// 2 x 2 dwords of 2-bit fields, then 2 dwords of high bits (one byte per 8 codes); f16 2 x 16 dwords of
// halves in k order.
template <int FMT>
struct WCodes {
    uint32_t w[FMT == FMT_F16 ? 32 : FMT == FMT_Q8 ? 16 : FMT == FMT_Q4 ? 8 : 6];
    uint32_t s[2], m[2];
};

typedef __attribute__((address_space(3))) void lds_void_t;

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// The multiply loop's LDS reads are inline asm. The compiler treats every direct global->LDS load
// as a write to LDS of unknown extent, and before any LDS read it emits while such a load may be in
// flight it waits for the load, that is for every memory load issued before it as well (the W
// prefetch of the following steps included): a full memory round trip per K step. The pipeline
// already orders its LDS reads against the direct loads that fill the same buffers (wait_vm before
// each step barrier), so these reads are issued as asm, invisible to that rule, and their completion
// is waited for explicitly: lds_wait, then tie on every value read, which orders its uses after the
// wait.
// OFF is the instruction's 16-bit immediate offset: reads at fixed distances from one base take no
// address arithmetic of their own.
template <int OFF = 0>
__device__ __forceinline__ half8_t ds_read_b128(uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    half8_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
template <int OFF = 0>
__device__ __forceinline__ uint32_t ds_read_u16(uint32_t addr)
{
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
// The A fragments of one slice: row block i at base + i * 32 rows.
template <int TM, int I = 0>
__device__ __forceinline__ void read_a(half8_t (&a)[TM], uint32_t base)
{
    if constexpr (I < TM) {
        a[I] = ds_read_b128<I * 32 * XROW>(base);
        read_a<TM, I + 1>(a, base);
    }
}
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)"); }
template <class V>
__device__ __forceinline__ void tie(V& v)
{
    asm volatile("" : "+v"(v));
}

// The loads of one step, split into ops that the multiply loop spreads over its slices: for each
// column block the code loads of W step t + 1, in slices 0-1; then, after the barrier in slice 4, the
// direct global->LDS loads of x step t + 2 (instruction i of wave w fills bytes [1024 (NW i + w), +1024)
// of the buffer, 16 bytes per lane: row 4 (NW i + w) + (lane >> 4), stored chunk lane & 15) over slices
// 4-7. The first step of every scale chunk (every SCH steps) also loads the next chunk, in slice 4.
// f16 weights: the group index given to a dead group's loads. Its byte offsets, 64 x this = 2^32 - 64
// up to 2^32 - 1, lie at or past the end of every f16 weight buffer the host accepts (fewer than 2^31
// elements with K a multiple of 32: at most 2^32 - 64 bytes), so they read zeros.
constexpr uint32_t kDeadF16Group = 0x03FFFFFFu;

template <int FMT, class T>
struct Loader {
    static constexpr int TN = T::TN, XI = T::XI, NSD = T::NSD;
    static constexpr int CODE_OPS = FMT == FMT_Q4 ? 2 : FMT == FMT_F16 ? 8 : 4;
    static constexpr int W_OPS = CODE_OPS * TN;
    static_assert(W_OPS == T::W_OPS, "load count");
    static constexpr int OPS = W_OPS + XI;
    static constexpr int WS = 2;                              // slices that issue the W loads
    static constexpr int XS = 4;                              // first slice of the x loads (the barrier)
    static constexpr int slice_of(int u) { return u < W_OPS ? u * WS / W_OPS : XS + (u - W_OPS) * (8 - XS) / XI; }

    brsrc_t p0, p1, rsc, rmn, rx;
    uint32_t colg[TN], sg[TN], xoff[XI];
    int h, G, wave;
    uint32_t slim;                 // last scale-chunk start that ends inside the plane (groups - SG)
    unsigned char* lds;
    // scale-chunk loads: flat group index of this lane's column for instruction k, and its LDS offset
    // within a chunk buffer
    uint32_t sdc[NSD], sdst[NSD];
    // of the W step being loaded: clamped group indices, and (f16) whether each group is live. q formats:
    // the lane half's two groups; f16: the step's four groups (every lane reads from each of them)
    uint32_t ia[TN], ib[TN];
    bool la, lb;
    uint32_t iq[FMT == FMT_F16 ? 4 : 1][TN];

    __device__ __forceinline__ void begin(int wstep)
    {
        if constexpr (FMT == FMT_F16) {
            // a group past the row end gets an index whose byte offsets lie past the end of the buffer
            // resource, so its loads return zeros without touching memory (and an Inf or NaN weight of
            // the next row cannot meet the zero padding of x); masking the loaded values instead made the
            // compiler wait for every load right where it was issued
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int g = 4 * wstep + q;
#pragma unroll
                for (int j = 0; j < TN; ++j) iq[q][j] = g < G ? colg[j] + (uint32_t)g : kDeadF16Group;
            }
            return;
        }
        const int g0 = 4 * wstep + 2 * h;
        const uint32_t ga = (uint32_t)min(g0, G - 1), gb = (uint32_t)min(g0 + 1, G - 1);
        la = g0 < G;
        lb = g0 + 1 < G;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            ia[j] = colg[j] + ga;
            ib[j] = colg[j] + gb;
        }
    }

    __device__ __forceinline__ void op(int u, WCodes<FMT> (&f)[TN], int xstep, uint32_t xbuf)
    {
        if (u >= W_OPS) {
            const int i = u - W_OPS;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(lds + xbuf + (T::NW * i + wave) * 1024), 16,
                                                     xoff[i], xstep * XROW, 0, 0);
            return;
        }
        const int j = u / CODE_OPS, k = u % CODE_OPS;
        WCodes<FMT>& w = f[j];
        if constexpr (FMT == FMT_Q4) {
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(p0, (k ? ib[j] : ia[j]) * 16, 0, 0);
            w.w[4 * k + 0] = v.x; w.w[4 * k + 1] = v.y; w.w[4 * k + 2] = v.z; w.w[4 * k + 3] = v.w;
        } else if constexpr (FMT == FMT_F16) {
            // the 16 bytes (8 halves) of slice k: k-th 16-k piece of the step, lane half h's 8 of them,
            // in group k >> 1 of the step at byte 32 (k & 1) + 16 h (zeros for a dead group)
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(p0, iq[k >> 1][j] * 64 + 32 * (k & 1) + 16 * h, 0, 0);
            w.w[4 * k + 0] = v.x; w.w[4 * k + 1] = v.y; w.w[4 * k + 2] = v.z; w.w[4 * k + 3] = v.w;
        } else if constexpr (FMT == FMT_Q8) {
            const uint32_t g = (k >> 1) ? ib[j] : ia[j];
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(p0, g * 32 + 16 * (k & 1), 0, 0);
            w.w[4 * k + 0] = v.x; w.w[4 * k + 1] = v.y; w.w[4 * k + 2] = v.z; w.w[4 * k + 3] = v.w;
        } else {
            if (k < 2) {
                const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(p0, (k ? ib[j] : ia[j]) * 8, 0, 0);
                w.w[2 * k] = v.x; w.w[2 * k + 1] = v.y;
            } else {
                w.w[4 + (k - 2)] = __builtin_amdgcn_raw_buffer_load_b32(p1, ((k - 2) ? ib[j] : ia[j]) * 4, 0, 0);
            }
        }
    }

    // all ops of slice sl
    __device__ __forceinline__ void issue(int sl, WCodes<FMT> (&f)[TN], int xstep, uint32_t xbuf)
    {
#pragma unroll
        for (int u = 0; u < OPS; ++u)
            if (slice_of(u) == sl) op(u, f, xstep, xbuf);
    }

    // Scale chunk v (groups SG v .. SG v + SG - 1 of every column of the block) into the chunk buffer at
    // byte offset `buf`: instruction k of wave w covers plane (NW k + w) / CPI and the 64 / LPC columns
    // that follow (NW k + w) % CPI times as many (CPI = instructions per plane), 16 bytes (8 groups)
    // per lane, LPC lanes per column. A chunk that would run past the end of the plane is moved back
    // to end inside it; the reader shifts its index by the same amount.
    __device__ __forceinline__ void scale_chunk(int v, uint32_t buf)
    {
        constexpr int CPI = T::SPLANE / 1024;
#pragma unroll
        for (int k = 0; k < NSD; ++k) {
            const uint32_t plane = (uint32_t)(T::NW * k + wave) / CPI;
            const uint32_t off = (min(sdc[k] + T::SG * v, slim) + 8 * (threadIdx.x % T::LPC)) * 2;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(plane ? rmn : rsc, (lds_void_t*)(lds + buf + sdst[k]), 16,
                                                     off, 0, 0, 0);
        }
    }

    // Issue the LDS reads of the scales and mins of W step t (chunk buffer at `buf`) into f: groups
    // 4 t + 2 h + e, e = 0, 1. The values may be used only after lds_wait and finish_scales.
    __device__ __forceinline__ void read_scales(WCodes<FMT> (&f)[TN], int t, uint32_t buf, int lane)
    {
        const uint32_t F0 = T::SG * (uint32_t)(t / T::SCH);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t F = sg[j] + F0;
            // shift of a moved chunk; a live group's position is at most 15, and the clamp keeps reads of
            // dead groups (masked in finish_scales) within the chunk buffer and its 64-byte pad
            const uint32_t pos = min((F - min(F, slim)) + 4 * (t % T::SCH) + 2 * h, (uint32_t)T::SG - 1);
            const uint32_t col = (uint32_t)(wave * 32 * TN + 32 * j + (lane & 31));
            const uint32_t ps = lds_addr(lds + buf) + col * (T::SG * 2) + pos * 2;
            f[j].s[0] = ds_read_u16(ps);
            f[j].s[1] = ds_read_u16<2>(ps);
            if constexpr (FMT != FMT_Q8) {
                f[j].m[0] = ds_read_u16<T::SPLANE>(ps);
                f[j].m[1] = ds_read_u16<T::SPLANE + 2>(ps);
            }
        }
    }

    // After lds_wait: order the values read by read_scales after the wait, and give groups past the row
    // end scale and min 0.
    __device__ __forceinline__ void finish_scales(WCodes<FMT> (&f)[TN], int t)
    {
        const int g0 = 4 * t + 2 * h;
        const bool la = g0 < G, lb = g0 + 1 < G;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            tie(f[j].s[0]);
            tie(f[j].s[1]);
            f[j].s[0] = la ? f[j].s[0] : 0u;
            f[j].s[1] = lb ? f[j].s[1] : 0u;
            if constexpr (FMT != FMT_Q8) {
                tie(f[j].m[0]);
                tie(f[j].m[1]);
                f[j].m[0] = la ? f[j].m[0] : 0u;
                f[j].m[1] = lb ? f[j].m[1] : 0u;
            } else {
                f[j].m[0] = f[j].m[1] = 0u;
            }
        }
    }
};

// Dequantize 8 codes to 4 packed f16 pairs (codes j and j + 4 in pair j). A code q placed in the
// mantissa of a power of two 2^E whose mantissa unit is 1 at the code's bit position reads as
// 2^E + q: 1024.0h (unit 1 at bit 0) for a code in bits 0-3, 64.0h (unit 1/16 at bit 0, so 1 at
// bit 4) for a code left in bits 4-7. One packed subtract (exact) and one packed FMA then give the
// dequantized pair (q s + m), rounded once, with the f16 scale itself: no scale is rescaled, so
// every normal or subnormal scale is used exactly. The pairs (j, j + 4) match the
// [0 4 1 5 2 6 3 7] order of the staged x.
// Mask and exponent constants of the dequantization, held in VGPRs so that a mask-and-insert is one
// v_and_or_b32 (a VOP3 instruction here takes no literal operand, and with literals the compiler
// emits a v_and_b32 / v_or_b32 pair instead).
struct DeqConst {
    uint32_t lo4, hi4, e1024, lo2, e64;
    __device__ __forceinline__ static DeqConst make()
    {
        DeqConst k{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x00030003u, 0x54005400u};
        asm volatile("" : "+v"(k.lo4), "+v"(k.hi4), "+v"(k.e1024), "+v"(k.lo2), "+v"(k.e64));
        return k;
    }
};

// q4: the low nibble of each byte on the mantissa units of 1024.0h, the high nibble in place on
// those of 64.0h.
__device__ __forceinline__ u32x4_t deq8_q4(uint32_t w, half2_t s2, half2_t m2, const DeqConst& k)
{
    const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
    const half2_t k64 = {(_Float16)64.f, (_Float16)64.f};
    const uint32_t w8 = w >> 8;
    u32x4_t r;
    r[0] = as_u32(__builtin_elementwise_fma(as_h2((w & k.lo4) | k.e1024) - k1024, s2, m2));
    r[1] = as_u32(__builtin_elementwise_fma(as_h2((w & k.hi4) | k.e64) - k64, s2, m2));
    r[2] = as_u32(__builtin_elementwise_fma(as_h2((w8 & k.lo4) | k.e1024) - k1024, s2, m2));
    r[3] = as_u32(__builtin_elementwise_fma(as_h2((w8 & k.hi4) | k.e64) - k64, s2, m2));
    return r;
}

// q3: `lo16` 8 two-bit fields, `hi8` their high bits.
__device__ __forceinline__ u32x4_t deq8_q3(uint32_t lo16, uint32_t hi8, half2_t s2, half2_t m2, const DeqConst& k)
{
    const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
    // code j sits at bits 2j of L and code j + 4 at bits 16 + 2j; high bits likewise at 2 + j, 18 + j of H
    const uint32_t L = lo16 | (lo16 << 8), H = (hi8 << 2) | (hi8 << 14);
    u32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = ((L >> (2 * j)) & k.lo2) | ((H >> j) & 0x00040004u) | k.e1024;
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

// Per-group scale operands of one column block for the current step: packed splats of the scale and
// min of groups e = 0, 1.
struct GroupOps {
    half2_t s2[2], m2[2];
    DeqConst k;
};

template <int FMT>
__device__ __forceinline__ GroupOps group_ops(const WCodes<FMT>& f, const DeqConst& k)
{
    GroupOps o;
    o.k = k;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)f.s[e]);
        const _Float16 m = __builtin_bit_cast(_Float16, (uint16_t)f.m[e]);
        o.s2[e] = half2_t{s, s};
        o.m2[e] = half2_t{m, m};
    }
    return o;
}

// B operand of slice sl (0..7): codes 8 (sl & 3) .. + 7 of group sl >> 2.
template <int FMT>
__device__ __forceinline__ half8_t b_frag(const WCodes<FMT>& f, const GroupOps& g, int sl)
{
    const int e = sl >> 2, c = sl & 3;
    u32x4_t o;
    if constexpr (FMT == FMT_Q4) {
        o = deq8_q4(f.w[sl], g.s2[e], g.m2[e], g.k);
    } else if constexpr (FMT == FMT_F16) {
        // halves w0 .. w7 (dwords d0 .. d3) -> pairs (w0 w4) (w1 w5) (w2 w6) (w3 w7), the staged x order
        const uint32_t* d = f.w + 4 * sl;
        o[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);
        o[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);
        o[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);
        o[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);
    } else if constexpr (FMT == FMT_Q8) {
        o = deq8_q8(f.w[2 * sl], f.w[2 * sl + 1], g.s2[e]);
    } else {
        o = deq8_q3((f.w[2 * e + (c >> 1)] >> (16 * (c & 1))) & 0xffffu, (f.w[4 + e] >> (8 * c)) & 0xffu, g.s2[e], g.m2[e], g.k);
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

// Wait until at most N vector-memory loads of this wave are in flight. The compiler does not track
// direct global->LDS loads as writers of LDS, so their completion is waited for explicitly (they
// complete in issue order with the other loads).
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The row scale of one tile row into LDS for the epilogue. Written as an ordinary store at the top of
// the prologue, it is an LDS write the compiler keeps ahead of the direct global->LDS loads that follow
// (it counts them as LDS writes too), so the code waited for the scale's own load before issuing the
// first of them: a memory round trip ahead of the prologue's weight and x loads. As asm after the
// prologue's loads it only waits for its value (the compiler's own wait on the loaded register); the
// step barriers that follow (each waits for this wave's LDS operations) make it visible to the
// epilogue's readers in the other waves.
__device__ __forceinline__ void store_rscale(uint32_t addr, float v)
{
    asm volatile("ds_write_b32 %0, %1" ::"v"(addr), "v"(v));
}

// Barrier between pipeline steps. A fence here would make the compiler wait for every direct
// global->LDS load in flight (it counts them as LDS writes), including the ones issued for two steps
// ahead; the LDS reads of this wave are waited for here, its direct loads by wait_vm before the call.
// The memory clobber keeps LDS accesses on their side of the barrier.
__device__ __forceinline__ void step_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One step of the multiply loop, 8 slices. On entry a[0] and b[0] hold the operands of slice 0,
// prepared by the previous step. Slice sl reads and dequantizes the operands of slice sl + 1 while its
// MFMAs run; slices 6-7 prepare slice 0 of the next step (its scales, codes in wn, and x). Loads: W
// codes of step t + PF into wl in slices 0-1; at slice 4 the wave waits for the loads of earlier steps
// (x step t + 1 among them) and meets the other waves at the barrier, after which x step t + 1 may be
// read and the buffer of step t - 1 refilled: x step t + PF + 1 goes there over slices 4-7, and at the
// first step of a scale chunk the next chunk is loaded. With PF = 1, wn and wl are the same registers.
template <int FMT, class T>
__device__ __forceinline__ void mma_step(const unsigned char* lds, const uint32_t (&aoff)[8], uint32_t abuf,
                                         uint32_t anext, const WCodes<FMT> (&wc)[T::TN], const GroupOps (&go)[T::TN],
                                         half8_t (&a)[2][T::TM], half8_t (&b)[2][T::TN],
                                         floatx16_t (&acc)[T::TM][T::TN], Loader<FMT, T>& ld,
                                         WCodes<FMT> (&wn)[T::TN], WCodes<FMT> (&wl)[T::TN], GroupOps (&gn)[T::TN],
                                         int t, int xstep, uint32_t xbuf, bool schunk, int sv, uint32_t sdst,
                                         uint32_t snext, int lane)
{
    constexpr int TM = T::TM, TN = T::TN;
    const uint32_t lbase = lds_addr(lds);
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
        const int cur = sl & 1, nxt = cur ^ 1;
        // the A fragments of this slice (read during the previous one) and, at slice 7, the scales read
        // at slice 6
        lds_wait();
#pragma unroll
        for (int i = 0; i < TM; ++i) tie(a[cur][i]);
        if constexpr (FMT != FMT_F16)
            if (sl == 7) ld.finish_scales(wn, t + 1);
        if (sl == Loader<FMT, T>::XS) {
            wait_vm<T::VM_NEXT_X>();
            step_barrier();
            if (schunk) ld.scale_chunk(sv, sdst);
        }
        ld.issue(sl, wl, xstep, xbuf);
        if constexpr (FMT != FMT_F16)
            if (sl == 6) ld.read_scales(wn, t + 1, snext, lane);
        if (sl < 7) {
            read_a<TM>(a[nxt], lbase + abuf + aoff[sl + 1]);
#pragma unroll
            for (int j = 0; j < TN; ++j) b[nxt][j] = b_frag<FMT>(wc[j], go[j], sl + 1);
        } else {
            read_a<TM>(a[nxt], lbase + anext + aoff[0]);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                gn[j] = group_ops<FMT>(wn[j], go[j].k);
                b[nxt][j] = b_frag<FMT>(wn[j], gn[j], 0);
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[cur][i], b[cur][j], acc[i][j], 0, 0, 0);
        // the next slice's A reads first, then each MFMA with a share of the dequantization; the
        // scheduling barrier keeps every slice's reads one slice ahead of their use
        constexpr int VALU_PER = (FMT == FMT_F16 ? 4 : FMT == FMT_Q8 ? 12 : 16) * TN / (TM * TN);
#pragma unroll
        for (int g = 0; g < TM * TN; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, VALU_PER > 0 ? VALU_PER : 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// GROUPED: the expert-grouped (MoE) form, a separate instantiation so that the dense kernels hold
// none of its code; blockIdx.y enumerates (expert, row tile) pairs, found by the block-wide lookup.
// gtile / gcol (grouped only): this block's (expert, row tile) pair and column tile.
// One block tile: rows [m0, min(m0 + BM, m_end)) and columns [n0, n0 + BN) of y, with weight slice e
// (GROUPED) of the planes, in `smem` (T::SMEM bytes, 1024-byte aligned).
template <int FMT, class T, bool GROUPED>
__device__ __forceinline__ void gemm_tile_run(unsigned char* smem, const uint16_t* __restrict__ xh,
                                              const float* __restrict__ rscale, const uint8_t* __restrict__ p0,
                                              const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc,
                                              const uint16_t* __restrict__ mn, float* __restrict__ y, int M, int K,
                                              int N, int E, int e, int m0, int m_end, int n0,
                                              const float* __restrict__ tbias = nullptr, int trans = 0)
{
    constexpr int BN = T::BN, TM = T::TM, TN = T::TN, XI = T::XI, NT = T::NT;
    const int G = K / BRIK_GROUP;
    const int Kp = (K + 2 * GK - 1) / (2 * GK) * (2 * GK);
    const int steps = Kp / GK;                 // even, >= 2

    // buffer resources: the staged x rows of this launch; the W planes of this matrix (expert slice);
    // the scales and mins of the whole (stacked) plane
    const size_t wel = (size_t)N * K;          // elements of one weight matrix
    const size_t gbase = (size_t)e * N * G;    // flat group offset of the expert slice
    const brsrc_t rx = make_rsrc(xh, (uint32_t)((size_t)M * Kp * 2));
    brsrc_t r0, r1 = rx, rsc, rmn = rx;
    if constexpr (FMT == FMT_F16) {
        static_assert(!GROUPED, "f16 weights: dense only");
        r0 = make_rsrc(p0, (uint32_t)(wel * 2));
    } else if constexpr (FMT == FMT_Q8) {
        r0 = make_rsrc(p0 + (size_t)e * wel, (uint32_t)wel);
    } else if constexpr (FMT == FMT_Q4) {
        r0 = make_rsrc(p0 + (size_t)e * wel / 2, (uint32_t)(wel / 2));
    } else {
        r0 = make_rsrc(p0 + (size_t)e * wel / 4, (uint32_t)(wel / 4));
        r1 = make_rsrc(p1 + (size_t)e * wel / 8, (uint32_t)(wel / 8));
    }
    const uint32_t sgroups = (uint32_t)((size_t)(GROUPED ? E : 1) * N * G);
    rsc = make_rsrc(sc, FMT == FMT_F16 ? 0u : sgroups * 2);
    if constexpr (FMT != FMT_Q8) rmn = make_rsrc(mn, FMT == FMT_F16 ? 0u : sgroups * 2);

    const int tid = threadIdx.x, lane = tid & 63;
    Loader<FMT, T> ld;
    ld.p0 = r0; ld.p1 = r1; ld.rsc = rsc; ld.rmn = rmn; ld.rx = rx;
    ld.h = lane >> 5; ld.G = G; ld.lds = smem;
    ld.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = ld.h, wave = ld.wave;
    // the row scales the epilogue applies: loaded first, so their latency hides behind the prologue's
    // instead of opening the epilogue (rows past the tile's end repeat a live row), and written into LDS
    // after the prologue's loads are issued (store_rscale)
    const float rs_row = tid < T::BM ? rscale[min(m0 + tid, m_end - 1)] : 0.f;
    // x staging: this lane's chunk of each direct-load instruction (row 4 (NW i + wave) + (lane >> 4),
    // stored chunk lane & 15, which holds logical chunk (lane & 15) ^ (row & 15))
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int r = 4 * (T::NW * i + wave) + (lane >> 4);
        const int m = min(m0 + r, m_end - 1);      // rows past the tile's end repeat a live row
        ld.xoff[i] = (uint32_t)(m * Kp + (((lane & 15) ^ (r & 15)) * 8)) * 2;
    }
    // A fragments of slice sl: row lane & 31 of a 32-row block, logical chunk 8 h + sl (quantized W: a
    // lane half owns two whole groups of the step), or 2 sl + h (f16 W: the two lane halves of a slice
    // read adjacent 16-byte pieces of a weight row, so a load instruction spans 32 rows x 32 bytes
    // instead of 64 rows' worth of 16-byte pieces)
    uint32_t aoff[8];
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
        const int chunk = FMT == FMT_F16 ? 2 * sl + h : 8 * h + sl;
        aoff[sl] = (uint32_t)((lane & 31) * XROW + ((chunk ^ (lane & 15)) * 16));
    }
    // W: flat group index of this lane's column in column block j, at group 0
    const int wn = wave * 32 * TN;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        ld.colg[j] = (uint32_t)(min(n0 + wn + 32 * j + (lane & 31), N - 1) * G);
        ld.sg[j] = (uint32_t)gbase + ld.colg[j];   // the same group in the whole scale plane
    }
    // scale chunks (the host routes planes of fewer than 16 groups elsewhere)
    ld.slim = sgroups - T::SG;
#pragma unroll
    for (int k = 0; k < T::NSD; ++k) {
        constexpr int CPI = T::SPLANE / 1024, COLS = 64 / T::LPC;   // instructions per plane, columns each
        const int gi = T::NW * k + wave, cb = gi % CPI, plane = gi / CPI;
        ld.sdc[k] = (uint32_t)gbase + (uint32_t)(min(n0 + COLS * cb + lane / T::LPC, N - 1) * G);
        ld.sdst[k] = (uint32_t)(plane * T::SPLANE + cb * 1024);
    }

    floatx16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Prologue, in the order the steps keep: W codes of step 0 into registers, scale chunk 0, x steps 0
    // and 1 into LDS, then W of step s and x of step s + 1 for s = 1 .. PF - 1; then the operands of
    // slice 0 of step 0. W step s sits in slot s of a ring of PF + 1 register sets, x step s in LDS
    // buffer s mod (PF + 2). Steps past the end are clamped (their loads are never used).
    constexpr int R = T::PF + 1;
    WCodes<FMT> wr[R][TN];
    GroupOps go[TN], gn[TN];
    half8_t a[2][TM], b[2][TN];
    ld.begin(0);
#pragma unroll
    for (int u = 0; u < ld.W_OPS; ++u) ld.op(u, wr[0], 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    ld.scale_chunk(0, T::S_OFF);
#pragma unroll
    for (int u = ld.W_OPS; u < ld.OPS; ++u) ld.op(u, wr[0], 0, 0);
#pragma unroll
    for (int u = ld.W_OPS; u < ld.OPS; ++u) ld.op(u, wr[0], min(1, steps - 1), T::XBUF);
#pragma unroll
    for (int s = 1; s < T::PF; ++s) {
        ld.begin(min(s, steps - 1));
#pragma unroll
        for (int u = 0; u < ld.W_OPS; ++u) ld.op(u, wr[s], 0, 0);
#pragma unroll
        for (int u = ld.W_OPS; u < ld.OPS; ++u) ld.op(u, wr[s], min(s + 1, steps - 1), (s + 1) * T::XBUF);
    }
    // x step 0 (and scale chunk 0) landed: at most x step 1 and the PF - 1 later (W, x) pairs in flight
    wait_vm<XI + (T::PF - 1) * (T::W_OPS + XI)>();
    step_barrier();
    if (tid < T::BM) store_rscale(lds_addr(smem + T::RS_OFF) + 4 * (uint32_t)tid, rs_row);
    if constexpr (FMT != FMT_F16) ld.read_scales(wr[0], 0, T::S_OFF, lane);
    const DeqConst dk = DeqConst::make();
    read_a<TM>(a[0], lds_addr(smem) + aoff[0]);
    lds_wait();
    if constexpr (FMT != FMT_F16) ld.finish_scales(wr[0], 0);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        go[j] = group_ops<FMT>(wr[0][j], dk);
        b[0][j] = b_frag<FMT>(wr[0][j], go[j], 0);
    }

    // Step t multiplies x step t (LDS buffer xq) by W step t (ring slot t mod R); it loads W step
    // t + PF into slot (t + PF) mod R and, once every wave is past its barrier, x step t + PF + 1 into
    // the buffer of step t - 1. The loop body runs R steps so that the ring slots are fixed registers.
    // Loads past the end are clamped, and the operands prepared for step `steps` are not used.
    const int nchunks = (steps + T::SCH - 1) / T::SCH;
    uint32_t xq = 0;
    int t = 0;
    do {     // steps >= 2: no loop guard for the prologue loads to sink past
#pragma unroll
        for (int r = 0; r < R; ++r) {
            ld.begin(min(t + T::PF, steps - 1));
            const int v = t / T::SCH;
            const uint32_t x1 = xq + 1 == (uint32_t)T::XQ ? 0u : xq + 1;     // buffer of step t + 1
            const uint32_t xf = xq == 0 ? (uint32_t)T::XQ - 1 : xq - 1;       // buffer of step t - 1
            mma_step<FMT, T>(smem, aoff, xq * T::XBUF, x1 * T::XBUF, wr[r], go, a, b, acc, ld, wr[(r + 1) % R],
                             wr[(r + T::PF) % R], gn, t, min(t + T::PF + 1, steps - 1), xf * T::XBUF,
                             t % T::SCH == 0, min(v + 1, nchunks - 1), T::S_OFF + ((v + 1) & 1) * T::SBUF,
                             T::S_OFF + (((t + 1) / T::SCH) & 1) * T::SBUF, lane);
#pragma unroll
            for (int j = 0; j < TN; ++j) go[j] = gn[j];
            xq = x1;
            ++t;
            // steps is even, so a two-step body never stops half way
            if (R > 2 && r + 1 < R && t >= steps) break;
        }
    } while (t < steps);
    // The A fragments the last slice read for a step that does not run: their registers must stay
    // allocated until those reads have landed, or the epilogue could reuse them while an LDS read is
    // still to write them.
    lds_wait();
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        tie(a[0][i]);
        tie(a[1][i]);
    }
    // the clamped loads of the last steps may still be writing LDS, which the epilogue reuses
    wait_vm<0>();
    if (!trans) {
        // Row-major y: every lane stores its accumulators straight from registers (D layout of a
        // 32x32 tile: lane holds column lane & 31, register r row 8 (r >> 2) + 4 h + (r & 3)), times
        // the row scale read from LDS, 4 rows per 16-byte read. One store instruction covers two rows
        // of 32 consecutive columns (two 128-byte runs). Staging the tile through LDS for 16-byte
        // stores cost two barriers per round of row blocks and let no store start before the whole
        // round was staged.
        const float* const rs = reinterpret_cast<const float*>(smem + T::RS_OFF);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r0 = 32 * i + 8 * q + 4 * h;
                const f32x4_t s4 = *reinterpret_cast<const f32x4_t*>(rs + r0);
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int n = n0 + wn + 32 * j + (lane & 31);
                    if (n >= N) continue;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int m = m0 + r0 + e;
                        if (m < m_end) y[(size_t)m * N + n] = acc[i][j][4 * q + e] * s4[e];
                    }
                }
            }
        return;
    }
    lds_barrier();

    // Epilogue of the transposed store (y [N, M], the convolution's layout), RF row blocks per round:
    // the accumulators are staged in LDS (the D layout above), then every thread scales 4 consecutive
    // rows of one column by rscale, adds the column's bias and stores them with one 16-byte store
    // (M % 4 == 0) or four 4-byte stores.
    float* const Cs = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int i0 = 0; i0 < TM; i0 += T::RF) {
        if (i0) lds_barrier();                      // the previous round's reads are done
#pragma unroll
        for (int ii = 0; ii < T::RF; ++ii)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    Cs[(ii * 32 + 8 * (r >> 2) + 4 * h + (r & 3)) * T::CLD + wn + 32 * j + (lane & 31)] = acc[i0 + ii][j][r];
        lds_barrier();
        // y[n, m] = C[m, n] rscale[m] + tbias[n] (one rounding, the product being exact), 4 consecutive
        // rows of one column per thread and store
        constexpr int RB = T::RF * 32 / 4;
        for (int c = tid; c < BN * RB; c += NT) {
            const int col = c / RB, row = (c % RB) * 4;
            const int m = m0 + i0 * 32 + row, n = n0 + col;
            if (m >= m_end || n >= N) continue;
            const float b = tbias ? tbias[n] : 0.f;
            f32x4_t v;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                v[k] = m + k < m_end ? Cs[(row + k) * T::CLD + col] * rscale[m + k] + b : 0.f;
            float* dst = y + (size_t)n * M + m;
            if ((M & 3) == 0 && m + 3 < m_end) {
                *(f32x4_t*)dst = v;
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (m + k < m_end) dst[k] = v[k];
            }
        }
    }
}

template <int FMT, class T, bool GROUPED>
__device__ __forceinline__ void gemm_body(const uint16_t* __restrict__ xh, const float* __restrict__ rscale,
                                          const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,
                                          const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn,
                                          float* __restrict__ y, int M, int K, int N,
                                          const int* __restrict__ row_off, int E, int gtile = 0, int gcol = 0,
                                          const float* __restrict__ tbias = nullptr, int trans = 0)
{
    constexpr int BM = T::BM, BN = T::BN;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[T::SMEM];
    int m0, m_end = M, n0, e = 0;
    if constexpr (GROUPED) {
        n0 = gcol * BN;
        // uniform across the block (the lookup ends with a barrier), before any other barrier
        if (!find_expert_tile<BM>(row_off, E, gtile, M, e, m0, m_end)) return;
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
    gemm_tile_run<FMT, T, GROUPED>(smem, xh, rscale, p0, p1, sc, mn, y, M, K, N, E, e, m0, m_end, n0, tbias, trans);
}

// Expert-grouped tile of TL::BM rows that runs the TS::BM-row body (the same columns and waves) when
// its expert tile holds no more live rows than that: an expert's last (or only) row tile is often
// about half full, and the smaller body skips the MFMAs, A-fragment reads and x loads of the empty
// 32-row block. The pairs are those of the TL::BM tiling.
template <int FMT, class TL, class TS>
__device__ __forceinline__ void gemm_grouped_adaptive(const uint16_t* __restrict__ xh, const float* __restrict__ rscale,
                                                      const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,
                                                      const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn,
                                                      float* __restrict__ y, int M, int K, int N,
                                                      const int* __restrict__ row_off, int E, int gtile, int gcol)
{
    static_assert(TL::BN == TS::BN && TL::NT == TS::NT && TS::BM < TL::BM, "adaptive tile pair");
    constexpr int SM = TL::SMEM > TS::SMEM ? TL::SMEM : TS::SMEM;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[SM];
    int e = 0, m0 = 0, m_end = M;
    if (!find_expert_tile<TL::BM>(row_off, E, gtile, M, e, m0, m_end)) return;
    const int n0 = gcol * TL::BN;
    if (m_end - m0 <= TS::BM)
        gemm_tile_run<FMT, TS, true>(smem, xh, rscale, p0, p1, sc, mn, y, M, K, N, E, e, m0, m_end, n0);
    else
        gemm_tile_run<FMT, TL, true>(smem, xh, rscale, p0, p1, sc, mn, y, M, K, N, E, e, m0, m_end, n0);
}

// ---- 3. split-K GEMM for few rows ---------------------------------------------------------------
// A launch with few rows per weight column (small M, or an expert's 20-50 routed rows) has too little
// MFMA work to hide the dequantization behind: the tiled kernel above then runs one wave per SIMD on
// the few blocks its tiles give, each paying the issue latency of ~150 VALU instructions per K step
// (measured: ~0.65 us per step whatever the prefetch depth). This kernel spreads the same work over
// many small blocks instead: a block owns 32 rows x 128 columns (4 waves, one 32-column MFMA block
// each) over a slice of at most KSL K steps. It issues every load of its slice at once (W codes,
// scales and mins into registers, the f16 x rows of the slice into LDS), waits once, and runs the
// slice's MFMAs without a barrier; several blocks per CU overlap one block's loads with another's
// arithmetic. With more than one slice (gridDim.z) every block writes its partial tile to `part`
// ([slice][row][column] f32, already times the row scale) and brik_splitk_reduce, the next launch on
// the stream, sums the slices in order into y: the result does not depend on which block finishes
// first. (Summing in the last block of each tile instead, behind device-scope fences and a counter,
// measured several times slower: every fence writes back and invalidates an XCD's L2.)
constexpr int SK_BM = 32, SK_BN = 128;

template <int FMT, int KSL>
__device__ __forceinline__ void gemm_sk_body(const uint16_t* __restrict__ xh, const float* __restrict__ rscale,
                                             const uint8_t* __restrict__ p0, const uint8_t* __restrict__ p1,
                                             const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn,
                                             float* __restrict__ y, int M, int K, int N,
                                             const int* __restrict__ row_off, int E, float* __restrict__ part)
{
    constexpr int SBUF = SK_BM * XROW;                   // one step of x rows in LDS
    __shared__ __attribute__((aligned(1024))) unsigned char smem[KSL * SBUF];

    const int G = K / BRIK_GROUP;
    const int Kp = (K + 2 * GK - 1) / (2 * GK) * (2 * GK);
    const int steps = Kp / GK;
    const int KS = (int)gridDim.z, slice = (int)blockIdx.z;
    const int t0 = slice * KSL;
    const int nst = min(KSL, steps - t0);                // >= 1: the host sizes gridDim.z so
    const int n0 = (int)blockIdx.x * SK_BN;
    int m0, m_end = M, e = 0;
    if (row_off) {
        // the whole block, and the same for every slice of the tile
        if (!find_expert_tile<SK_BM>(row_off, E, (int)blockIdx.y, M, e, m0, m_end)) return;
    } else {
        m0 = (int)blockIdx.y * SK_BM;
        if (m0 >= M) return;
    }

    const size_t wel = (size_t)N * K;
    const size_t gbase = (size_t)e * N * G;
    const brsrc_t rx = make_rsrc(xh, (uint32_t)((size_t)M * Kp * 2));
    brsrc_t r0, r1 = rx;
    if constexpr (FMT == FMT_Q8) {
        r0 = make_rsrc(p0 + (size_t)e * wel, (uint32_t)wel);
    } else if constexpr (FMT == FMT_Q4) {
        r0 = make_rsrc(p0 + (size_t)e * wel / 2, (uint32_t)(wel / 2));
    } else {
        r0 = make_rsrc(p0 + (size_t)e * wel / 4, (uint32_t)(wel / 4));
        r1 = make_rsrc(p1 + (size_t)e * wel / 8, (uint32_t)(wel / 8));
    }
    const uint32_t sgroups = (uint32_t)((size_t)(row_off ? E : 1) * N * G);
    const brsrc_t rsc = make_rsrc(sc, sgroups * 2);
    const brsrc_t rmn = FMT == FMT_Q8 ? rsc : make_rsrc(mn, sgroups * 2);

    const int tid = (int)threadIdx.x, lane = tid & 63, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ncol = n0 + wave * 32 + (lane & 31);        // this lane's column (D layout and B operand)
    const uint32_t colg = (uint32_t)(min(ncol, N - 1) * G);
    const uint32_t sgb = (uint32_t)gbase + colg;

    // every load of the slice: W codes, scales and mins of each step (lane half h holds groups
    // 4t + 2h and 4t + 2h + 1 of its column), then the x rows of each step into LDS
    WCodes<FMT> wr[KSL];
    uint32_t gs[KSL];                                    // first group of the lane's pair, per step
#pragma unroll
    for (int t = 0; t < KSL; ++t) {
        const int g0 = 4 * min(t0 + t, steps - 1) + 2 * h;
        gs[t] = (uint32_t)g0;
        const uint32_t ga = colg + (uint32_t)min(g0, G - 1), gb = colg + (uint32_t)min(g0 + 1, G - 1);
        WCodes<FMT>& f = wr[t];
        if constexpr (FMT == FMT_Q4) {
            const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(r0, ga * 16, 0, 0);
            const u32x4_t b = __builtin_amdgcn_raw_buffer_load_b128(r0, gb * 16, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) { f.w[j] = a[j]; f.w[4 + j] = b[j]; }
        } else if constexpr (FMT == FMT_Q8) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r0, (k >> 1 ? gb : ga) * 32 + 16 * (k & 1), 0, 0);
#pragma unroll
                for (int j = 0; j < 4; ++j) f.w[4 * k + j] = v[j];
            }
        } else {
            const u32x2_t a = __builtin_amdgcn_raw_buffer_load_b64(r0, ga * 8, 0, 0);
            const u32x2_t b = __builtin_amdgcn_raw_buffer_load_b64(r0, gb * 8, 0, 0);
            f.w[0] = a.x; f.w[1] = a.y; f.w[2] = b.x; f.w[3] = b.y;
            f.w[4] = __builtin_amdgcn_raw_buffer_load_b32(r1, ga * 4, 0, 0);
            f.w[5] = __builtin_amdgcn_raw_buffer_load_b32(r1, gb * 4, 0, 0);
        }
        const uint32_t sa = sgb + (uint32_t)min(g0, G - 1), sb = sgb + (uint32_t)min(g0 + 1, G - 1);
        f.s[0] = __builtin_amdgcn_raw_buffer_load_b16(rsc, sa * 2, 0, 0);
        f.s[1] = __builtin_amdgcn_raw_buffer_load_b16(rsc, sb * 2, 0, 0);
        if constexpr (FMT != FMT_Q8) {
            f.m[0] = __builtin_amdgcn_raw_buffer_load_b16(rmn, sa * 2, 0, 0);
            f.m[1] = __builtin_amdgcn_raw_buffer_load_b16(rmn, sb * 2, 0, 0);
        } else {
            f.m[0] = f.m[1] = 0u;
        }
    }
    // x: step t of the slice fills LDS bytes [t SBUF, (t + 1) SBUF), 32 rows x 256 bytes, as eight
    // 1 KiB direct loads (16 bytes per lane: row 4 i + (lane >> 4), stored chunk lane & 15, which holds
    // logical chunk (lane & 15) ^ (row & 15)); wave w issues i = w and w + 4. Rows past the tile's end
    // repeat a live row.
#pragma unroll
    for (int t = 0; t < KSL; ++t) {
        const int tt = min(t0 + t, steps - 1);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = 4 * j + wave;
            const int r = 4 * i + (lane >> 4);
            const int m = min(m0 + r, m_end - 1);
            const uint32_t off = (uint32_t)((size_t)m * Kp + (size_t)tt * GK + (((lane & 15) ^ (r & 15)) * 8)) * 2;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(smem + t * SBUF + i * 1024), 16, off, 0, 0, 0);
        }
    }
    // every load above stays ahead of the wait: the loaded registers are consumed here (an empty asm),
    // so no load can be sunk down to the step that uses it (each step would then pay a memory round
    // trip), not even into the steps that run only when the slice is that long
#pragma unroll
    for (int t = 0; t < KSL; ++t) {
#pragma unroll
        for (int j = 0; j < (int)(sizeof(wr[t].w) / 4); ++j) asm volatile("" ::"v"(wr[t].w[j]));
        asm volatile("" ::"v"(wr[t].s[0]), "v"(wr[t].s[1]), "v"(wr[t].m[0]), "v"(wr[t].m[1]));
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vm<0>();
    step_barrier();

    uint32_t aoff[8];
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) aoff[sl] = (uint32_t)((lane & 31) * XROW + (((8 * h + sl) ^ (lane & 15)) * 16));
    const DeqConst dk = DeqConst::make();
    floatx16_t acc[2];
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[q][r] = 0.f;
#pragma unroll
    for (int t = 0; t < KSL; ++t) {
        if (t >= nst) break;                             // uniform: the last slice may be shorter
        // groups past the row end: scale and min 0 (their x is zero padding as well)
        WCodes<FMT> f = wr[t];
        const bool la = (int)gs[t] < G, lb = (int)gs[t] + 1 < G;
        f.s[0] = la ? f.s[0] : 0u; f.s[1] = lb ? f.s[1] : 0u;
        f.m[0] = la ? f.m[0] : 0u; f.m[1] = lb ? f.m[1] : 0u;
        const GroupOps go = group_ops<FMT>(f, dk);
#pragma unroll
        for (int sl = 0; sl < 8; ++sl) {
            const half8_t a = *(const half8_t*)(smem + t * SBUF + aoff[sl]);
            const half8_t b = b_frag<FMT>(f, go, sl);
            acc[sl & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[sl & 1], 0, 0, 0);
        }
    }

    // D layout of a 32x32 tile: lane holds column lane & 31, register r row 8 (r >> 2) + 4 h + (r & 3)
    const bool colok = ncol < N;
    if (KS == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (colok && m < m_end) y[(size_t)m * N + ncol] = (acc[0][r] + acc[1][r]) * rscale[m];
        }
        return;
    }
    float* const P = part + (size_t)slice * M * N;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int m = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (colok && m < m_end) P[(size_t)m * N + ncol] = (acc[0][r] + acc[1][r]) * rscale[m];
    }
}

}  // namespace

// Kernel names: brik_gemm_<fmt>_<BM>x<TN> (block tile BM x 128 TN, 256 threads = 4 waves) and
// brik_gemm_<fmt>_<BM>x<TN>w8 (BM x 256 TN, 512 threads = 8 waves), with p<PF> for the prefetching
// tiles; the runtime picks the tile. Dense kernels ignore row_off / E.
#define BRIK_GEMM_DENSE(FMTN, FMT, BM_, TN_, NW_, PF_, SUFFIX)                                            \
    extern "C" __global__ __launch_bounds__(64 * NW_) void brik_gemm_##FMTN##_##BM_##x##TN_##SUFFIX(      \
        const uint16_t* __restrict__ xh, const float* __restrict__ rscale, const uint8_t* __restrict__ p0, \
        const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, \
        float* __restrict__ y, int M, int K, int N, const int* __restrict__ row_off, int E,               \
        const float* __restrict__ tbias, int trans)                                                       \
    {                                                                                                     \
        gemm_body<FMT, Tile<FMT, BM_, TN_, NW_, PF_>, false>(xh, rscale, p0, p1, sc, mn, y, M, K, N, row_off, E, \
                                                            0, 0, tbias, trans);                         \
    }
// Expert-grouped kernels, q4 only: brik_gemmg_q4_<tile>, a 1-D grid over (pair, column tile, matrix)
// with `mats` matrices: the second (codes p0b, scales scb, mins mnb, into yb) is multiplied by the same
// staged rows (the gate and up projections of an MoE layer in one launch). Blocks are dealt to the 8
// XCDs round-robin by linear index, so the index is decoded to put every block of one (expert, row
// tile) pair, all its column tiles of both matrices, on the same XCD, back to back: the pair's staged
// rows then come from HBM once and stay in that XCD's L2 for all of them. Indices past the last pair
// (the grid is rounded up to a multiple of 8 pairs) exit. Experts hold few rows, so a launch has few blocks per
// CU, each bound by the latency of its steps: the narrow 8-wave tiles (BM <= 64, one column block per
// wave, PF = 1) are held to 128 VGPRs so that two blocks share a CU.
constexpr int grouped_waves_per_eu(int bm, int tn, int nw, int pf) { return bm <= 64 && tn == 1 && nw == 8 && pf == 1 ? 4 : 1; }
#define BRIK_GEMM_GROUPED(FMTN, FMT, BM_, TN_, NW_, PF_, SUFFIX)                                          \
    extern "C" __global__ __launch_bounds__(64 * NW_)                                                     \
    __attribute__((amdgpu_waves_per_eu(grouped_waves_per_eu(BM_, TN_, NW_, PF_))))                                 \
    void brik_gemmg_##FMTN##_##BM_##x##TN_##SUFFIX(                                                       \
        const uint16_t* __restrict__ xh, const float* __restrict__ rscale, const uint8_t* __restrict__ p0, \
        const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, \
        float* __restrict__ y, int M, int K, int N, const int* __restrict__ row_off, int E,               \
        const uint8_t* __restrict__ p0b, const uint16_t* __restrict__ scb, const uint16_t* __restrict__ mnb, \
        float* __restrict__ yb, int mats)                                                                 \
    {                                                                                                     \
        using T_ = Tile<FMT, BM_, TN_, NW_, PF_>;                                                         \
        const int per = (N + T_::BN - 1) / T_::BN * mats;   /* blocks of one pair */                      \
        const int s = (int)(blockIdx.x >> 3), r = s % per;                                                \
        const int gtile = s / per * 8 + (int)(blockIdx.x & 7);                                            \
        if (gtile >= (M + BM_ - 1) / BM_ + E) return;                                                     \
        if (r % mats) {                                                                                   \
            p0 = p0b;                                                                                     \
            sc = scb;                                                                                     \
            mn = mnb;                                                                                     \
            y = yb;                                                                                       \
        }                                                                                                 \
        gemm_body<FMT, T_, true>(xh, rscale, p0, p1, sc, mn, y, M, K, N, row_off, E, gtile, r / mats);   \
    }

// Tiles in the order of the runtime's table: (BM, TN, waves, PF, name suffix).
#define BRIK_GEMM_TILE_LIST(X, FMTN, FMT)                                                                     \
    X(FMTN, FMT, 128, 2, 4, 1, ) X(FMTN, FMT, 128, 1, 4, 1, ) X(FMTN, FMT, 128, 3, 4, 1, )                \
    X(FMTN, FMT, 64, 2, 4, 1, ) X(FMTN, FMT, 64, 1, 4, 1, ) X(FMTN, FMT, 64, 3, 4, 1, )                   \
    X(FMTN, FMT, 32, 2, 4, 1, ) X(FMTN, FMT, 32, 1, 4, 1, ) X(FMTN, FMT, 32, 3, 4, 1, )                   \
    X(FMTN, FMT, 96, 2, 4, 1, ) X(FMTN, FMT, 96, 1, 4, 1, ) X(FMTN, FMT, 96, 3, 4, 1, )                   \
    X(FMTN, FMT, 128, 1, 8, 1, w8) X(FMTN, FMT, 96, 1, 8, 1, w8) X(FMTN, FMT, 64, 1, 8, 1, w8)            \
    X(FMTN, FMT, 32, 1, 8, 1, w8) X(FMTN, FMT, 64, 2, 8, 1, w8)                                           \
    X(FMTN, FMT, 32, 1, 8, 4, w8p4) X(FMTN, FMT, 64, 1, 8, 3, w8p3) X(FMTN, FMT, 32, 1, 4, 4, p4)         \
    X(FMTN, FMT, 64, 1, 4, 3, p3) X(FMTN, FMT, 32, 1, 8, 2, w8p2) X(FMTN, FMT, 64, 1, 8, 2, w8p2)

BRIK_GEMM_TILE_LIST(BRIK_GEMM_DENSE, q4, FMT_Q4)
BRIK_GEMM_TILE_LIST(BRIK_GEMM_DENSE, q8, FMT_Q8)
BRIK_GEMM_TILE_LIST(BRIK_GEMM_DENSE, q3, FMT_Q3)
BRIK_GEMM_TILE_LIST(BRIK_GEMM_GROUPED, q4, FMT_Q4)

// Adaptive expert-grouped kernels (gemm_grouped_adaptive): brik_gemmg_q4_64a<suffix> runs a 64-row tile
// whose expert tile has at most 32 live rows as the 32-row tile of the same columns and waves.
#define BRIK_GEMM_GROUPED_ADAPTIVE(NW_, SUFFIX)                                                           \
    extern "C" __global__ __launch_bounds__(64 * NW_)                                                     \
    __attribute__((amdgpu_waves_per_eu(grouped_waves_per_eu(64, 1, NW_, 1))))                            \
    void brik_gemmg_q4_64a##SUFFIX(                                                                       \
        const uint16_t* __restrict__ xh, const float* __restrict__ rscale, const uint8_t* __restrict__ p0, \
        const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, \
        float* __restrict__ y, int M, int K, int N, const int* __restrict__ row_off, int E,               \
        const uint8_t* __restrict__ p0b, const uint16_t* __restrict__ scb, const uint16_t* __restrict__ mnb, \
        float* __restrict__ yb, int mats)                                                                 \
    {                                                                                                     \
        using TL_ = Tile<FMT_Q4, 64, 1, NW_, 1>;                                                          \
        using TS_ = Tile<FMT_Q4, 32, 1, NW_, 1>;                                                          \
        const int per = (N + TL_::BN - 1) / TL_::BN * mats;                                               \
        const int s = (int)(blockIdx.x >> 3), r = s % per;                                                \
        const int gtile = s / per * 8 + (int)(blockIdx.x & 7);                                            \
        if (gtile >= (M + 63) / 64 + E) return;                                                           \
        if (r % mats) {                                                                                   \
            p0 = p0b;                                                                                     \
            sc = scb;                                                                                     \
            mn = mnb;                                                                                     \
            y = yb;                                                                                       \
        }                                                                                                 \
        gemm_grouped_adaptive<FMT_Q4, TL_, TS_>(xh, rscale, p0, p1, sc, mn, y, M, K, N, row_off, E, gtile, r / mats); \
    }
BRIK_GEMM_GROUPED_ADAPTIVE(4, )
BRIK_GEMM_GROUPED_ADAPTIVE(8, w8)
// f16 weights (the reference's MATMUL_T_F16W for M > 1, K % 32 == 0): the one-column-block tiles,
// brik_gemm_f16_<BM>x1[w8]; the codes are the weights, so there is nothing to dequantize
BRIK_GEMM_DENSE(f16, FMT_F16, 128, 1, 8, 1, w8) BRIK_GEMM_DENSE(f16, FMT_F16, 96, 1, 8, 1, w8)
BRIK_GEMM_DENSE(f16, FMT_F16, 64, 1, 8, 1, w8) BRIK_GEMM_DENSE(f16, FMT_F16, 32, 1, 8, 1, w8)
BRIK_GEMM_DENSE(f16, FMT_F16, 128, 1, 4, 1, ) BRIK_GEMM_DENSE(f16, FMT_F16, 96, 1, 4, 1, )
BRIK_GEMM_DENSE(f16, FMT_F16, 64, 1, 4, 1, ) BRIK_GEMM_DENSE(f16, FMT_F16, 32, 1, 4, 1, )

// Split-K few-row kernels: brik_gemm_sk_<fmt>_k<KSL> (32 x 128 tiles, 256 threads, K slices of at most
// KSL steps of 128); grid (column tiles, row tiles or expert row-tile pairs, slices).
#define BRIK_GEMM_SK(FMTN, FMT, KSL_)                                                                     \
    extern "C" __global__ __launch_bounds__(256) void brik_gemm_sk_##FMTN##_k##KSL_(                       \
        const uint16_t* __restrict__ xh, const float* __restrict__ rscale, const uint8_t* __restrict__ p0, \
        const uint8_t* __restrict__ p1, const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, \
        float* __restrict__ y, int M, int K, int N, const int* __restrict__ row_off, int E,               \
        float* __restrict__ part)                                                                         \
    {                                                                                                     \
        gemm_sk_body<FMT, KSL_>(xh, rscale, p0, p1, sc, mn, y, M, K, N, row_off, E, part);                 \
    }
// y[i] = sum over slices q = 0 .. ks - 1, in that order, of part[q * n + i], for i < n (n = rows x N of a
// split-K launch); float4 accesses when n % 4 == 0.
extern "C" __global__ __launch_bounds__(256) void brik_splitk_reduce(const float* __restrict__ part,
                                                                    float* __restrict__ y, size_t n, int ks)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    if ((n & 3) == 0) {
        const size_t n4 = n / 4;
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
            f32x4_t v = *(const f32x4_t*)(part + 4 * i);
            for (int q = 1; q < ks; ++q) v = v + *(const f32x4_t*)(part + (size_t)q * n + 4 * i);
            *(f32x4_t*)(y + 4 * i) = v;
        }
        return;
    }
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float v = part[i];
        for (int q = 1; q < ks; ++q) v += part[(size_t)q * n + i];
        y[i] = v;
    }
}

BRIK_GEMM_SK(q4, FMT_Q4, 2) BRIK_GEMM_SK(q4, FMT_Q4, 4) BRIK_GEMM_SK(q4, FMT_Q4, 8)
BRIK_GEMM_SK(q8, FMT_Q8, 2) BRIK_GEMM_SK(q8, FMT_Q8, 4) BRIK_GEMM_SK(q8, FMT_Q8, 8)
BRIK_GEMM_SK(q3, FMT_Q3, 2) BRIK_GEMM_SK(q3, FMT_Q3, 4) BRIK_GEMM_SK(q3, FMT_Q3, 8)
