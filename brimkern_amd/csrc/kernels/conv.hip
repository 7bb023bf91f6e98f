// 2-D convolution with a .brik q8 / q4 weight dequantized on the fly: the reference's conv2d_direct_q8
// and conv2d_direct_q4 (src/lib/webgpu/shaders.ts:1026-1123; recConv2dDirectQ8 / Q4 at
// kernels.ts:1233-1256):
//   out[co, oy, ox] = bias[co] + sum_{ci, ky, kx} inp[ci, oy s + ky - pad, ox s + kx - pad] * w[co, ci, ky, kx]
// over the taps inside the image, with the weight a flat OIHW tensor quantized in 32-element groups of
// its flat index (groups may straddle kernels and output channels), inp [Cin, H, W] and out
// [Cout, OH, OW] f32, OH = (H + 2 pad - kh) / s + 1 (likewise OW).
//
// Two paths (chosen by the host):
//   * implicit GEMM, when K = Cin kh kw is a multiple of 32 (then the groups of a weight row are
//     exactly the matmul's, W[Cout, K]): brik_xprep_im2col_f16 stages the im2col rows of the input
//     (one per output pixel, K taps) as scaled f16 rows, the way brik_xprep_f16 stages matmul
//     activations, the MFMA GEMM of gemm.hip computes Y[pixels, Cout] = X . deq(W)^T, and
//     brik_conv_out transposes Y to [Cout, pixels] adding the bias;
//   * direct, for any shape: brik_conv2d_direct_<fmt>, every output accumulated in f32 in the
//     reference's (ci, ky, kx) order over the in-image taps, each weight dequantized as dequantizeQ8 /
//     Q4 do. A block owns 256 output pixels x 16 output channels: it dequantizes the weights of its
//     channels into LDS a chunk of 256 (ci, ky, kx) taps at a time, and every thread runs the 16
//     channels of its pixel, so each input value it loads feeds 16 FMAs and each weight is dequantized
//     once per block instead of once per output.
#include "common.h"

namespace {

// Weight i of the flat tensor: q8 codes[i] * s, q4 nibble i * s + m (one rounding, as the f64
// expression of dequantizeQ8 / dequantizeQ4 stored into a Float32Array).
template <int FMT>
__device__ __forceinline__ float conv_weight(const void* __restrict__ p0, const uint16_t* __restrict__ sc,
                                             const uint16_t* __restrict__ mn, uint32_t i)
{
    const float s = f16_bits_to_f32(sc[i >> 5]);
    if (FMT == FMT_Q8) return (float)static_cast<const int8_t*>(p0)[i] * s;
    const uint32_t q = (static_cast<const uint8_t*>(p0)[i >> 1] >> ((i & 1) * 4)) & 15u;
    return fmaf((float)q, s, f16_bits_to_f32(mn[i >> 5]));
}

constexpr int DC_PIX = 256;     // output pixels per block (one per thread)
constexpr int DC_CO = 16;       // output channels per block (accumulators per thread)
constexpr int DC_TAPS = 256;    // (ci, ky, kx) taps of a weight chunk in LDS
constexpr int DC_LD = 20;       // LDS row stride of a tap's 16 weights (floats; 16-byte aligned rows)
constexpr int DC_U = 8;         // taps whose input loads a thread issues together

// Block (bx, by): pixels p = 256 bx + t (p = oy OW + ox), channels 16 by + j. For each chunk of 256 taps
// k = (ci kh + ky) kw + kx (the flat weight order within a channel), the block dequantizes the 16 x 256
// weights into LDS, then every thread walks the chunk's taps in order and adds x * w to its 16 sums. The
// walk's position (ci, ky, kx) is the same for every thread (scalar registers); a thread's input offset
// is its origin plus ci H W + ky W + kx, and a tap is inside the image when bit ky of its row mask and
// bit kx of its column mask are set (kernels of up to 32 x 32; larger ones test the coordinates). When
// every weight of the chunk is finite an outside tap reads x = 0 (an offset past the end of a buffer
// resource) and its FMA adds a signed zero, so the walk has no branch per tap; a chunk holding an
// infinite or NaN weight skips the outside taps one by one as the reference does (0 * inf is NaN).
template <int FMT>
__device__ __forceinline__ void conv_direct(const float* __restrict__ inp, const void* __restrict__ p0,
                                            const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn,
                                            const float* __restrict__ bias, float* __restrict__ out, int Cin, int H,
                                            int W, int Cout, int kh, int kw, int stride, int pad, int OH, int OW)
{
    __shared__ __attribute__((aligned(16))) float wl[DC_TAPS * DC_LD];
    const int t = threadIdx.x;
    const int M = OH * OW;
    const int p = (int)blockIdx.x * DC_PIX + t;
    const int co0 = (int)blockIdx.y * DC_CO;
    const bool live = p < M;
    const int oy = live ? p / OW : 0, ox = live ? p % OW : 0;
    const int y0 = oy * stride - pad, x0 = ox * stride - pad;
    const int taps = kh * kw, K = Cin * taps;
    const bool masks = kh <= 32 && kw <= 32;
    uint32_t rmask = 0u, cmask = 0u;
    if (masks && live) {
        for (int ky = 0; ky < kh; ++ky) rmask |= (y0 + ky >= 0 && y0 + ky < H) ? 1u << ky : 0u;
        for (int kx = 0; kx < kw; ++kx) cmask |= (x0 + kx >= 0 && x0 + kx < W) ? 1u << kx : 0u;
    }
    const long origin = (long)y0 * W + x0;         // may be negative; only in-image taps are read
    // the branch-free walk reads the input through a buffer resource (32-bit byte offsets); with fewer
    // than 2^29 elements its range is below 2^31 bytes, so the offset 2^32 - 16 given to the taps
    // outside the image lies past it
    const bool fast = masks && (long)Cin * H * W < (1L << 29);
    const brsrc_t rin = make_rsrc(inp, fast ? (uint32_t)((long)Cin * H * W * 4) : 0u);
    float acc[DC_CO];
#pragma unroll
    for (int j = 0; j < DC_CO; ++j) acc[j] = bias && co0 + j < Cout ? bias[co0 + j] : 0.f;
    // the walk's position, the same for every thread
    int ci = 0, ky = 0, kx = 0;
    long uoff = 0;                                   // ci H W + ky W
    for (int k0 = 0; k0 < K; k0 += DC_TAPS) {
        const int nk = min(DC_TAPS, K - k0);
        __syncthreads();                          // the previous chunk's reads are done
        bool fin = true;
        const int nkp = (nk + DC_U - 1) / DC_U * DC_U;    // rows past nk (the last chunk) hold zeros
        for (int e = t; e < nkp * DC_CO; e += DC_PIX) {
            const int kk = e % nkp, j = e / nkp, co = co0 + j;
            const float w = co < Cout && kk < nk ? conv_weight<FMT>(p0, sc, mn, (uint32_t)((size_t)co * K + k0 + kk))
                                                  : 0.f;
            fin = fin && __builtin_isfinite(w);
            wl[kk * DC_LD + j] = w;
        }
        // every weight of the chunk finite: an outside tap then adds x = 0 times a finite weight, a
        // signed zero, which leaves every sum as skipping the tap does (up to the sign of a zero sum),
        // so the taps need no branch; otherwise they are skipped one by one
        const bool all_fin = __syncthreads_and(fin);
        if (all_fin && fast) {
            // the input loads of the next DC_U taps go out before the sums of these
            auto fetch = [&](float (&xv)[DC_U], int kb) {
#pragma unroll
                for (int u = 0; u < DC_U; ++u) {
                    const bool ok = (((rmask >> ky) & (cmask >> kx) & 1u) != 0u) & (kb + u < nk);
                    // an offset past the resource's end reads 0: no branch and no select per tap
                    const uint32_t off = ok ? (uint32_t)(origin + uoff + kx) * 4u : 0xFFFFFFF0u;
                    xv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rin, off, 0u, 0));
                    if (++kx == kw) {
                        kx = 0;
                        uoff += W;
                        if (++ky == kh) {
                            ky = 0;
                            ++ci;
                            uoff = (long)ci * H * W;
                        }
                    }
                }
            };
            float xa[DC_U], xb[DC_U];
            fetch(xa, 0);
            for (int k = 0; k < nk; k += DC_U) {
                if (k + DC_U < nk) fetch(xb, k + DC_U);
#pragma unroll
                for (int u = 0; u < DC_U; ++u) {
                    const f32x4_t* wr = reinterpret_cast<const f32x4_t*>(wl + (k + u) * DC_LD);
#pragma unroll
                    for (int q = 0; q < DC_CO / 4; ++q) {
                        const f32x4_t w = wr[q];
                        acc[4 * q + 0] = fmaf(xa[u], w.x, acc[4 * q + 0]);
                        acc[4 * q + 1] = fmaf(xa[u], w.y, acc[4 * q + 1]);
                        acc[4 * q + 2] = fmaf(xa[u], w.z, acc[4 * q + 2]);
                        acc[4 * q + 3] = fmaf(xa[u], w.w, acc[4 * q + 3]);
                    }
                }
#pragma unroll
                for (int u = 0; u < DC_U; ++u) xa[u] = xb[u];
            }
            continue;
        }
        for (int k = 0; k < nk; k += DC_U) {
            float xv[DC_U];
            bool in[DC_U];
#pragma unroll
            for (int u = 0; u < DC_U; ++u) {
                bool ok;
                if (masks) ok = ((rmask >> ky) & (cmask >> kx) & 1u) != 0u;
                else ok = live && y0 + ky >= 0 && y0 + ky < H && x0 + kx >= 0 && x0 + kx < W;
                in[u] = ok && k + u < nk;
                xv[u] = inp[in[u] ? origin + uoff + kx : 0];
                if (++kx == kw) {
                    kx = 0;
                    uoff += W;
                    if (++ky == kh) {
                        ky = 0;
                        ++ci;
                        uoff = (long)ci * H * W;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < DC_U; ++u) {
                if (!in[u]) continue;
                const f32x4_t* wr = reinterpret_cast<const f32x4_t*>(wl + (k + u) * DC_LD);
#pragma unroll
                for (int q = 0; q < DC_CO / 4; ++q) {
                    const f32x4_t w = wr[q];
                    acc[4 * q + 0] = fmaf(xv[u], w.x, acc[4 * q + 0]);
                    acc[4 * q + 1] = fmaf(xv[u], w.y, acc[4 * q + 1]);
                    acc[4 * q + 2] = fmaf(xv[u], w.z, acc[4 * q + 2]);
                    acc[4 * q + 3] = fmaf(xv[u], w.w, acc[4 * q + 3]);
                }
            }
        }
    }
    if (live) {
#pragma unroll
        for (int j = 0; j < DC_CO; ++j)
            if (co0 + j < Cout) out[(size_t)(co0 + j) * M + p] = acc[j];
    }
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void brik_conv2d_direct_q8(
    const float* __restrict__ inp, const int8_t* __restrict__ codes, const uint16_t* __restrict__ sc,
    const float* __restrict__ bias, float* __restrict__ out, int Cin, int H, int W, int Cout, int kh, int kw,
    int stride, int pad, int OH, int OW)
{
    conv_direct<FMT_Q8>(inp, codes, sc, nullptr, bias, out, Cin, H, W, Cout, kh, kw, stride, pad, OH, OW);
}

extern "C" __global__ __launch_bounds__(256) void brik_conv2d_direct_q4(
    const float* __restrict__ inp, const uint8_t* __restrict__ nib, const uint16_t* __restrict__ sc,
    const uint16_t* __restrict__ mn, const float* __restrict__ bias, float* __restrict__ out, int Cin, int H, int W,
    int Cout, int kh, int kw, int stride, int pad, int OH, int OW)
{
    conv_direct<FMT_Q4>(inp, nib, sc, mn, bias, out, Cin, H, W, Cout, kh, kw, stride, pad, OH, OW);
}

// im2col staging for the MFMA GEMM: row m = output pixel (oy, ox) = (m / OW, m % OW), element k =
// (ci, ky, kx) = (k / (kh kw), (k / kw) % kh, k % kw) is the input tap or 0 outside the image. The row
// is written exactly as brik_xprep_f16 writes an activation row (power-of-two row scale, f16, the
// [0 4 1 5 2 6 3 7] order per 8 elements, zero padding to Kp). Two launches:
//   a. brik_conv_chanmax: cmax[p] = max over the channels of |inp[ci, p]| for every input position p
//      (half waves along positions, so every load is contiguous; 32 groups split the channels);
//   b. brik_xprep_im2col_f16: a row's maximum is the maximum of cmax over its kh x kw in-image taps (the
//      same set of values; out-of-image taps are 0), so no pass over the row is needed for its scale.
//      Lanes are 64 consecutive pixels and a wave takes 8 consecutive chunks of 8 elements of their
//      rows: each tap load is contiguous across the wave; the rows go out through LDS, 512 contiguous
//      bytes per row and store.
// fmaxf drops NaN here as in brik_xprep_f16. (One wave per row gathering its own taps, the first form,
// issued 64 scattered 4-byte loads per instruction: 29 us on a 320 x 64 x 64 3 x 3 input.)
extern "C" __global__ __launch_bounds__(1024) void brik_conv_chanmax(const float* __restrict__ inp,
                                                                    float* __restrict__ cmax, int Cin, int HW)
{
    // 32 positions per block (one per lane of a half wave), 32 channel groups; a thread's loads of
    // 8 channels at a time are independent, so they are in flight together
    __shared__ float part[32][33];
    const int q = threadIdx.x & 31, g = threadIdx.x >> 5;
    const int p = blockIdx.x * 32 + q;
    float mx = 0.f;
    if (p < HW)
        for (int ci = g; ci < Cin; ci += 256) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = ci + 32 * u < Cin ? fabsf(inp[(size_t)(ci + 32 * u) * HW + p]) : 0.f;
#pragma unroll
            for (int u = 0; u < 8; ++u) mx = fmaxf(mx, t[u]);
        }
    part[g][q] = mx;
    __syncthreads();
    if (g == 0 && p < HW) {
#pragma unroll
        for (int k = 1; k < 32; ++k) mx = fmaxf(mx, part[k][q]);
        cmax[p] = mx;
    }
}

// The pixel's row scale from the channel maxima of its in-image taps (as brik_xprep_f16 scales a row).
__device__ __forceinline__ float im2col_scale(const float* __restrict__ cmax, int y0, int x0, int H, int W, int kh,
                                              int kw, int& e)
{
    // every load in range (clamped coordinates) and unconditional, a tap outside the image then
    // dropped: the loads issue together instead of one guarded round trip each
    float mx = 0.f;
    for (int ky = 0; ky < kh; ++ky) {
        const int iy = y0 + ky, cy = min(max(iy, 0), H - 1);
        for (int kx = 0; kx < kw; ++kx) {
            const int ix = x0 + kx, cx = min(max(ix, 0), W - 1);
            const float c = cmax[cy * W + cx];
            mx = fmaxf(mx, (iy >= 0 && iy < H && ix >= 0 && ix < W) ? c : 0.f);
        }
    }
    e = 15;                                                        // zero / non-finite rows: scale 1
    if (mx > 0.f && mx <= 3.4028235e38f) (void)frexpf(mx, &e);    // mx = f * 2^e, f in [0.5, 1)
    return ldexpf(1.f, 15 - e);
}

constexpr int IM2COL_CPT = 8;    // chunks of 8 elements per thread

extern "C" __global__ __launch_bounds__(256) void brik_xprep_im2col_f16(
    const float* __restrict__ inp, const float* __restrict__ cmax, uint16_t* __restrict__ xh,
    float* __restrict__ rscale, int M, int K, int Kp, int Cin, int H, int W, int kh, int kw, int stride, int pad,
    int OW)
{
    // w through readfirstlane: the compiler then keeps the tap walk below, uniform per wave, in scalar
    // registers, and the buffer loads' scalar offset needs no per-lane loop
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // rows past M compute row M - 1 again (in range) and are not written
    const int m = min((int)blockIdx.x * 64 + lane, M - 1);
    const int oy = m / OW, ox = m % OW, kk = kh * kw;
    const int y0 = oy * stride - pad, x0 = ox * stride - pad;
    int e;
    const float up = im2col_scale(cmax, y0, x0, H, W, kh, kw, e);
    if (blockIdx.y == 0 && w == 0 && (int)blockIdx.x * 64 + lane < M) rscale[m] = ldexpf(1.f, e - 15);
    const int nchp = Kp / 8;
    const int c0 = (blockIdx.y * 4 + w) * IM2COL_CPT;              // the same for the whole wave
    // Taps through a buffer resource: the per-thread offset is the pixel's corner (y0, x0), the tap's
    // (ci, ky, kx) offset is uniform (a scalar register, added by the addressing hardware), and a tap
    // outside the image gets an offset past the end of the buffer, which loads 0 without an access.
    // The resource starts pad rows and pad columns before the input, so every corner offset is
    // nonnegative (y0, x0 >= -pad); only taps inside the image are ever addressed. The input has fewer
    // than 2^29 elements here (the host checks), so the offsets stay below 2^31.
    const int lead = pad * W + pad;
    const brsrc_t rin = make_rsrc((const void*)((uintptr_t)inp - (uintptr_t)lead * 4),
                                  (uint32_t)(((size_t)Cin * H * W + lead) * 4));
    uint64_t rowbits = 0, colbits = 0;                             // bit ky / kx: the tap row / column is inside
    for (int ky = 0; ky < kh; ++ky) rowbits |= (uint64_t)(y0 + ky >= 0 && y0 + ky < H) << ky;
    for (int kx = 0; kx < kw; ++kx) colbits |= (uint64_t)(x0 + kx >= 0 && x0 + kx < W) << kx;
    const uint32_t vbase = (uint32_t)((y0 * W + x0 + lead) * 4);
    // every tap of the thread's chunks is loaded before any is converted, so the loads are in flight
    // together (one memory round trip per thread)
    float v[IM2COL_CPT][8];
    {
        const int k0 = 8 * c0;
        int ci = k0 / kk, r = k0 - ci * kk, ky = r / kw, kx = r - ky * kw;
#pragma unroll
        for (int j = 0; j < IM2COL_CPT; ++j)
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const bool live = 8 * (c0 + j) + t < K;                // uniform; ci < Cin when set
                const bool in = live && ((rowbits >> ky) & (colbits >> kx) & 1u);
                const int soff = live ? ((ci * H + ky) * W + kx) * 4 : 0;
                v[j][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rin, in ? vbase : 0x80000000u,
                                                                                       soff, 0));
                if (++kx == kw) {
                    kx = 0;
                    if (++ky == kh) {
                        ky = 0;
                        ++ci;
                    }
                }
            }
    }
    // Rows of the block through LDS: [64 rows][32 chunks] of 16 bytes, chunk c of a row at
    // (c ^ (row & 31)) so the writes below (8 chunks of one row per lane) and the reads (consecutive
    // chunks of two rows per wave instruction) are spread over the banks. Each wave then writes 16 rows,
    // two per instruction, 512 contiguous bytes each: every lane writing its own row instead put 64 rows
    // 6 KB apart into one instruction (21 us for this launch on the 320 x 64 x 64 3 x 3 input).
    __shared__ __attribute__((aligned(16))) half8_t tile[64 * 32];
    const int row = lane, cb = w * IM2COL_CPT;
#pragma unroll
    for (int j = 0; j < IM2COL_CPT; ++j)
        tile[row * 32 + ((cb + j) ^ (row & 31))] =
            to_h8(f32x4_t{v[j][0], v[j][1], v[j][2], v[j][3]}, f32x4_t{v[j][4], v[j][5], v[j][6], v[j][7]}, up);
    __syncthreads();
    const int cc = lane & 31, cblk = blockIdx.y * 32;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int rr = w * 16 + 2 * i + (lane >> 5);                // the wave's rows 16 w .. 16 w + 15
        const int mm = blockIdx.x * 64 + rr;
        if (mm < M && cblk + cc < nchp)
            *(half8_t*)(xh + (size_t)mm * Kp + (cblk + cc) * 8) = tile[rr * 32 + (cc ^ (rr & 31))];
    }
}

// 3 x 3 form: a wave takes 8 whole channels of its 64 pixels, 72 taps = 9 chunks of 8 (a window
// that starts on a channel, so every tap's place in the row is a compile-time constant), a block of 4
// waves 32 channels (8 waves, 1152 bytes of each row in whole cache lines, measured slower: 11.6 against
// 10.3 us). The 9 per-pixel tap offsets (the corner, or past the end for a tap outside the image)
// are computed once; each load then only adds the uniform offset of its channel and tap, so the walk
// costs no per-tap arithmetic. The rows go out through LDS as in the generic form.
constexpr int IM2COL3_WAVES = 4;
constexpr int IM2COL3_CPB = 9 * IM2COL3_WAVES;    // chunks per block: 36

extern "C" __global__ __launch_bounds__(64 * IM2COL3_WAVES) void brik_xprep_im2col3_f16(
    const float* __restrict__ inp, const float* __restrict__ cmax, uint16_t* __restrict__ xh,
    float* __restrict__ rscale, int M, int K, int Kp, int Cin, int H, int W, int stride, int pad, int OW)
{
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m = min((int)blockIdx.x * 64 + lane, M - 1);        // rows past M: row M - 1, not written
    const int oy = m / OW, ox = m % OW;
    const int y0 = oy * stride - pad, x0 = ox * stride - pad;
    int e;
    const float up = im2col_scale(cmax, y0, x0, H, W, 3, 3, e);
    if (blockIdx.y == 0 && w == 0 && (int)blockIdx.x * 64 + lane < M) rscale[m] = ldexpf(1.f, e - 15);
    // taps through a buffer resource starting pad rows and columns before the input (see the generic
    // form); the host keeps every offset below 2^31
    const int lead = pad * W + pad;
    const brsrc_t rin = make_rsrc((const void*)((uintptr_t)inp - (uintptr_t)lead * 4),
                                  (uint32_t)(((size_t)Cin * H * W + lead) * 4));
    const uint32_t vbase = (uint32_t)((y0 * W + x0 + lead) * 4);
    uint32_t voff[3][3];
#pragma unroll
    for (int ky = 0; ky < 3; ++ky)
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
            const bool in = y0 + ky >= 0 && y0 + ky < H && x0 + kx >= 0 && x0 + kx < W;
            voff[ky][kx] = in ? vbase : 0x80000000u;
        }
    const int ci0 = (blockIdx.y * IM2COL3_WAVES + w) * 8;           // uniform
    float v[72];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const bool live = ci0 + c < Cin;                            // uniform: channels past Cin are padding
#pragma unroll
        for (int ky = 0; ky < 3; ++ky)
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                const int soff = live ? (((ci0 + c) * H + ky) * W + kx) * 4 : 0;
                v[c * 9 + ky * 3 + kx] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(rin, live ? voff[ky][kx] : 0x80000000u, soff, 0));
            }
    }
    __shared__ __attribute__((aligned(16))) half8_t tile[64 * (IM2COL3_CPB + 1)];
#pragma unroll
    for (int c = 0; c < 9; ++c)
        tile[lane * (IM2COL3_CPB + 1) + w * 9 + c] =
            to_h8(f32x4_t{v[8 * c], v[8 * c + 1], v[8 * c + 2], v[8 * c + 3]},
                  f32x4_t{v[8 * c + 4], v[8 * c + 5], v[8 * c + 6], v[8 * c + 7]}, up);
    __syncthreads();
    const int nchp = Kp / 8, cblk = blockIdx.y * IM2COL3_CPB;
    for (int idx = threadIdx.x; idx < 64 * IM2COL3_CPB; idx += 64 * IM2COL3_WAVES) {
        const int rr = idx / IM2COL3_CPB, cc = idx - rr * IM2COL3_CPB;
        const int mm = blockIdx.x * 64 + rr;
        if (mm < M && cblk + cc < nchp)
            *(half8_t*)(xh + (size_t)mm * Kp + (cblk + cc) * 8) = tile[rr * (IM2COL3_CPB + 1) + cc];
    }
}

// out[co, p] = y[p, co] + bias[co] for P pixels and Cout channels: 32 x 32 tiles through LDS, so both
// the reads of y and the writes of out are row-contiguous.
extern "C" __global__ __launch_bounds__(256) void brik_conv_out(const float* __restrict__ y,
                                                                const float* __restrict__ bias,
                                                                float* __restrict__ out, int P, int Cout)
{
    __shared__ float tile[32][33];
    const int p0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;       // 32 x 8 threads
#pragma unroll
    for (int r = ty; r < 32; r += 8) {
        const int p = p0 + r, c = c0 + tx;
        if (p < P && c < Cout) tile[r][tx] = y[(size_t)p * Cout + c];
    }
    __syncthreads();
#pragma unroll
    for (int r = ty; r < 32; r += 8) {
        const int c = c0 + r, p = p0 + tx;
        if (p < P && c < Cout) out[(size_t)c * P + p] = tile[tx][r] + (bias ? bias[c] : 0.f);
    }
}
