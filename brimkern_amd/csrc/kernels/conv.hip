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
//   * direct, for any shape: brik_conv2d_direct_<fmt>, one output per thread accumulating in f32 in
//     the reference's (ci, ky, kx) order, each weight dequantized as dequantizeQ8 / Q4 do.
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

template <int FMT>
__device__ __forceinline__ void conv_direct(const float* __restrict__ inp, const void* __restrict__ p0,
                                            const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn,
                                            const float* __restrict__ bias, float* __restrict__ out, int Cin, int H,
                                            int W, int Cout, int kh, int kw, int stride, int pad, int OH, int OW)
{
    const long np = (long)OH * OW;
    for (long idx = (long)blockIdx.x * 256 + threadIdx.x; idx < (long)Cout * np; idx += (long)gridDim.x * 256) {
        const int ox = (int)(idx % OW), oy = (int)((idx / OW) % OH), co = (int)(idx / np);
        float acc = bias ? bias[co] : 0.f;
        for (int ci = 0; ci < Cin; ++ci) {
            const float* ib = inp + (size_t)ci * H * W;
            const uint32_t wb = (uint32_t)(((size_t)co * Cin + ci) * kh * kw);
            for (int ky = 0; ky < kh; ++ky) {
                const int iy = oy * stride + ky - pad;
                if (iy < 0 || iy >= H) continue;
                for (int kx = 0; kx < kw; ++kx) {
                    const int ix = ox * stride + kx - pad;
                    if (ix < 0 || ix >= W) continue;
                    acc = fmaf(ib[(size_t)iy * W + ix], conv_weight<FMT>(p0, sc, mn, wb + ky * kw + kx), acc);
                }
            }
        }
        out[idx] = acc;
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
// [0 4 1 5 2 6 3 7] order per 8 elements, zero padding to Kp). One wave per row.
extern "C" __global__ __launch_bounds__(256) void brik_xprep_im2col_f16(
    const float* __restrict__ inp, uint16_t* __restrict__ xh, float* __restrict__ rscale, int M, int K, int Kp,
    int H, int W, int kh, int kw, int stride, int pad, int OW)
{
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;     // a whole wave; no block-level synchronisation follows
    const int lane = threadIdx.x & 63;
    const int oy = m / OW, ox = m % OW, kk = kh * kw;
    const int y0 = oy * stride - pad, x0 = ox * stride - pad;
    uint16_t* hr = xh + (size_t)m * Kp;
    const int nch = K / 8, nchp = Kp / 8;
    // the 8 taps of chunk c, walking (ci, ky, kx) from k = 8 c
    auto gather = [&](int c, f32x4_t& a, f32x4_t& b) {
        float v[8];
        int k = 8 * c, ci = k / kk, r = k - ci * kk, ky = r / kw, kx = r - ky * kw;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int iy = y0 + ky, ix = x0 + kx;
            v[j] = (iy >= 0 && iy < H && ix >= 0 && ix < W) ? inp[((size_t)ci * H + iy) * W + ix] : 0.f;
            if (++kx == kw) {
                kx = 0;
                if (++ky == kh) {
                    ky = 0;
                    ++ci;
                }
            }
        }
        a = f32x4_t{v[0], v[1], v[2], v[3]};
        b = f32x4_t{v[4], v[5], v[6], v[7]};
    };
    auto scale_of = [&](float mx, float& up) {
        int e = 15;                                                    // zero / non-finite rows: scale 1
        if (mx > 0.f && mx <= 3.4028235e38f) (void)frexpf(mx, &e);
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
            if (c < nch) gather(c, a[i], b[i]);
            mx = fmaxf(mx, absmax8(a[i], b[i]));
        }
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
    for (int c = lane; c < nch; c += 64) {
        f32x4_t a, b;
        gather(c, a, b);
        mx = fmaxf(mx, absmax8(a, b));
    }
    float up;
    scale_of(wave_max(mx), up);
    for (int c = lane; c < nchp; c += 64) {
        f32x4_t a = {0.f, 0.f, 0.f, 0.f}, b = {0.f, 0.f, 0.f, 0.f};
        if (c < nch) gather(c, a, b);
        *(half8_t*)(hr + c * 8) = to_h8(a, b, up);
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
