// y[M, N] = x[M, K] . W[N, K]^T with W stored as IEEE f16 and x, y f32: the reference's f16-weight
// matmul MATMUL_T_F16W (src/lib/webgpu/shaders.ts:2240-2259), chosen by matmulTShader for f16
// weights (kernels.ts:410-426; K % 4 == 0). Two kernels:
//   * brik_gemv_f16w (one activation row per blockIdx.y): x staged in LDS as f32, each wave streams
//     two weight rows with 16-byte (8-half) loads (8-byte when K % 8 != 0), converts to f32 and
//     accumulates in f32, then reduces across the wave. For decode (M == 1) this is HBM-bound on the
//     2 bytes per weight.
//   * brik_gemm_f16w (M > 1, K % 8 == 0): x staged by brik_xprep_f16 (row-scaled f16, the k order
//     [0 4 1 5 2 6 3 7] within each 8), a 64 x 128 block tile per 4 waves, K steps of 32 through LDS,
//     v_mfma_f32_32x32x16_f16 with f32 accumulation; W is permuted into the same k order when it is
//     staged, so A and B contract over matching k.
#include "common.h"

namespace {

__device__ __forceinline__ float dot8_f16(u32x4_t w, const float* __restrict__ x)
{
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(x), b = *reinterpret_cast<const f32x4_t*>(x + 4);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float acc = 0.f;
    const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        acc = fmaf(f16_bits_to_f32(ws[j] & 0xffffu), xs[2 * j], acc);
        acc = fmaf(f16_bits_to_f32(ws[j] >> 16), xs[2 * j + 1], acc);
    }
    return acc;
}

__device__ __forceinline__ float wave_sum(float v)
{
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

}  // namespace

// Block: 4 waves x 2 rows = 8 weight rows; blockIdx.y = activation row. VEC8: K % 8 == 0 (16-byte
// weight loads), else 8-byte loads of 4 halves. Dynamic LDS: K floats.
template <bool VEC8>
__device__ __forceinline__ void gemv_f16w(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                          float* __restrict__ y, int K, int N)
{
    extern __shared__ __attribute__((aligned(16))) float xs[];
    const int m = blockIdx.y;
    const float* xr = x + (size_t)m * K;
    for (int i = threadIdx.x * 4; i < K; i += 256 * 4) *reinterpret_cast<f32x4_t*>(xs + i) = *reinterpret_cast<const f32x4_t*>(xr + i);
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (long n0 = ((long)blockIdx.x * 4 + wave) * 2; n0 < N; n0 += (long)gridDim.x * 8) {
        const bool two = n0 + 1 < N;
        const uint16_t* w0 = w + (size_t)n0 * K;
        const uint16_t* w1 = two ? w0 + K : w0;
        float a0 = 0.f, a1 = 0.f;
        if (VEC8) {
#pragma unroll 2
            for (int k = lane * 8; k < K; k += 64 * 8) {
                const u32x4_t v0 = ld_stream(reinterpret_cast<const u32x4_t*>(w0 + k));
                const u32x4_t v1 = ld_stream(reinterpret_cast<const u32x4_t*>(w1 + k));
                a0 += dot8_f16(v0, xs + k);
                a1 += dot8_f16(v1, xs + k);
            }
        } else {
#pragma unroll 2
            for (int k = lane * 4; k < K; k += 64 * 4) {
                const u32x2_t v0 = ld_stream(reinterpret_cast<const u32x2_t*>(w0 + k));
                const u32x2_t v1 = ld_stream(reinterpret_cast<const u32x2_t*>(w1 + k));
                const f32x4_t xv = *reinterpret_cast<const f32x4_t*>(xs + k);
                a0 = fmaf(f16_bits_to_f32(v0.x & 0xffffu), xv.x, a0);
                a0 = fmaf(f16_bits_to_f32(v0.x >> 16), xv.y, a0);
                a0 = fmaf(f16_bits_to_f32(v0.y & 0xffffu), xv.z, a0);
                a0 = fmaf(f16_bits_to_f32(v0.y >> 16), xv.w, a0);
                a1 = fmaf(f16_bits_to_f32(v1.x & 0xffffu), xv.x, a1);
                a1 = fmaf(f16_bits_to_f32(v1.x >> 16), xv.y, a1);
                a1 = fmaf(f16_bits_to_f32(v1.y & 0xffffu), xv.z, a1);
                a1 = fmaf(f16_bits_to_f32(v1.y >> 16), xv.w, a1);
            }
        }
        a0 = wave_sum(a0);
        a1 = wave_sum(a1);
        if (lane == 0) {
            y[(size_t)m * N + n0] = a0;
            if (two) y[(size_t)m * N + n0 + 1] = a1;
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void brik_gemv_f16w_v8(const float* __restrict__ x,
                                                                    const uint16_t* __restrict__ w,
                                                                    float* __restrict__ y, int K, int N)
{
    gemv_f16w<true>(x, w, y, K, N);
}

extern "C" __global__ __launch_bounds__(256) void brik_gemv_f16w_v4(const float* __restrict__ x,
                                                                    const uint16_t* __restrict__ w,
                                                                    float* __restrict__ y, int K, int N)
{
    gemv_f16w<false>(x, w, y, K, N);
}

namespace {

constexpr int FW_BM = 64, FW_BN = 128, FW_BK = 32;
constexpr int FW_ROW = FW_BK + 8;          // halves per staged row: 32 + a 16-byte pad

// W (natural k order) -> the staged x order [0 4 1 5 2 6 3 7] within each 8: halves (w0 .. w7) in
// dwords (w0 w1) (w2 w3) (w4 w5) (w6 w7) become (w0 w4) (w1 w5) (w2 w6) (w3 w7).
__device__ __forceinline__ u32x4_t interleave8(u32x4_t v)
{
    u32x4_t r;
    r.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
    r.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
    r.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
    r.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
    return r;
}

}  // namespace

// Block (bx, by): rows [64 by, 64 by + 64) of x, columns [128 bx, 128 bx + 128) of W. Wave w owns
// columns 32 w .. 32 w + 31 for all 64 rows (two 32 x 32 MFMA tiles). Per K step of 32: thread t stages
// x rows t / 4 (chunk t % 4) and W rows t / 4, t / 4 + 64 (chunk t % 4) into LDS; rows past M or N and
// chunks past K are zeros. D layout of the 32x32x16 MFMA: lane l, register e -> column l & 31, row
// 8 (e >> 2) + 4 (l >> 5) + (e & 3).
extern "C" __global__ __launch_bounds__(256) void brik_gemm_f16w(const uint16_t* __restrict__ xh,
                                                                 const float* __restrict__ rscale,
                                                                 const uint16_t* __restrict__ w,
                                                                 float* __restrict__ y, int M, int K, int N, int Kp)
{
    __shared__ __attribute__((aligned(16))) uint16_t As[FW_BM * FW_ROW];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[FW_BN * FW_ROW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bm0 = blockIdx.y * FW_BM, bn0 = blockIdx.x * FW_BN;
    const int sr = tid >> 2, sc = (tid & 3) * 8;               // staging row / half offset
    floatx16_t acc[2] = {};
    const u32x4_t zero = {0u, 0u, 0u, 0u};
    for (int k0 = 0; k0 < K; k0 += FW_BK) {
        const int kc = k0 + sc;
        const u32x4_t a = bm0 + sr < M ? *reinterpret_cast<const u32x4_t*>(xh + (size_t)(bm0 + sr) * Kp + kc) : zero;
        u32x4_t b[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int n = bn0 + sr + 64 * h;
            b[h] = (n < N && kc < K) ? interleave8(ld_stream(reinterpret_cast<const u32x4_t*>(w + (size_t)n * K + kc)))
                                     : zero;
        }
        __syncthreads();                                        // the previous step's reads are done
        *reinterpret_cast<u32x4_t*>(As + sr * FW_ROW + sc) = a;
        *reinterpret_cast<u32x4_t*>(Bs + sr * FW_ROW + sc) = b[0];
        *reinterpret_cast<u32x4_t*>(Bs + (sr + 64) * FW_ROW + sc) = b[1];
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int kk = 16 * s + 8 * (lane >> 5);
            const half8_t bf = *reinterpret_cast<const half8_t*>(Bs + (32 * wave + (lane & 31)) * FW_ROW + kk);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const half8_t af = *reinterpret_cast<const half8_t*>(As + (32 * i + (lane & 31)) * FW_ROW + kk);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[i], 0, 0, 0);
            }
        }
    }
    const int col = bn0 + 32 * wave + (lane & 31);
    if (col >= N) return;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = bm0 + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            if (row < M) y[(size_t)row * N + col] = acc[i][e] * rscale[row];
        }
}
