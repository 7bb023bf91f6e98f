/*
 * CPU oracle for Brimkern's fused quantized matmul family (matmul_t_q8 / _q4 / _q3).
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker, never the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The shipped path
 * (brimkern_amd/) never links or calls it and fails loudly when its HIP library is missing.
 *
 * It restates, in plain C, the reference's own CPU-side arithmetic for this path:
 *   - f16 decode / encode ........ src/lib/brik/f16.ts:8-22, 25-34
 *   - q8 dequant ................. src/lib/brik/q8web.ts:74-83   (w = code * s)
 *   - q4 dequant ................. src/lib/brik/q4web.ts:82-96   (w = q * s + m, low nibble = even index)
 *   - q3 dequant ................. src/lib/brik/q3web.ts:97-110   (q = lo2 | hi1 << 2, w = q * s + m)
 *   - reference matmul ........... src/lib/webgpu/kernels.ts:2335-2337 (and its q3/q8/tiled/shared
 *                                  siblings at 2364-2365, 2381-2382, 2397-2398, 2412-2414,
 *                                  2438-2439, 2455-2456): Wd = dequantize(q) as Float32Array,
 *                                  ref[r,c] = Math.fround(sum_i a[r,i] * Wd[c,i]) with the sum
 *                                  taken left to right in a JS double.
 *
 * JS semantics that matter and are reproduced exactly:
 *   - f16BitsToF32 returns a double; subnormals use the literal 5.9604645e-8 (not exactly 2^-24),
 *     e == 31 gives +-Infinity / NaN (f16.ts:30-31).
 *   - dequant arithmetic (q * s + m) runs in double and is rounded to f32 once on the store
 *     into the Float32Array.
 *   - the matmul products a*w are f32*f32, exact in double; the running sum is double,
 *     sequential in i; the result is rounded to f32 once.
 * The file is compiled with -ffp-contract=off and without -ffast-math so that no fused or
 * reassociated arithmetic changes these roundings.
 *
 * Layouts (all little-endian, planes exactly as packQ8/packQ4/packQ3 write them):
 *   q8: codes int8[n]            | scales f16[n/32]
 *   q4: nibbles u8[n/2]          | scales f16[n/32] | mins f16[n/32]
 *   q3: lo u32[n/16] (2 bits/code, code i at bits (i&15)*2) | hi u32[n/32] (bit i&31)
 *       | scales f16[n/32] | mins f16[n/32]
 * W is [N, K] row-major (the transposed weight of y = x . W^T), so group g of row n is
 * flat group n*(K/32) + g.
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <math.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define GROUP 32

/* src/lib/brik/f16.ts:25-34 — IEEE binary16 bits -> number (a JS double). */
double oracle_f16_to_f64(uint16_t h)
{
    int s = (h >> 15) & 1;
    int e = (h >> 10) & 0x1f;
    int m = h & 0x3ff;
    double val;
    if (e == 0)
        val = (double)m * 5.9604645e-8;
    else if (e == 31)
        val = m ? NAN : INFINITY;
    else
        val = (1.0 + (double)m / 1024.0) * ldexp(1.0, e - 15);
    return s ? -val : val;
}

/* src/lib/brik/f16.ts:8-22 — f32 -> binary16 bits: RNE on the mantissa, |x| < 2^-14 flushes
 * to +-0, overflow clamps to +-max-normal (0x7bff). Integer shifts follow the JS code
 * (>> on a u32 read through Uint32Array, so logical). */
uint16_t oracle_f32_to_f16(float val)
{
    uint32_t x;
    memcpy(&x, &val, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t exp = (int32_t)((x >> 23) & 0xffu) - 127 + 15;
    uint32_t mant = x & 0x7fffffu;
    if (exp <= 0) return (uint16_t)sign;
    if (exp >= 31) return (uint16_t)(sign | 0x7bffu);
    uint32_t round = (mant >> 13) + ((mant >> 12) & 1u);
    mant = round;
    if (mant == 0x400u) { mant = 0; exp += 1; }
    return (uint16_t)(sign | ((uint32_t)exp << 10) | (mant & 0x3ffu));
}

void oracle_f16_to_f64_n(const uint16_t *h, size_t n, double *out)
{
    for (size_t i = 0; i < n; i++) out[i] = oracle_f16_to_f64(h[i]);
}

void oracle_f32_to_f16_n(const float *v, size_t n, uint16_t *out)
{
    for (size_t i = 0; i < n; i++) out[i] = oracle_f32_to_f16(v[i]);
}

/* ---- dequantization of a contiguous range of elements [e0, e0 + cnt) ---------------------- */

/* q8web.ts:74-83: out[i] = codes[i] * s (double), stored to f32. */
static void deq_q8_range(const int8_t *codes, const uint16_t *sc, size_t e0, size_t cnt, float *out)
{
    for (size_t j = 0; j < cnt; j++) {
        size_t i = e0 + j;
        double s = oracle_f16_to_f64(sc[i / GROUP]);
        out[j] = (float)((double)codes[i] * s);
    }
}

/* q4web.ts:82-96: byte = nibbles[i >> 1]; q = even i ? low nibble : high nibble; q*s + m. */
static void deq_q4_range(const uint8_t *nib, const uint16_t *sc, const uint16_t *mn,
                         size_t e0, size_t cnt, float *out)
{
    for (size_t j = 0; j < cnt; j++) {
        size_t i = e0 + j;
        double s = oracle_f16_to_f64(sc[i / GROUP]);
        double m = oracle_f16_to_f64(mn[i / GROUP]);
        uint8_t byte = nib[i >> 1];
        int q = ((i % GROUP) & 1) == 0 ? (byte & 0xf) : (byte >> 4);
        out[j] = (float)((double)q * s + m);
    }
}

/* q3web.ts:97-110: q = ((lo[i>>4] >> ((i&15)*2)) & 3) | (((hi[i>>5] >> (i&31)) & 1) << 2). */
static void deq_q3_range(const uint32_t *lo, const uint32_t *hi, const uint16_t *sc,
                         const uint16_t *mn, size_t e0, size_t cnt, float *out)
{
    for (size_t j = 0; j < cnt; j++) {
        size_t i = e0 + j;
        double s = oracle_f16_to_f64(sc[i / GROUP]);
        double m = oracle_f16_to_f64(mn[i / GROUP]);
        uint32_t q = ((lo[i >> 4] >> ((i & 15) * 2)) & 3u) | (((hi[i >> 5] >> (i & 31)) & 1u) << 2);
        out[j] = (float)((double)q * s + m);
    }
}

void oracle_dequant_q8(const int8_t *codes, const uint16_t *sc, size_t n, float *out)
{
    deq_q8_range(codes, sc, 0, n, out);
}

void oracle_dequant_q4(const uint8_t *nib, const uint16_t *sc, const uint16_t *mn, size_t n, float *out)
{
    deq_q4_range(nib, sc, mn, 0, n, out);
}

void oracle_dequant_q3(const uint32_t *lo, const uint32_t *hi, const uint16_t *sc,
                       const uint16_t *mn, size_t n, float *out)
{
    deq_q3_range(lo, hi, sc, mn, 0, n, out);
}

/* ---- reference matmul: y[M,N] = x[M,K] . deq(W[N,K])^T ---------------------------------- */

/* One output row of W at a time: dequantize row n (K floats, exactly what the reference's
 * whole-tensor dequantize would hold for that row), then for each x row the sequential double
 * sum of kernels.ts:2337. absden (optional) receives sum_i |a[r,i] * w[n,i]| in double,
 * the denominator of the componentwise error bound. */
enum { FMT_Q8 = 8, FMT_Q4 = 4, FMT_Q3 = 3 };

static void matmul_rows(int fmt, const float *x, const void *p0, const void *p1, const void *p2,
                        const void *p3, int M, int K, int N, float *y, double *absden, int threads)
{
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#endif
    (void)threads;
    #pragma omp parallel
    {
        float *w = (float *)malloc((size_t)K * sizeof(float) + 16);
        #pragma omp for schedule(static)
        for (long n = 0; n < N; n++) {
            size_t e0 = (size_t)n * (size_t)K;
            if (fmt == FMT_Q8)
                deq_q8_range((const int8_t *)p0, (const uint16_t *)p1, e0, (size_t)K, w);
            else if (fmt == FMT_Q4)
                deq_q4_range((const uint8_t *)p0, (const uint16_t *)p1, (const uint16_t *)p2, e0, (size_t)K, w);
            else
                deq_q3_range((const uint32_t *)p0, (const uint32_t *)p1, (const uint16_t *)p2,
                             (const uint16_t *)p3, e0, (size_t)K, w);
            for (int r = 0; r < M; r++) {
                const float *a = x + (size_t)r * K;
                double s = 0.0, d = 0.0;
                for (int i = 0; i < K; i++) {
                    double prod = (double)a[i] * (double)w[i];
                    s += prod;
                    d += fabs(prod);
                }
                y[(size_t)r * N + n] = (float)s;
                if (absden) absden[(size_t)r * N + n] = d;
            }
        }
        free(w);
    }
}

void oracle_matmul_t_q8(const float *x, const int8_t *codes, const uint16_t *sc, int M, int K, int N,
                        float *y, double *absden, int threads)
{
    matmul_rows(FMT_Q8, x, codes, sc, NULL, NULL, M, K, N, y, absden, threads);
}

void oracle_matmul_t_q4(const float *x, const uint8_t *nib, const uint16_t *sc, const uint16_t *mn,
                        int M, int K, int N, float *y, double *absden, int threads)
{
    matmul_rows(FMT_Q4, x, nib, sc, mn, NULL, M, K, N, y, absden, threads);
}

void oracle_matmul_t_q3(const float *x, const uint32_t *lo, const uint32_t *hi, const uint16_t *sc,
                        const uint16_t *mn, int M, int K, int N, float *y, double *absden, int threads)
{
    matmul_rows(FMT_Q3, x, lo, hi, sc, mn, M, K, N, y, absden, threads);
}

/* ---- MoE expert-grouped matmul (no reference counterpart; the benchmarked 64-expert MoE layer) -------------
 * The reference has no MoE. The oracle applies the reference matmul above per expert:
 * rows [row_off[e], row_off[e+1]) of x_sorted times deq(W_e)^T, where W is a stacked q4 tensor
 * [E, N, K] in one .brik blob (expert e's nibbles start at e*N*K/2, its scales/mins at e*N*K/32). */
void oracle_moe_matmul_t_q4(const float *x_sorted, const int32_t *row_off, const uint8_t *nib,
                            const uint16_t *sc, const uint16_t *mn, int E, int K, int N,
                            float *y_sorted, int threads)
{
    size_t per_nib = (size_t)N * K / 2, per_g = (size_t)N * K / GROUP;
    for (int e = 0; e < E; e++) {
        int r0 = row_off[e], r1 = row_off[e + 1];
        if (r1 <= r0) continue;
        matmul_rows(FMT_Q4, x_sorted + (size_t)r0 * K, nib + e * per_nib, sc + e * per_g,
                    mn + e * per_g, NULL, r1 - r0, K, N, y_sorted + (size_t)r0 * N, NULL, threads);
    }
}

/* ---- 2-D convolution on dequantized weights (fused-dequant consumers conv2d_direct_q8 / q4) -----
 * src/lib/webgpu/kernels.ts:3049-3061 (the self-validation reference conv, used for the q8 / q4
 * conv checks at 3085-3120 on dequantizeQ8 / dequantizeQ4 weights): acc starts at bias[co] and adds
 * inp * w over ci, ky, kx (taps inside the image) in a JS double; the result is stored to f32.
 * absden (optional) receives sum |inp * w| + |bias| per output, the scale of its rounding error. */
void oracle_conv2d(const float *inp, const float *w, const float *bias, int Cin, int H, int W, int Cout,
                   int kh, int kw, int stride, int pad, float *out, double *absden)
{
    int OH = (H + 2 * pad - kh) / stride + 1, OW = (W + 2 * pad - kw) / stride + 1;
#pragma omp parallel for schedule(static)
    for (int co = 0; co < Cout; co++)
        for (int oy = 0; oy < OH; oy++)
            for (int ox = 0; ox < OW; ox++) {
                double acc = bias ? bias[co] : 0.0, den = bias ? fabs((double)bias[co]) : 0.0;
                for (int ci = 0; ci < Cin; ci++)
                    for (int ky = 0; ky < kh; ky++) {
                        int iy = oy * stride + ky - pad;
                        if (iy < 0 || iy >= H) continue;
                        for (int kx = 0; kx < kw; kx++) {
                            int ix = ox * stride + kx - pad;
                            if (ix < 0 || ix >= W) continue;
                            double p = (double)inp[((size_t)ci * H + iy) * W + ix] *
                                       (double)w[(((size_t)co * Cin + ci) * kh + ky) * kw + kx];
                            acc += p;
                            den += fabs(p);
                        }
                    }
                size_t o = ((size_t)co * OH + oy) * OW + ox;
                out[o] = (float)acc;
                if (absden) absden[o] = den;
            }
}
