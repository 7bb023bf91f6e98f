"""Pins the oracle's reference matmul (kernels.ts:2335-2337: f64-accumulated sum of x*deq(W), one
f32 rounding) with checks that do not retype it:

* numpy float64 GEMM (BLAS order) on the oracle's own dequantized W: catches transposition, row/
  column index and accumulation mistakes (agreement to ~1e-12 relative, the f64 summation-order gap);
* closed forms: x = 1 gives sum_g (s_g * sum q + 32 m_g); zero codes give sum_g m_g * sum_{k in g} x_k;
  a one-hot x = e_k returns column k of deq(W) exactly;
* exact-sum property: with dyadic inputs every partial sum is exact in f64, so the result equals
  the exact rational sum (fractions) rounded once to f32.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth


def _planes(fmt, seed, N, K):
    t = synth.tensor(fmt, seed, N, K)
    if fmt == "q8":
        return (t["codes"], t["sc"]), O.dequant_q8(t["codes"], t["sc"])
    if fmt == "q4":
        return (t["nib"], t["sc"], t["mn"]), O.dequant_q4(t["nib"], t["sc"], t["mn"])
    return (t["lo"], t["hi"], t["sc"], t["mn"]), O.dequant_q3(t["lo"], t["hi"], t["sc"], t["mn"])


def _mm(fmt, x, planes, M, K, N, **kw):
    return {"q8": O.matmul_t_q8, "q4": O.matmul_t_q4, "q3": O.matmul_t_q3}[fmt](x, *planes, M, K, N, **kw)


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
@pytest.mark.parametrize("M,K,N", [(1, 128, 6), (5, 128, 6), (20, 128, 18), (3, 896, 37)])
def test_matches_float64_blas(fmt, M, K, N):
    planes, wd = _planes(fmt, 100 + M + N, N, K)
    x = synth.normal(7 + M, M * K)
    y, den = _mm(fmt, x, planes, M, K, N, absden=True)
    ref = x.reshape(M, K).astype(np.float64) @ wd.reshape(N, K).astype(np.float64).T
    assert np.allclose(y, ref.astype(np.float32), rtol=0, atol=1e-6 * np.abs(ref).max())
    assert np.allclose(den, np.abs(x.reshape(M, K).astype(np.float64))
                       @ np.abs(wd.reshape(N, K).astype(np.float64)).T, rtol=1e-12)


@pytest.mark.parametrize("fmt", ["q4", "q3"])
def test_closed_form_ones(fmt):
    M, K, N = 1, 256, 9
    planes, _ = _planes(fmt, 31, N, K)
    y = _mm(fmt, np.ones(K, np.float32), planes, M, K, N)
    sc = planes[-2].view(np.float16).astype(np.float64).reshape(N, K // 32)
    mn = planes[-1].view(np.float16).astype(np.float64).reshape(N, K // 32)
    if fmt == "q4":
        nib = planes[0]
        q = np.stack([nib & 15, nib >> 4], axis=1).ravel().astype(np.float64)
    else:
        lo, hi = planes[0], planes[1]
        i = np.arange(N * K)
        q = ((lo[i >> 4] >> ((i & 15) * 2)) & 3) | (((hi[i >> 5] >> (i & 31)) & 1) << 2)
    qsum = q.reshape(N, K // 32, 32).sum(axis=2)
    want = (sc * qsum + 32 * mn).sum(axis=1)
    assert np.allclose(y.ravel(), want, rtol=2e-6, atol=1e-6)


def test_closed_form_zero_codes():
    M, K, N = 2, 128, 5
    t = synth.q4_tensor(41, N, K)
    nib = np.zeros_like(t["nib"])
    x = synth.normal(42, M * K)
    y = O.matmul_t_q4(x, nib, t["sc"], t["mn"], M, K, N)
    mn = t["mn"].view(np.float16).astype(np.float64).reshape(N, K // 32)
    xs = x.astype(np.float64).reshape(M, K // 32, 32).sum(axis=2)
    assert np.allclose(y, xs @ mn.T, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_one_hot_returns_dequant_column(fmt):
    K, N = 96, 7
    planes, wd = _planes(fmt, 51, N, K)
    for k in (0, 1, 31, 32, 63, 95):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        y = _mm(fmt, x, planes, 1, K, N)
        assert np.array_equal(y.ravel(), wd.reshape(N, K)[:, k])


def test_exact_dyadic_sum():
    # x in multiples of 2^-4 with |x| <= 4, W in q4 with power-of-two scale/min: every product and
    # partial sum is a short dyadic rational, exact in f64; the result is the exact sum rounded once.
    M, K, N = 2, 64, 3
    rng = np.random.default_rng(61)
    x = (rng.integers(-64, 65, M * K) / 16).astype(np.float32)
    nib = rng.integers(0, 256, N * K // 2).astype(np.uint8)
    sc = synth.f16_bits(np.full(N * K // 32, 2.0 ** -5, np.float32))
    mn = synth.f16_bits(np.full(N * K // 32, -0.25, np.float32))
    y = O.matmul_t_q4(x, nib, sc, mn, M, K, N)
    q = np.stack([nib & 15, nib >> 4], axis=1).ravel().reshape(N, K)
    for r in range(M):
        for n in range(N):
            exact = sum(Fraction(float(x[r * K + k])) * (Fraction(int(q[n, k]), 32) - Fraction(1, 4))
                        for k in range(K))
            assert y[r, n] == np.float32(float(exact))


def test_moe_oracle_is_per_expert_matmul():
    E, K, N = 4, 64, 9
    row_off = np.array([0, 3, 3, 8, 10], np.int32)
    t = synth.q4_tensor(71, E * N, K)
    x = synth.normal(72, 10 * K)
    y = O.moe_matmul_t_q4(x, row_off, t["nib"], t["sc"], t["mn"], E, K, N)
    for e in range(E):
        r0, r1 = row_off[e], row_off[e + 1]
        if r1 == r0:
            continue
        g0, g1 = e * N * K // 32, (e + 1) * N * K // 32
        ye = O.matmul_t_q4(x[r0 * K:r1 * K], t["nib"][e * N * K // 2:(e + 1) * N * K // 2],
                           t["sc"][g0:g1], t["mn"][g0:g1], r1 - r0, K, N)
        assert np.array_equal(y[r0:r1], ye)
