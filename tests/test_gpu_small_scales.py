"""GPU parity of the MFMA paths (prefill GEMM, expert-grouped MoE, implicit-GEMM convolution) on q4
planes whose scales are small: f16 scales in [2^-14, 2^-10) (any group whose value range is below
about 0.015 gets one from the encoder, q4web.ts:36-41), zero scales (a constant group), and planes the
GPU encoder makes from N(0, 3e-3) data. The dequantization rounds q s + m once to f16 with the
scale as stored, so these hold the same 1e-3 bar as every other scale (normwise and componentwise,
|y - r| <= 1e-3 sum|x w|).
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import layout, synth
from brimkern_amd.capi import BRIK_OPT_PATH, BRIK_OPT_GEMM_TILE, BRIK_GEMM_TILES
from helpers import Gpu, PLANES, normwise_rel, componentwise_ok, REL_TOL

pytestmark = pytest.mark.gpu
TINY = (2.0 ** -14, 2.0 ** -10)


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    ctx.set_option(BRIK_OPT_PATH, 0)
    ctx.set_option(BRIK_OPT_GEMM_TILE, 0)
    g.free()


def check(y, r, den):
    rel = normwise_rel(y, r)
    assert rel <= REL_TOL, f"normwise rel {rel:.3e}"
    assert componentwise_ok(y, r, den, REL_TOL), "componentwise bound violated"


def tiny_tensor(fmt, seed, N, K):
    t = synth.tensor(fmt, seed, N, K, s_lo=TINY[0], s_hi=TINY[1])
    s = t["sc"].view(np.float16).astype(np.float32)
    assert s.min() >= 2.0 ** -14 and s.max() < 2.0 ** -10 + 2.0 ** -20
    return t


def oracle_mm(fmt, x, t, M):
    fn = getattr(O, f"matmul_t_{fmt}")
    return fn(x, *[t[k] for k in PLANES[fmt]], M, t["K"], t["N"], absden=True)


@pytest.mark.parametrize("fmt", ["q4", "q3", "q8"])
@pytest.mark.parametrize("M,K,N", [(512, 2560, 1024), (37, 640, 300)])
def test_gemm_tiny_scales(gpu, fmt, M, K, N):
    t = tiny_tensor(fmt, 810 + M, N, K)
    x = synth.normal(811 + M, M * K)
    gpu.ctx.set_option(BRIK_OPT_PATH, 2)          # the MFMA GEMM
    y = gpu.matmul(fmt, x, gpu.planes(fmt, t), M, K, N)
    r, den = oracle_mm(fmt, x, t, M)
    check(y, r, den)


@pytest.mark.parametrize("tile", [0] + list(range(1, BRIK_GEMM_TILES + 1)))
def test_gemm_tiny_scales_every_tile(gpu, tile):
    M, K, N = 130, 96, 1100
    t = tiny_tensor("q4", 820, N, K)
    x = synth.normal(821, M * K)
    gpu.ctx.set_option(BRIK_OPT_GEMM_TILE, tile)
    y = gpu.matmul("q4", x, gpu.planes("q4", t), M, K, N)
    r, den = oracle_mm("q4", x, t, M)
    check(y, r, den)


def test_gemm_zero_scales(gpu):
    """A zero scale (a constant group, q4web.ts:40's `|| 1e-8` aside, or a hand-made plane): every
    weight of the group is its min."""
    M, K, N = 64, 512, 256
    t = synth.q4_tensor(830, N, K)
    sc = t["sc"].copy()
    sc[::3] = 0
    t = dict(t, sc=sc)
    x = synth.normal(831, M * K)
    gpu.ctx.set_option(BRIK_OPT_PATH, 2)
    y = gpu.matmul("q4", x, gpu.planes("q4", t), M, K, N)
    r, den = oracle_mm("q4", x, t, M)
    check(y, r, den)


def test_gemm_on_gpu_encoded_small_weights(gpu):
    """Weights ~ N(0, 3e-3) encoded by brik_quantize_q4 on the device (scales near 1.5e-3, below 2^-10
    in many groups), then the prefill GEMM on those device planes."""
    M, K, N = 256, 2560, 768
    n = N * K
    w = synth.normal(840, n) * np.float32(3e-3)
    src = gpu.up(w)
    blob = gpu.ctx.alloc(layout.byte_length("q4", n))
    gpu.bufs.append(blob)
    offs = layout.plane_offsets("q4", n)
    planes = [blob.offset(offs[p][0]) for p in PLANES["q4"]]
    gpu.ctx.quantize("q4", src, planes, n)
    raw = gpu.ctx.download(blob, np.uint8, layout.byte_length("q4", n))
    t = {"N": N, "K": K, "nib": raw[:n // 2], "sc": raw[offs["sc"][0]:offs["mn"][0]].view("<u2"),
         "mn": raw[offs["mn"][0]:].view("<u2")}
    s = t["sc"].view(np.float16).astype(np.float32)
    assert (s < 2.0 ** -10).mean() > 0.1
    x = synth.normal(841, M * K)
    gpu.ctx.set_option(BRIK_OPT_PATH, 2)
    y = gpu.matmul("q4", x, planes, M, K, N)
    r, den = oracle_mm("q4", x, t, M)
    check(y, r, den)


@pytest.mark.parametrize("K,N", [(2048, 768), (768, 2048)])
def test_moe_tiny_scales(gpu, K, N):
    T, E, TOPK = 64, 16, 4
    rows, row_off = synth.moe_routing(850, T, E, TOPK)
    R = rows.size
    t = tiny_tensor("q4", 851, E * N, K)
    x = synth.normal(852, R * K)
    planes = gpu.planes("q4", t)
    xb, rb = gpu.up(x), gpu.up(row_off)
    yb = gpu.up(np.full(R * N, np.nan, np.float32))
    gpu.ctx.moe_matmul_t_q4(xb, rb, *planes, yb, E, R, K, N)
    y = gpu.ctx.download(yb, np.float32, R * N).reshape(R, N)
    r = O.moe_matmul_t_q4(x, row_off, t["nib"], t["sc"], t["mn"], E, K, N)
    # componentwise denominators: sum |x w| per routed row against its expert's dequantized rows
    deq = O.dequant_q4(t["nib"], t["sc"], t["mn"]).reshape(E, N, K).astype(np.float64)
    xr = np.abs(x.reshape(R, K).astype(np.float64))
    den = np.zeros((R, N))
    for e in range(E):
        a, b = row_off[e], row_off[e + 1]
        den[a:b] = xr[a:b] @ np.abs(deq[e]).T
    check(y, r.reshape(R, N), den)


def test_conv_implicit_gemm_tiny_scales(gpu):
    Cin, H, W, Cout, kh, kw, st, pd = 32, 12, 12, 48, 3, 3, 1, 1
    K = Cin * kh * kw
    t = tiny_tensor("q4", 860, Cout, K)
    deq = O.dequant_q4(t["nib"], t["sc"], t["mn"])
    x = synth.normal(861, Cin * H * W)
    b = synth.normal(862, Cout) * np.float32(1e-3)
    buf = gpu.up(layout.pack("q4", t))
    offs = layout.plane_offsets("q4", Cout * K)
    planes = [buf.offset(offs[p][0]) for p in PLANES["q4"]]
    xb, bb = gpu.up(x), gpu.up(b)
    ob = gpu.up(np.full(Cout * H * W, np.nan, np.float32))
    gpu.ctx.set_option(BRIK_OPT_PATH, 2)        # the implicit MFMA GEMM
    gpu.ctx.conv2d("q4", xb, planes, bb, ob, Cin, H, W, Cout, kh, kw, st, pd)
    y = gpu.ctx.download(ob, np.float32, Cout * H * W)
    ref, den = O.conv2d(x, deq, b, Cin, H, W, Cout, kh, kw, st, pd, return_absden=True)
    check(y, ref.ravel(), den.ravel())
