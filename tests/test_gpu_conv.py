"""GPU parity of the fused-dequant convolutions (brik_conv2d_q8 / q4, the reference's conv2d_direct_q8 /
conv2d_direct_q4) through the C ABI, against the oracle conv on the dequantized weights.

The first case is the reference's own check (kernels.ts:3085-3120: Cin 8, 4x4 input, Cout 4, 3x3,
stride 1, pad 1, weights quantized by quantizeQ8 / quantizeQ4, compared with the f32 conv of the
dequantized weights). Both paths run on every shape that allows them: the direct kernel (f32
accumulation in the reference's order; bar: the f32 summation bound (K + 2) 2^-24 sum |x w|) and the
implicit MFMA GEMM (f16 staging; the matmul bar 1e-3 sum |x w|).
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import layout
from brimkern_amd.capi import BrikError, BRIK_EINVAL, BRIK_OPT_PATH
from brimkern_amd.engine import Engine, QWeight
from helpers import Gpu, PLANES

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()
    ctx.set_option(BRIK_OPT_PATH, 0)


def quantized(fmt, w):
    parts = getattr(O, f"quantize_{fmt}")(w)
    blob = getattr(O, f"pack_{fmt}")(*parts)
    deq = getattr(O, f"dequant_{fmt}")(*parts)
    return blob, deq


def run(gpu, fmt, x, blob, n_w, b, shape, path):
    Cin, H, W, Cout, kh, kw, st, pd = shape
    OH, OW = (H + 2 * pd - kh) // st + 1, (W + 2 * pd - kw) // st + 1
    buf = gpu.up(blob)
    offs = layout.plane_offsets(fmt, n_w)
    planes = [buf.offset(offs[p][0]) for p in PLANES[fmt]]
    xb = gpu.up(x)
    bb = gpu.up(b) if b is not None else None
    ob = gpu.ctx.alloc(4 * Cout * OH * OW)
    gpu.bufs.append(ob)
    gpu.ctx.set_option(BRIK_OPT_PATH, path)
    gpu.ctx.conv2d(fmt, xb, planes, bb, ob, Cin, H, W, Cout, kh, kw, st, pd)
    return gpu.ctx.download(ob, np.float32, Cout * OH * OW).reshape(Cout, OH, OW)


def check(y, ref, den, K, path):
    tol = (K + 2) * 2.0 ** -24 if path == 1 else 1e-3
    err = np.abs(y.astype(np.float64) - ref)
    assert np.all(err <= tol * den + 1e-30), float((err / np.maximum(den, 1e-30)).max())


SHAPES = [
    (8, 4, 4, 4, 3, 3, 1, 1),          # the reference's validation case
    (32, 16, 16, 16, 3, 3, 1, 1),      # K = 288: both paths
    (64, 20, 13, 40, 3, 3, 2, 1),      # stride 2, ragged
    (96, 9, 9, 33, 1, 1, 1, 0),        # 1x1
    (32, 12, 12, 8, 5, 5, 1, 2),       # 5x5
    (3, 17, 15, 32, 3, 3, 1, 1),       # K = 27: direct only (groups straddle rows)
    (64, 8, 8, 16, 4, 4, 4, 0),        # patchify
]


@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[0]}x{s[1]}x{s[2]}-{s[3]}-k{s[4]}x{s[5]}s{s[6]}p{s[7]}" for s in SHAPES])
def test_conv_paths(gpu, fmt, shape):
    Cin, H, W, Cout, kh, kw, st, pd = shape
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(Cin * H * W).astype(np.float32)
    w = (rng.standard_normal(Cout * Cin * kh * kw) * 0.2).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    blob, deq = quantized(fmt, w)
    ref, den = O.conv2d(x, deq, b, Cin, H, W, Cout, kh, kw, st, pd, return_absden=True)
    K = Cin * kh * kw
    for path in (1, 2) if K % 32 == 0 else (1,):
        y = run(gpu, fmt, x, blob, w.size, b, shape, path)
        check(y, ref, den, K, path)


@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_conv_unet_shape_gemm(gpu, fmt):
    # a UNet-sized 3x3 conv (K = 2880) on the MFMA path, no bias
    shape = (320, 24, 24, 320, 3, 3, 1, 1)
    Cin, H, W, Cout, kh, kw, st, pd = shape
    rng = np.random.default_rng(77)
    x = rng.standard_normal(Cin * H * W).astype(np.float32)
    w = (rng.standard_normal(Cout * Cin * 9) * 0.05).astype(np.float32)
    blob, deq = quantized(fmt, w)
    ref, den = O.conv2d(x, deq, None, Cin, H, W, Cout, kh, kw, st, pd, return_absden=True)
    y = run(gpu, fmt, x, blob, w.size, None, shape, 0)
    check(y, ref, den, Cin * 9, 2)


def test_conv_rejects_bad_shapes(gpu):
    w = np.zeros(4 * 3 * 9, np.float32)
    blob, _ = quantized("q8", np.zeros(4 * 8 * 9, np.float32))
    buf = gpu.up(blob)
    x = gpu.up(np.zeros(3 * 4 * 4, np.float32))
    o = gpu.up(np.zeros(64, np.float32))
    offs = layout.plane_offsets("q8", 4 * 8 * 9)
    planes = [buf.offset(offs["codes"][0]), buf.offset(offs["sc"][0])]
    for args in [(3, 4, 4, 4, 3, 3, 1, 1),     # 4*3*9 = 108 weights: not a multiple of 32
                 (8, 2, 2, 4, 5, 5, 1, 0),     # kernel larger than the input
                 (8, 4, 4, 4, 3, 3, 0, 1)]:    # stride 0
        with pytest.raises(BrikError) as e:
            gpu.ctx.conv2d("q8", x, planes, None, o, *args)
        assert e.value.code == BRIK_EINVAL, args
    assert w.size == 108


def test_engine_conv2d_session_form(ctx):
    # the reference's session call shape: conv2d(inp, w, bias, ...) with a quantized handle
    eng = Engine(ctx=ctx)
    rng = np.random.default_rng(3)
    Cin, H, W, Cout = 8, 4, 4, 4
    x = rng.standard_normal(Cin * H * W).astype(np.float32)
    w = rng.standard_normal(Cout * Cin * 9).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    for fmt in ("q8", "q4"):
        blob, deq = quantized(fmt, w)
        h = eng.weight(fmt, blob, w.size)
        try:
            yb = eng.conv2d(x, h, b, Cin, H, W, Cout, 3, 3, 1, 1)
            y = ctx.download(yb, np.float32, Cout * H * W).reshape(Cout, H, W)
            ctx.free(yb)
        finally:
            ctx.free(h["_buf"])
        ref, den = O.conv2d(x, deq, b, Cin, H, W, Cout, 3, 3, 1, 1, return_absden=True)
        check(y, ref, den, Cin * 9, 1)
    with pytest.raises(BrikError):
        eng.conv2d(x, QWeight({"q3": True, "lo": 0, "hi": 0, "sc": 0, "mn": 0}), b, Cin, H, W, Cout, 3, 3, 1, 1)


@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_direct_skips_outside_taps_with_infinite_weights(gpu, fmt):
    """A weight group with an infinite scale (channel 1 of a 1x1 conv padded by 1): the reference skips
    the taps outside the image, so the outputs on the padding ring are exactly the bias while the
    interior ones are not finite. The direct kernel's branch-free walk (x = 0 at outside taps) would make
    the ring NaN (0 * inf), so a chunk holding a non-finite weight must take the skipping walk."""
    shape = (32, 5, 5, 4, 1, 1, 1, 1)
    Cin, H, W, Cout, kh, kw, st, pd = shape
    rng = np.random.default_rng(41)
    x = rng.standard_normal(Cin * H * W).astype(np.float32)
    w = (rng.standard_normal(Cout * Cin) * 0.2).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    parts = list(getattr(O, f"quantize_{fmt}")(w))
    sc = np.array(parts[1], np.uint16).copy()
    sc[1] = 0x7C00                                   # channel 1's group (K = 32): scale +inf
    parts[1] = sc
    blob = getattr(O, f"pack_{fmt}")(*parts)
    deq = getattr(O, f"dequant_{fmt}")(*parts)
    ref, den = O.conv2d(x, deq, b, Cin, H, W, Cout, kh, kw, st, pd, return_absden=True)
    y = run(gpu, fmt, x, blob, w.size, b, shape, 1)
    ring = np.ones((H + 2, W + 2), bool)
    ring[1:-1, 1:-1] = False
    assert np.array_equal(y[1][ring], np.full(ring.sum(), b[1], np.float32))
    assert not np.isfinite(y[1][~ring]).any()
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(y), fin)
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    check(np.where(fin, y, 0), np.where(fin, ref, 0), np.where(fin, den, 0), Cin, 1)
