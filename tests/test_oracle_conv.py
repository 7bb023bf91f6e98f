"""Pins of the oracle convolution (oracle.conv2d, the reference's CPU conv of kernels.ts:3049-3061),
the checker of the fused-dequant conv kernels: an independent numpy formulation (sliding windows over
the zero-padded input, products summed with einsum), and closed forms (a 1x1 convolution is the
matrix product W . X; a centred delta kernel with pad 1 copies its input channel; all-ones weights
count the taps inside the image)."""
import numpy as np
import pytest

import oracle as O


def numpy_conv(x, w, b, Cin, H, W, Cout, kh, kw, stride, pad):
    xp = np.pad(x.reshape(Cin, H, W).astype(np.float64), ((0, 0), (pad, pad), (pad, pad)))
    win = np.lib.stride_tricks.sliding_window_view(xp, (kh, kw), axis=(1, 2))[:, ::stride, ::stride]
    y = np.einsum("chwij,ocij->ohw", win, w.reshape(Cout, Cin, kh, kw).astype(np.float64))
    if b is not None:
        y += b[:, None, None]
    return y


@pytest.mark.parametrize("Cin,H,W,Cout,kh,kw,stride,pad", [
    (2, 4, 4, 3, 3, 3, 1, 1), (8, 4, 4, 4, 3, 3, 1, 1), (3, 9, 7, 5, 3, 3, 2, 1), (4, 6, 8, 2, 1, 1, 1, 0),
    (2, 11, 10, 3, 5, 5, 2, 2), (1, 5, 5, 1, 5, 5, 1, 0), (3, 7, 9, 4, 2, 3, 3, 0)])
def test_matches_independent_numpy_conv(Cin, H, W, Cout, kh, kw, stride, pad):
    rng = np.random.default_rng(Cin * 100 + H)
    x = rng.standard_normal(Cin * H * W).astype(np.float32)
    w = rng.standard_normal(Cout * Cin * kh * kw).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    got = O.conv2d(x, w, b, Cin, H, W, Cout, kh, kw, stride, pad)
    ref = numpy_conv(x, w, b, Cin, H, W, Cout, kh, kw, stride, pad)
    assert got.shape == ref.shape
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)


def test_closed_forms():
    rng = np.random.default_rng(5)
    Cin, H, W, Cout = 6, 5, 7, 4
    x = rng.standard_normal(Cin * H * W).astype(np.float32)
    w1 = rng.standard_normal(Cout * Cin).astype(np.float32)
    y = O.conv2d(x, w1, None, Cin, H, W, Cout, 1, 1)
    np.testing.assert_allclose(y.reshape(Cout, -1), w1.reshape(Cout, Cin).astype(np.float64) @ x.reshape(Cin, -1),
                               rtol=1e-6, atol=1e-6)
    delta = np.zeros((Cout, Cin, 3, 3), np.float32)
    for co in range(Cout):
        delta[co, co % Cin, 1, 1] = 1.0
    y = O.conv2d(x, delta, None, Cin, H, W, Cout, 3, 3, 1, 1)
    for co in range(Cout):
        assert np.array_equal(y[co], x.reshape(Cin, H, W)[co % Cin])
    y = O.conv2d(np.ones(2 * 4 * 4, np.float32), np.ones(3 * 2 * 9, np.float32), np.full(3, 0.5, np.float32),
                 2, 4, 4, 3, 3, 3, 1, 1)
    taps = np.array([[4, 6, 6, 4], [6, 9, 9, 6], [6, 9, 9, 6], [4, 6, 6, 4]])
    assert np.array_equal(y, np.broadcast_to(2 * taps + 0.5, (3, 4, 4)))
