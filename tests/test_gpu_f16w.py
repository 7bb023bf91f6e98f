"""GPU parity of the f16-weight matmul (brik_matmul_t_f16w, the reference's MATMUL_T_F16W) through the C
ABI, against y = x . W^T in f64 (W widened exactly from its f16 bits). The streaming kernel accumulates
in f32 (bar: the f32 summation bound (K + 2) 2^-24 sum |x w|); the MFMA kernel stages x as row-scaled
f16 (the matmuls' bar 1e-3 sum |x w|). Both run on every shape that allows them."""
import numpy as np
import pytest

import oracle as O
from brimkern_amd.capi import BrikError, BRIK_EINVAL, BRIK_EALIGN, BRIK_OPT_PATH, BRIK_OPT_GEMM_TILE
from brimkern_amd.engine import Engine
from helpers import Gpu

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()
    ctx.set_option(BRIK_OPT_PATH, 0)
    ctx.set_option(BRIK_OPT_GEMM_TILE, 0)


def run(gpu, x, wb, M, K, N, path):
    xb = gpu.up(x)
    yb = gpu.ctx.alloc(max(M * N, 1) * 4)
    gpu.bufs.append(yb)
    gpu.ctx.set_option(BRIK_OPT_PATH, path)
    gpu.ctx.matmul_t_f16w(xb, wb, yb, M, K, N)
    return gpu.ctx.download(yb, np.float32, M * N).reshape(M, N)


@pytest.mark.parametrize("M,K,N", [(1, 2560, 9728), (1, 100, 37), (1, 16384, 64), (2, 256, 130), (5, 260, 33),
                                   (64, 2560, 1000), (200, 512, 129), (3, 8, 1), (130, 1024, 256),
                                   # the tiled f16 kernels (K % 32 == 0): every row tile, K not a multiple of
                                   # the 128-k step (dead groups) and of 256 (odd step counts padded)
                                   (512, 2560, 1024), (300, 640, 520), (96, 320, 300), (40, 96, 77), (33, 32, 5)])
def test_f16w(gpu, M, K, N):
    rng = np.random.default_rng(M * 7 + K + N)
    x = (rng.standard_normal(M * K) * 2).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.05).astype(np.float16).view(np.uint16)
    ref, den = O.matmul_t_f16w(x, w, M, K, N)
    wb = gpu.up(w)
    paths = [p for p in (1, 2) if (p == 1 and K <= 16384) or (p == 2 and K % 8 == 0)]
    for path in paths:
        y = run(gpu, x, wb, M, K, N, path)
        tol = (K + 2) * 2.0 ** -24 if path == 1 else 1e-3
        err = np.abs(y - ref)
        assert np.all(err <= tol * den + 1e-30), (path, float((err / np.maximum(den, 1e-30)).max()))


def test_f16w_rejects(gpu):
    x = gpu.up(np.zeros(64, np.float32))
    w = gpu.up(np.zeros(64, np.uint16))
    y = gpu.up(np.zeros(64, np.float32))
    with pytest.raises(BrikError) as e:
        gpu.ctx.matmul_t_f16w(x, w, y, 1, 6, 2)          # K % 4 != 0
    assert e.value.code == BRIK_EINVAL
    with pytest.raises(BrikError) as e:
        gpu.ctx.matmul_t_f16w(x.offset(4), w, y, 1, 8, 2)
    assert e.value.code == BRIK_EALIGN


def test_engine_matmul_t_readback(ctx):
    eng = Engine(ctx=ctx)
    M, K, N = 3, 512, 70
    rng = np.random.default_rng(9)
    x = rng.standard_normal(M * K).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.1).astype(np.float16).view(np.uint16)
    wb = ctx.upload(w)
    try:
        y = eng.matmul_t_f16w(x, wb, M, K, N).reshape(M, N)
    finally:
        ctx.free(wb)
    ref, den = O.matmul_t_f16w(x, w, M, K, N)
    assert np.all(np.abs(y - ref) <= 1e-3 * den)


def test_f16w_tiled_dead_groups_keep_inf(gpu):
    """K = 96 (three 32-k groups in a 128-k step): the fourth group of each step is past the row end and
    is loaded clamped to the third, which holds a +Inf weight. The dead group reads as zeros, so the
    product stays +Inf where x is positive instead of picking up 0 * Inf = NaN."""
    M, K, N = 8, 96, 16
    rng = np.random.default_rng(5)
    x = np.abs(rng.standard_normal(M * K)).astype(np.float32) + 0.5
    w = (rng.standard_normal(N * K) * 0.05).astype(np.float16)
    w[3 * K + 70] = np.float16(np.inf)                 # column 3, k = 70 (third group)
    wb = gpu.up(w.view(np.uint16))
    y = run(gpu, x, wb, M, K, N, 2)
    assert np.all(np.isposinf(y[:, 3]))
    mask = np.ones(N, bool)
    mask[3] = False
    ref, den = O.matmul_t_f16w(x, w.view(np.uint16), M, K, N)
    assert np.all(np.abs(y[:, mask] - ref[:, mask]) <= 1e-3 * den[:, mask])


# tiles with an f16 form: one 32-column block per wave, no prefetch ring (1 + index into the tile table)
F16_TILES = [2, 5, 8, 11, 13, 14, 15, 16]


@pytest.mark.parametrize("tile", F16_TILES)
def test_f16w_every_tile(gpu, tile):
    M, K, N = 130, 352, 300            # ragged rows and columns, K of 11 groups (dead groups in the last step)
    rng = np.random.default_rng(tile)
    x = (rng.standard_normal(M * K) * 2).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.05).astype(np.float16).view(np.uint16)
    ref, den = O.matmul_t_f16w(x, w, M, K, N)
    gpu.ctx.set_option(BRIK_OPT_GEMM_TILE, tile)
    y = run(gpu, x, gpu.up(w), M, K, N, 2)
    assert np.all(np.abs(y - ref) <= 1e-3 * den + 1e-30)


def test_f16w_tile_without_f16_form_is_refused(gpu):
    w = gpu.up(np.zeros(64 * 64, np.uint16))
    gpu.ctx.set_option(BRIK_OPT_GEMM_TILE, 1)          # 128 x 256 with two column blocks per wave
    with pytest.raises(BrikError) as e:
        run(gpu, np.zeros(4 * 64, np.float32), w, 4, 64, 64, 2)
    assert e.value.code == BRIK_EINVAL
