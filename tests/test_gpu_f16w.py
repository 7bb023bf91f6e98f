"""GPU parity of the f16-weight matmul (brik_matmul_t_f16w, the reference's MATMUL_T_F16W) through the C
ABI, against y = x . W^T in f64 (W widened exactly from its f16 bits). The streaming kernel accumulates
in f32 (bar: the f32 summation bound (K + 2) 2^-24 sum |x w|); the MFMA kernel stages x as row-scaled
f16 (the matmuls' bar 1e-3 sum |x w|). Both run on every shape that allows them."""
import numpy as np
import pytest

import oracle as O
from brimkern_amd.capi import BrikError, BRIK_EINVAL, BRIK_EALIGN, BRIK_OPT_PATH
from brimkern_amd.engine import Engine
from helpers import Gpu

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()
    ctx.set_option(BRIK_OPT_PATH, 0)


def run(gpu, x, wb, M, K, N, path):
    xb = gpu.up(x)
    yb = gpu.ctx.alloc(max(M * N, 1) * 4)
    gpu.bufs.append(yb)
    gpu.ctx.set_option(BRIK_OPT_PATH, path)
    gpu.ctx.matmul_t_f16w(xb, wb, yb, M, K, N)
    return gpu.ctx.download(yb, np.float32, M * N).reshape(M, N)


@pytest.mark.parametrize("M,K,N", [(1, 2560, 9728), (1, 100, 37), (1, 16384, 64), (2, 256, 130), (5, 260, 33),
                                   (64, 2560, 1000), (200, 512, 129), (3, 8, 1), (130, 1024, 256)])
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
