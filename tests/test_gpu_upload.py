"""brik_h2d_async (the reference's queue.writeBuffer, kernels.ts:231-235) through the C ABI: the bytes are
staged at once (the source changes right after each call), uploads wrap around the pinned staging ring
many times, an upload is ordered against the kernels enqueued before and after it on the context stream,
uploads larger than half the ring take the blocking path, and a graph capture refuses it."""
import numpy as np
import pytest

from brimkern_amd import synth
from brimkern_amd.capi import BrikError, BRIK_EINVAL, BRIK_STAGING_RING_BYTES
from helpers import Gpu

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()


def test_staged_uploads_wrap_the_ring(gpu):
    ctx = gpu.ctx
    rng = np.random.default_rng(5)
    sizes = [int(s) for s in rng.integers(1, 3 << 20, 60)]         # ~90 MB in total: the ring wraps
    assert sum(sizes) > 2 * BRIK_STAGING_RING_BYTES
    bufs = [ctx.alloc(n) for n in sizes]
    gpu.bufs.extend(bufs)
    expect = []
    src = np.empty(max(sizes), np.uint8)
    for i, (b, n) in enumerate(zip(bufs, sizes)):
        src[:n] = rng.integers(0, 256, n, dtype=np.uint8)
        expect.append(src[:n].copy())
        ctx.h2d_async(b, src[:n])
        src[:n] ^= 0xFF                                            # the caller reuses its array at once
    ctx.sync()
    for i, (b, n) in enumerate(zip(bufs, sizes)):
        assert np.array_equal(ctx.download(b, np.uint8, n), expect[i]), f"upload {i} ({n} bytes)"


def test_upload_is_ordered_with_kernels(gpu):
    """x, matmul, new x into the same buffer, matmul: each matmul sees the x uploaded before it."""
    ctx = gpu.ctx
    K, N = 2560, 1024
    t = synth.q4_tensor(40, N, K)
    nib, sc, mn = gpu.planes("q4", t)
    xb = gpu.up(np.zeros(K, np.float32))
    ya, yb, yc, yd = (gpu.up(np.zeros(N, np.float32)) for _ in range(4))
    xa, x2 = synth.normal(41, K), synth.normal(42, K)
    ctx.h2d_async(xb, xa)
    ctx.matmul_t_q4(xb, nib, sc, mn, ya, 1, K, N)
    ctx.h2d_async(xb, x2)
    ctx.matmul_t_q4(xb, nib, sc, mn, yb, 1, K, N)
    ctx.sync()
    ctx.h2d(xb, xa)
    ctx.matmul_t_q4(xb, nib, sc, mn, yc, 1, K, N)
    ctx.h2d(xb, x2)
    ctx.matmul_t_q4(xb, nib, sc, mn, yd, 1, K, N)
    ctx.sync()
    got = [ctx.download(y, np.float32, N) for y in (ya, yb, yc, yd)]
    assert np.array_equal(got[0], got[2]) and np.array_equal(got[1], got[3])
    assert not np.array_equal(got[0], got[1])


def test_large_upload_takes_the_blocking_path(gpu):
    ctx = gpu.ctx
    n = BRIK_STAGING_RING_BYTES // 2 + 4096
    a = np.random.default_rng(6).integers(0, 256, n, dtype=np.uint8)
    b = ctx.alloc(n)
    gpu.bufs.append(b)
    ctx.h2d_async(b, a)
    ctx.sync()
    assert np.array_equal(ctx.download(b, np.uint8, n), a)


def test_capture_refuses_the_upload(gpu):
    ctx = gpu.ctx
    b = gpu.up(np.zeros(64, np.float32))
    ctx.graph_begin()
    try:
        with pytest.raises(BrikError) as e:
            ctx.h2d_async(b, np.ones(64, np.float32))
        assert e.value.code == BRIK_EINVAL
    finally:
        ctx.graph_end().destroy()
