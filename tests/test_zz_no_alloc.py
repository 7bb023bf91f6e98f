"""The no-allocation entry point (brik_matmul_t_q4_noalloc) through the C ABI against the ordinary
brik_matmul_t_q4 on the same inputs: the same kernels run on the library's fixed per-device scratch
instead of the context workspaces, so the outputs must be bit-identical. Two calls in a row, the
second smaller, on each path that uses scratch (the MFMA GEMM's staged f16 rows; the staged image of a
large M = 1 GEMV) and on one that uses none; a call needing more than the scratch holds is refused
before anything runs; and the call records into a graph and replays like the eager call.
"""
import numpy as np
import pytest

from brimkern_amd import synth
from brimkern_amd.capi import BrikError, BRIK_EINVAL, BRIK_NOALLOC_SCRATCH_BYTES
from helpers import Gpu

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()


def both(gpu, M, K, N, seed):
    """(no-allocation result, ordinary result) for one seeded q4 problem."""
    t = synth.q4_tensor(seed, N, K)
    nib, sc, mn = gpu.planes("q4", t)
    xb = gpu.up(synth.normal(seed + 1, M * K))
    ya = gpu.up(np.full(M * N, np.nan, np.float32))
    yb = gpu.up(np.full(M * N, np.nan, np.float32))
    gpu.ctx.matmul_t_q4_noalloc(xb, nib, sc, mn, ya, M, K, N)
    gpu.ctx.matmul_t_q4(xb, nib, sc, mn, yb, M, K, N)
    return gpu.ctx.download(ya, np.float32, M * N), gpu.ctx.download(yb, np.float32, M * N)


@pytest.mark.parametrize("first,second", [
    ((512, 2560, 1024), (100, 1024, 300)),       # MFMA GEMM: staged f16 rows in the scratch
    ((1, 2560, 24583), (1, 512, 24577)),         # M = 1, N >= 24576: the staged x image in the scratch
    ((1, 2560, 4096), (1, 1024, 700)),           # M = 1 GEMV staging in-block: no scratch at all
], ids=["gemm", "gemv_staged", "gemv"])
def test_noalloc_matches_ordinary_call_twice(gpu, first, second):
    for i, (M, K, N) in enumerate((first, second)):
        a, b = both(gpu, M, K, N, 900 + 10 * i)
        assert np.isfinite(b).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"call {i}: M={M} K={K} N={N}"


def test_noalloc_refuses_beyond_scratch(gpu):
    M, K, N = 2048, 4096, 64                     # 2 M roundup(K, 256) + 4 M = 16 MiB + 8 KiB
    assert 2 * M * K + 4 * M > BRIK_NOALLOC_SCRATCH_BYTES
    t = synth.q4_tensor(950, N, K)
    nib, sc, mn = gpu.planes("q4", t)
    xb = gpu.up(np.zeros(M * K, np.float32))
    yb = gpu.up(np.full(M * N, np.nan, np.float32))
    with pytest.raises(BrikError) as e:
        gpu.ctx.matmul_t_q4_noalloc(xb, nib, sc, mn, yb, M, K, N)
    assert e.value.code == BRIK_EINVAL and "scratch" in str(e.value)
    gpu.ctx.sync()
    assert np.isnan(gpu.ctx.download(yb, np.float32, M * N)).all()     # nothing ran
    # the largest row count that fits runs
    Mfit = (BRIK_NOALLOC_SCRATCH_BYTES // (2 * K + 4))
    gpu.ctx.matmul_t_q4_noalloc(xb, nib, sc, mn, yb, Mfit, K, N)
    gpu.ctx.sync()
    assert np.array_equal(gpu.ctx.download(yb, np.float32, Mfit * N), np.zeros(Mfit * N, np.float32))


def test_noalloc_records_into_a_graph(gpu):
    ctx = gpu.ctx
    M, K, N = 64, 512, 256
    t = synth.q4_tensor(960, N, K)
    nib, sc, mn = gpu.planes("q4", t)
    xb = gpu.up(np.zeros(M * K, np.float32))
    ya = gpu.up(np.zeros(M * N, np.float32))
    yb = gpu.up(np.zeros(M * N, np.float32))
    ctx.graph_begin()
    ctx.matmul_t_q4_noalloc(xb, nib, sc, mn, ya, M, K, N)
    graph = ctx.graph_end()
    try:
        for rep in range(3):
            ctx.h2d(xb, synth.normal(961 + rep, M * K))
            ctx.h2d(ya, np.full(M * N, np.nan, np.float32))
            graph.launch()
            ctx.matmul_t_q4(xb, nib, sc, mn, yb, M, K, N)          # eager work between replays
            ctx.sync()
            a, b = ctx.download(ya, np.float32, M * N), ctx.download(yb, np.float32, M * N)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"replay {rep}"
    finally:
        graph.destroy()
