"""The no-allocation entry point (brik_matmul_t_q4_noalloc) through the C ABI against the ordinary
brik_matmul_t_q4 on the same inputs: the same kernels run on the library's fixed per-device scratch
instead of the context workspaces, so the outputs must be bit-identical. Two calls in a row, the
second smaller, on each path that uses scratch (the tiled MFMA GEMM's staged f16 rows; the split-K
GEMM's staged rows and partial tiles; the staged image of a large M = 1 GEMV) and on one that uses
none, each call's path asserted (brik_last_path); a call needing more than the scratch holds is refused
before anything runs; and the call records into a graph and replays like the eager call, also after a
larger eager call has reallocated the context workspace.
"""
import numpy as np
import pytest

from brimkern_amd import synth
from brimkern_amd.capi import (BrikError, Context, BRIK_EINVAL, BRIK_NOALLOC_SCRATCH_BYTES, BRIK_PATH_GEMV,
                               BRIK_PATH_GEMV_STAGED, BRIK_PATH_SPLITK, BRIK_PATH_TILED)
from helpers import Gpu

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()


def both(gpu, M, K, N, seed):
    """(no-allocation result, ordinary result, path of each) for one seeded q4 problem."""
    t = synth.q4_tensor(seed, N, K)
    nib, sc, mn = gpu.planes("q4", t)
    xb = gpu.up(synth.normal(seed + 1, M * K))
    ya = gpu.up(np.full(M * N, np.nan, np.float32))
    yb = gpu.up(np.full(M * N, np.nan, np.float32))
    gpu.ctx.matmul_t_q4_noalloc(xb, nib, sc, mn, ya, M, K, N)
    pa = gpu.ctx.last_path()
    gpu.ctx.matmul_t_q4(xb, nib, sc, mn, yb, M, K, N)
    pb = gpu.ctx.last_path()
    return gpu.ctx.download(ya, np.float32, M * N), gpu.ctx.download(yb, np.float32, M * N), (pa, pb)


@pytest.mark.parametrize("first,second,path", [
    ((512, 2560, 1024), (96, 2560, 1024), BRIK_PATH_TILED),       # staged f16 rows in the scratch
    ((32, 9728, 2560), (24, 2560, 2560), BRIK_PATH_SPLITK),       # staged rows, then the partial tiles
    ((1, 2560, 24583), (1, 512, 24577), BRIK_PATH_GEMV_STAGED),   # the staged x image in the scratch
    ((1, 2560, 4096), (1, 1024, 700), BRIK_PATH_GEMV),            # staging in-block: no scratch at all
], ids=["gemm", "splitk", "gemv_staged", "gemv"])
def test_noalloc_matches_ordinary_call_twice(gpu, first, second, path):
    for i, (M, K, N) in enumerate((first, second)):
        print(f"noalloc call {i}: M={M} K={K} N={N}", flush=True)
        a, b, paths = both(gpu, M, K, N, 900 + 10 * i)
        assert paths == (path, path), f"call {i}: M={M} K={K} N={N} took paths {paths}"
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


def test_noalloc_refuses_splitk_partials_beyond_scratch(gpu):
    """A split-K shape whose staged rows fit (2 MiB) but whose partial tiles (16 slices x 64 x 8192 f32,
    32 MiB) do not: refused before anything is enqueued. The planes are never read."""
    ctx = gpu.ctx
    M, K, N = 64, 16384, 8192
    bufs = [ctx.alloc(N * K // 2), ctx.alloc(N * K // 16), ctx.alloc(N * K // 16)]
    gpu.bufs.extend(bufs)
    xb = gpu.up(np.zeros(M * K, np.float32))
    yb = gpu.up(np.full(M * N, np.nan, np.float32))
    with pytest.raises(BrikError) as e:
        ctx.matmul_t_q4_noalloc(xb, *bufs, yb, M, K, N)
    assert e.value.code == BRIK_EINVAL and "split-K" in str(e.value)
    ctx.sync()
    assert np.isnan(ctx.download(yb, np.float32, M * N)).all()     # nothing ran


@pytest.mark.parametrize("M,K,N,path", [(128, 2560, 1024, BRIK_PATH_TILED), (24, 2560, 2560, BRIK_PATH_SPLITK)],
                         ids=["tiled", "splitk"])
def test_noalloc_records_into_a_graph(M, K, N, path):
    """Replays equal the eager ordinary call; between replays the ordinary call runs on the context
    workspaces, and before the last replay a larger ordinary call reallocates them (a fresh context, so
    the workspaces start empty): the recorded graph holds only the fixed scratch's address, so it
    still replays."""
    ctx = Context(0)
    gpu = Gpu(ctx)
    try:
        graph_case(ctx, gpu, M, K, N, path)
    finally:
        gpu.free()
        ctx.close()


def graph_case(ctx, gpu, M, K, N, path):
    t = synth.q4_tensor(960, N, K)
    nib, sc, mn = gpu.planes("q4", t)
    xb = gpu.up(np.zeros(M * K, np.float32))
    ya = gpu.up(np.zeros(M * N, np.float32))
    yb = gpu.up(np.zeros(M * N, np.float32))
    Mbig = 1024                                   # a larger GEMM: grows the context workspace
    xbig = gpu.up(np.zeros(Mbig * K, np.float32))
    ybig = gpu.up(np.zeros(Mbig * N, np.float32))
    ctx.matmul_t_q4_noalloc(xb, nib, sc, mn, ya, M, K, N)      # the shape's path, outside the capture
    assert ctx.last_path() == path
    ctx.sync()
    ctx.graph_begin()
    ctx.matmul_t_q4_noalloc(xb, nib, sc, mn, ya, M, K, N)
    graph = ctx.graph_end()
    try:
        for rep in range(3):
            print(f"noalloc graph replay {rep}: M={M} K={K} N={N}", flush=True)
            ctx.h2d(xb, synth.normal(961 + rep, M * K))
            ctx.h2d(ya, np.full(M * N, np.nan, np.float32))
            if rep == 2:
                ctx.matmul_t_q4(xbig, nib, sc, mn, ybig, Mbig, K, N)
            graph.launch()
            ctx.matmul_t_q4(xb, nib, sc, mn, yb, M, K, N)          # eager work between replays
            assert ctx.last_path() == path
            ctx.sync()
            a, b = ctx.download(ya, np.float32, M * N), ctx.download(yb, np.float32, M * N)
            assert np.isfinite(b).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"replay {rep}"
    finally:
        graph.destroy()
