"""Recorded launches (brik_graph_*): a captured sequence of plan runs, matmuls and the sampling
passes replays to the same results as the eager calls. Every replay is checked against an eager run
on the same inputs, with eager work and synchronisations between replays, and the inputs change
between replays (the graph keeps pointers, not contents)."""
import numpy as np
import pytest

from brimkern_amd import synth
from brimkern_amd.capi import (BrikError, BRIK_EINVAL, BRIK_OPT_PATH, BRIK_PATH_GEMV, BRIK_PATH_SPLITK,
                               BRIK_PATH_TILED, PATH_AUTO, PATH_GEMM)
from helpers import Gpu

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()


def test_graph_replays_match_eager(gpu):
    ctx = gpu.ctx
    K, N, M, vocab, k = 1024, 2048, 64, 20000, 16
    t = synth.q4_tensor(120, N, K)
    nib, sc, mn = gpu.planes("q4", t)
    tq = synth.tensor("q3", 121, vocab, K)
    qp = gpu.planes("q3", tq)
    x1 = gpu.up(np.zeros(K, np.float32))
    xm = gpu.up(np.zeros(M * K, np.float32))
    g1 = gpu.up(np.zeros(K, np.float32))
    w1 = gpu.up(np.ones(K, np.float32))
    y1 = gpu.up(np.zeros(N, np.float32))
    ym = gpu.up(np.zeros(M * N, np.float32))
    ids = gpu.up(np.zeros(2 * k, np.int32))
    plan = ctx.gemv_plan("q4", [dict(x=x1, p0=nib, sc=sc, mn=mn, y=y1, K=K, N=N, gate=g1, norm_w=w1, eps=1e-6)])

    def enqueue():
        plan.run()
        ctx.matmul_t_q4(xm, nib, sc, mn, ym, M, K, N)
        ctx.lm_head_topk("q3", x1, qp, K, vocab, None, 0, 1.0, 30.0, k, ids, ids.offset(4 * k))

    def results():
        return (ctx.download(y1, np.float32, N), ctx.download(ym, np.float32, M * N),
                ctx.download(ids, np.int32, 2 * k))

    def set_inputs(seed):
        ctx.h2d(x1, synth.normal(seed, K))
        ctx.h2d(xm, synth.normal(seed + 1, M * K))
        ctx.h2d(g1, synth.normal(seed + 2, K))

    set_inputs(1)
    enqueue()                     # grows the workspaces before the capture
    ctx.sync()
    ctx.graph_begin()
    enqueue()
    graph = ctx.graph_end()
    try:
        for rep, seed in enumerate((10, 20, 20, 30)):
            set_inputs(seed)
            enqueue()
            ctx.sync()
            eager = results()
            ctx.h2d(y1, np.full(N, np.nan, np.float32))          # the replay must overwrite
            ctx.h2d(ym, np.full(M * N, np.nan, np.float32))
            graph.launch()
            ctx.sync()
            got = results()
            for a, b in zip(eager, got):
                assert np.array_equal(a, b), f"replay {rep}"
            ctx.matmul_t_q4(xm, nib, sc, mn, ym, M, K, N)       # eager work between replays
            ctx.sync()
    finally:
        graph.destroy()
        plan.destroy()


def test_capture_refuses_workspace_growth_and_copies(gpu):
    ctx = gpu.ctx
    K, N, M = 2048, 256, 8192          # a 32 MiB GEMM staging workspace, larger than any earlier call needed
    t = synth.q4_tensor(130, N, K)
    nib, sc, mn = gpu.planes("q4", t)
    xm = gpu.up(synth.normal(131, M * K))
    ym = gpu.up(np.zeros(M * N, np.float32))
    ctx.graph_begin()
    with pytest.raises(BrikError) as e:
        ctx.matmul_t_q4(xm, nib, sc, mn, ym, M, K, N)
    assert e.value.code == BRIK_EINVAL
    with pytest.raises(BrikError) as e:
        ctx.h2d(ym, np.zeros(4, np.float32))
    assert e.value.code == BRIK_EINVAL
    ctx.graph_end().destroy()
    # after the capture the same call runs eagerly
    ctx.matmul_t_q4(xm, nib, sc, mn, ym, M, K, N)
    ctx.sync()
    assert np.isfinite(ctx.download(ym, np.float32, M * N)).all()


def test_replay_after_workspace_reallocation_is_refused(gpu):
    """A graph records the context workspace's address; an eager call that needs a larger workspace
    frees and reallocates it, after which replaying the old graph would touch freed memory. The
    library refuses that launch (no GPU work is enqueued) and a graph recorded afterwards replays. A
    graph whose launches hold no workspace address (a GEMV) still replays after the reallocation."""
    ctx = gpu.ctx
    K, N, M = 256, 64, 16
    t = synth.q4_tensor(140, N, K)
    nib, sc, mn = gpu.planes("q4", t)
    xm = gpu.up(synth.normal(141, M * K))
    ym = gpu.up(np.zeros(M * N, np.float32))
    yg = gpu.up(np.zeros(M * N, np.float32))
    # the MFMA GEMM path (staged rows in the context workspace) for the recorded call
    ctx.set_option(BRIK_OPT_PATH, PATH_GEMM)
    try:
        ctx.matmul_t_q4(xm, nib, sc, mn, ym, M, K, N)
        assert ctx.last_path() in (BRIK_PATH_TILED, BRIK_PATH_SPLITK)
        ctx.sync()
        ctx.graph_begin()
        ctx.matmul_t_q4(xm, nib, sc, mn, ym, M, K, N)
        old = ctx.graph_end()
    finally:
        ctx.set_option(BRIK_OPT_PATH, PATH_AUTO)
    ctx.matmul_t_q4(xm, nib, sc, mn, yg, M, K, N)
    assert ctx.last_path() == BRIK_PATH_GEMV
    ctx.sync()
    ctx.graph_begin()
    ctx.matmul_t_q4(xm, nib, sc, mn, yg, M, K, N)
    gemv_graph = ctx.graph_end()
    # 128 MiB of staged activation rows (M_big x K_big halves): more than any earlier call of the session
    M_big, K_big = 16384, 4096
    xb = gpu.up(np.zeros(M_big * K_big, np.float32))
    yb = gpu.up(np.zeros(M_big * 32, np.float32))
    tb = synth.q4_tensor(142, 32, K_big)
    ctx.matmul_t_q4(xb, *gpu.planes("q4", tb), yb, M_big, K_big, 32)
    ctx.sync()
    try:
        with pytest.raises(BrikError) as e:
            old.launch()
        assert e.value.code == BRIK_EINVAL
        eager = ctx.download(yg, np.float32, M * N)
        ctx.h2d(yg, np.full(M * N, np.nan, np.float32))
        gemv_graph.launch()
        ctx.sync()
        assert np.array_equal(ctx.download(yg, np.float32, M * N), eager)
    finally:
        old.destroy()
        gemv_graph.destroy()
    ctx.set_option(BRIK_OPT_PATH, PATH_GEMM)
    try:
        ctx.graph_begin()
        ctx.matmul_t_q4(xm, nib, sc, mn, ym, M, K, N)
        new = ctx.graph_end()
    finally:
        ctx.set_option(BRIK_OPT_PATH, PATH_AUTO)
    try:
        ctx.set_option(BRIK_OPT_PATH, PATH_GEMM)
        ctx.matmul_t_q4(xm, nib, sc, mn, ym, M, K, N)
        ctx.set_option(BRIK_OPT_PATH, PATH_AUTO)
        ctx.sync()
        eager = ctx.download(ym, np.float32, M * N)
        ctx.h2d(ym, np.full(M * N, np.nan, np.float32))
        new.launch()
        ctx.sync()
        assert np.array_equal(ctx.download(ym, np.float32, M * N), eager)
    finally:
        new.destroy()
