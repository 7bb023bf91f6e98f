"""GPU checks of the stream fences (brik_fence_*) and the load-time self-validation
(brik_self_validate) through the C ABI: a fence's copy sees exactly the work enqueued before it, from
another thread while the context keeps enqueueing, and every built-in kernel check passes on the device.
"""
import threading

import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth
from brimkern_amd.capi import BrikError
from helpers import Gpu, normwise_rel, REL_TOL

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()


def test_self_validate_passes(ctx):
    assert ctx.self_validate() is None
    assert ctx.self_validate() is None      # repeatable: its scratch is released and re-made


def test_fence_sees_work_before_it(gpu):
    """A fence taken after one matmul: its copy holds that matmul's result although eight more (into
    another buffer) are enqueued before the copy is asked for."""
    M, K, N = 64, 2560, 4096
    t1, t2 = synth.q4_tensor(1500, N, K), synth.q4_tensor(1501, N, K)
    x = synth.normal(1502, M * K)
    p1, p2 = gpu.planes("q4", t1), gpu.planes("q4", t2)
    xb = gpu.up(x)
    y1 = gpu.up(np.zeros(M * N, np.float32))
    y2 = gpu.up(np.zeros(M * N, np.float32))
    gpu.ctx.matmul_t_q4(xb, *p1, y1, M, K, N)
    f = gpu.ctx.fence()
    try:
        for _ in range(8):
            gpu.ctx.matmul_t_q4(xb, *p2, y2, M, K, N)
        got = f.d2h(y1, np.float32, M * N)
    finally:
        f.destroy()
    r = O.matmul_t_q4(x, t1["nib"], t1["sc"], t1["mn"], M, K, N)
    assert normwise_rel(got, r) <= REL_TOL
    gpu.ctx.sync()
    r2 = O.matmul_t_q4(x, t2["nib"], t2["sc"], t2["mn"], M, K, N)
    assert normwise_rel(gpu.ctx.download(y2, np.float32, M * N), r2) <= REL_TOL


def test_fence_d2h_from_another_thread(gpu):
    """Fences drained by a worker thread while the main thread keeps enqueueing: each copy holds the
    result of the matmul its fence followed."""
    M, K, N = 8, 512, 256
    t = synth.q4_tensor(1510, N, K)
    planes = gpu.planes("q4", t)
    xs = [synth.normal(1511 + i, M * K) for i in range(6)]
    xbs = [gpu.up(x) for x in xs]
    ys = [gpu.up(np.full(M * N, np.nan, np.float32)) for _ in xs]
    busy = gpu.up(np.zeros(M * N, np.float32))
    fences = []
    for xb, yb in zip(xbs, ys):
        gpu.ctx.matmul_t_q4(xb, *planes, yb, M, K, N)
        fences.append(gpu.ctx.fence())
    out = [None] * len(xs)
    err = []

    def drain():
        try:
            for i, f in enumerate(fences):
                out[i] = f.d2h(ys[i], np.float32, M * N)
        except BrikError as e:          # reported by the assertion below
            err.append(e)

    th = threading.Thread(target=drain)
    th.start()
    for _ in range(50):                 # more work on the same stream meanwhile
        gpu.ctx.matmul_t_q4(xbs[0], *planes, busy, M, K, N)
    th.join(timeout=60)
    assert not th.is_alive() and not err, err
    for f in fences:
        f.destroy()
    for x, o in zip(xs, out):
        r = O.matmul_t_q4(x, t["nib"], t["sc"], t["mn"], M, K, N)
        assert normwise_rel(o, r) <= REL_TOL
    gpu.ctx.sync()


def test_fence_rejects_null_copy(ctx):
    f = ctx.fence()
    try:
        with pytest.raises(BrikError):
            f.d2h(None, np.float32, 4)
    finally:
        f.destroy()
