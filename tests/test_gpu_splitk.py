"""GPU parity of the split-K few-row GEMM (brik_gemm_sk_<fmt>_k<KSL>) through the C ABI: dense calls of
few rows and expert-grouped (MoE) calls, against the oracle at the 1e-3 bar (normwise and
componentwise), over every slice size the runtime picks from (one slice, and several slices whose
partials the last block of each tile sums), ragged M / N / K, empty experts and experts of more than
one 32-row tile. The sum over slices runs in slice order whatever order the blocks finish in, so
repeated calls are bit-identical; the tile counters are left at zero by every call, so calls of other
shapes in between do not disturb it.
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth
from brimkern_amd.capi import BRIK_OPT_PATH, BRIK_OPT_SPLITK, BRIK_OPT_GEMM_TILE
from helpers import Gpu, PLANES, normwise_rel, componentwise_ok, REL_TOL

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    ctx.set_option(BRIK_OPT_SPLITK, 2)
    ctx.set_option(BRIK_OPT_PATH, 2)        # the MFMA path, whatever the small-M routing would pick
    yield g
    ctx.set_option(BRIK_OPT_SPLITK, 0)
    ctx.set_option(BRIK_OPT_PATH, 0)
    ctx.set_option(BRIK_OPT_GEMM_TILE, 0)
    g.free()


def check(y, r, den):
    rel = normwise_rel(y, r)
    assert rel <= REL_TOL, f"normwise rel {rel:.3e}"
    assert componentwise_ok(y, r, den, REL_TOL), "componentwise bound violated"


def oracle_mm(fmt, x, t, M):
    return getattr(O, f"matmul_t_{fmt}")(x, *[t[k] for k in PLANES[fmt]], M, t["K"], t["N"], absden=True)


# (M, K, N): one slice (K = 256: 2 steps), several slices (K = 2560: 20 steps, K = 9728: 76), K not a
# multiple of 128 (dead groups in the last step), N not a multiple of 128, M past one 32-row tile
SHAPES = [(1, 256, 300), (2, 2560, 1024), (5, 2560, 4096), (8, 9728, 2560), (17, 1056, 777), (33, 160, 130),
          (64, 2560, 9728), (3, 96, 65)]


@pytest.mark.parametrize("fmt", ["q4", "q8", "q3"])
@pytest.mark.parametrize("M,K,N", SHAPES)
def test_splitk_dense(gpu, fmt, M, K, N):
    t = synth.tensor(fmt, 1000 + M + K, N, K)
    x = synth.normal(1001 + M, M * K)
    planes = gpu.planes(fmt, t)
    r, den = oracle_mm(fmt, x, t, M)
    y = gpu.matmul(fmt, x, planes, M, K, N)
    check(y, r, den)
    # again, after a call of another shape: bit-identical (slice order, counters back at zero)
    t2 = synth.tensor(fmt, 1100, 200, 512)
    gpu.matmul(fmt, synth.normal(1101, 7 * 512), gpu.planes(fmt, t2), 7, 512, 200)
    y2 = gpu.matmul(fmt, x, planes, M, K, N)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def test_splitk_matches_tiled_kernel(gpu):
    """The same product through the split-K kernel and through a forced tile of the tiled kernel: both
    within the bar of the oracle (they add the same f16 products in different orders)."""
    M, K, N = 24, 2560, 1100
    t = synth.q4_tensor(1200, N, K)
    x = synth.normal(1201, M * K)
    planes = gpu.planes("q4", t)
    r, den = oracle_mm("q4", x, t, M)
    a = gpu.matmul("q4", x, planes, M, K, N)
    gpu.ctx.set_option(BRIK_OPT_GEMM_TILE, 8)
    b = gpu.matmul("q4", x, planes, M, K, N)
    check(a, r, den)
    check(b, r, den)


@pytest.mark.parametrize("K,N", [(2048, 768), (768, 2048), (1056, 300)])
def test_splitk_moe(gpu, K, N):
    """Expert-grouped: routed rows of 0 to 70 per expert (empty experts, experts spanning three 32-row
    tiles), every slice count the shapes give."""
    E = 10
    counts = np.array([0, 5, 33, 70, 0, 1, 32, 64, 20, 0])
    row_off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    R = int(row_off[-1])
    t = synth.q4_tensor(1300 + K, E * N, K)
    x = synth.normal(1301, R * K)
    planes = gpu.planes("q4", t)
    xb, rb = gpu.up(x), gpu.up(row_off)
    yb = gpu.up(np.full(R * N, np.nan, np.float32))
    gpu.ctx.moe_matmul_t_q4(xb, rb, *planes, yb, E, R, K, N)
    y = gpu.ctx.download(yb, np.float32, R * N).reshape(R, N)
    r = O.moe_matmul_t_q4(x, row_off, t["nib"], t["sc"], t["mn"], E, K, N)
    deq = O.dequant_q4(t["nib"], t["sc"], t["mn"]).reshape(E, N, K).astype(np.float64)
    xr = np.abs(x.reshape(R, K).astype(np.float64))
    den = np.zeros((R, N))
    for e in range(E):
        a, b = row_off[e], row_off[e + 1]
        den[a:b] = xr[a:b] @ np.abs(deq[e]).T
    check(y, r.reshape(R, N), den)
    gpu.ctx.moe_matmul_t_q4(xb, rb, *planes, yb, E, R, K, N)
    y2 = gpu.ctx.download(yb, np.float32, R * N).reshape(R, N)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def test_splitk_moe_cfg5_shapes(gpu):
    """The benchmark's MoE layer (256 tokens, top-8 of 64 experts, gate 2048 -> 768, down 768 -> 2048) on
    the automatic choice, which is the split-K kernel for expert-grouped calls."""
    gpu.ctx.set_option(BRIK_OPT_SPLITK, 0)
    T, H, E, F, TOPK = 256, 2048, 64, 768, 8
    rows, row_off = synth.moe_routing(77, T, E, TOPK)
    R = rows.size
    for K, N, seed in ((H, F, 1400), (F, H, 1401)):
        t = synth.q4_tensor(seed, E * N, K)
        x = synth.normal(seed + 1, R * K)
        planes = gpu.planes("q4", t)
        xb, rb = gpu.up(x), gpu.up(row_off)
        yb = gpu.up(np.full(R * N, np.nan, np.float32))
        gpu.ctx.moe_matmul_t_q4(xb, rb, *planes, yb, E, R, K, N)
        y = gpu.ctx.download(yb, np.float32, R * N)
        r = O.moe_matmul_t_q4(x, row_off, t["nib"], t["sc"], t["mn"], E, K, N)
        assert normwise_rel(y, r) <= REL_TOL
