"""GPU parity of brik_moe_matmul_t_q4_x2 (two expert-stacked q4 tensors on the same routed rows, one
x staging and one launch) through the C ABI: each output bit-identical to its own
brik_moe_matmul_t_q4 call, and within the 1e-3 bar of the per-expert oracle, on the benchmark's
64-expert layer, under every tile, with empty experts, experts past one row tile, a malformed row
table and K = 0; argument errors are reported before anything runs.
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth
from brimkern_amd.capi import BrikError, BRIK_OPT_GEMM_TILE, BRIK_OPT_SPLITK, BRIK_GEMM_TILES
from helpers import Gpu, componentwise_ok, moe_oracle_abs, normwise_rel, REL_TOL

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    ctx.set_option(BRIK_OPT_GEMM_TILE, 0)
    ctx.set_option(BRIK_OPT_SPLITK, 0)
    g.free()


def run_pair(gpu, x, row_off, ta, tb, E, K, N):
    """(x2 outputs, single-call outputs) for tensors ta, tb."""
    R = int(row_off[-1])
    pa, pb = gpu.planes("q4", ta), gpu.planes("q4", tb)
    xb, rb = gpu.up(np.ascontiguousarray(x, np.float32)), gpu.up(row_off)
    ya = gpu.up(np.full(max(R * N, 1), np.nan, np.float32))
    yb = gpu.up(np.full(max(R * N, 1), np.nan, np.float32))
    gpu.ctx.moe_matmul_t_q4_x2(xb, rb, pa, ya, pb, yb, E, R, K, N)
    pair = [gpu.ctx.download(b, np.float32, R * N) for b in (ya, yb)]
    single = []
    for p in (pa, pb):
        ys = gpu.up(np.full(max(R * N, 1), np.nan, np.float32))
        gpu.ctx.moe_matmul_t_q4(xb, rb, *p, ys, E, R, K, N)
        single.append(gpu.ctx.download(ys, np.float32, R * N))
    return pair, single


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_x2_benchmark_layer(gpu):
    """The benchmark's gate/up pair: 256 tokens, top-8 of 64 experts, 2048 -> 768."""
    T, H, E, F, TOPK = 256, 2048, 64, 768, 8
    rows, row_off = synth.moe_routing(77, T, E, TOPK)
    x = synth.normal(1600, T * H).reshape(T, H)[rows]
    ta, tb = synth.q4_tensor(1601, E * F, H), synth.q4_tensor(1602, E * F, H)
    (ya, yb), (sa, sb) = run_pair(gpu, x, row_off, ta, tb, E, H, F)
    assert same_bits(ya, sa) and same_bits(yb, sb)
    for y, t in ((ya, ta), (yb, tb)):
        r = O.moe_matmul_t_q4(x, row_off, t["nib"], t["sc"], t["mn"], E, H, F)
        ra, den = moe_oracle_abs(x, row_off, t, E, H, F)
        assert np.array_equal(ra, r)
        assert normwise_rel(y, r) <= REL_TOL
        assert componentwise_ok(y, r, den), "componentwise bound violated"


@pytest.mark.parametrize("tile", range(0, BRIK_GEMM_TILES + 1))
def test_x2_every_tile(gpu, tile):
    """Uneven experts (an empty one, some past 64 rows) under every tile."""
    E, K, N = 12, 1536, 160
    row_off = np.array([0, 3, 3, 40, 110, 111, 150, 230, 250, 251, 300, 330, 332], np.int32)
    R = int(row_off[-1])
    x = synth.normal(1610, R * K)
    ta, tb = synth.q4_tensor(1611, E * N, K), synth.q4_tensor(1612, E * N, K)
    gpu.ctx.set_option(BRIK_OPT_GEMM_TILE, tile)
    (ya, yb), (sa, sb) = run_pair(gpu, x, row_off, ta, tb, E, K, N)
    assert same_bits(ya, sa) and same_bits(yb, sb)
    for y, t in ((ya, ta), (yb, tb)):
        r, den = moe_oracle_abs(x, row_off, t, E, K, N)
        assert normwise_rel(y, r) <= REL_TOL
        assert componentwise_ok(y, r, den), "componentwise bound violated"


def test_x2_forced_splitk(gpu):
    """With the split-K kernel forced, the pair runs as two split-K launches on one staging."""
    E, K, N = 6, 1024, 96
    row_off = np.array([0, 0, 20, 50, 51, 90, 120], np.int32)
    R = int(row_off[-1])
    x = synth.normal(1620, R * K)
    ta, tb = synth.q4_tensor(1621, E * N, K), synth.q4_tensor(1622, E * N, K)
    gpu.ctx.set_option(BRIK_OPT_SPLITK, 2)
    (ya, yb), (sa, sb) = run_pair(gpu, x, row_off, ta, tb, E, K, N)
    assert same_bits(ya, sa) and same_bits(yb, sb)
    for y, t in ((ya, ta), (yb, tb)):
        r, den = moe_oracle_abs(x, row_off, t, E, K, N)
        assert normwise_rel(y, r) <= REL_TOL
        assert componentwise_ok(y, r, den), "componentwise bound violated"


def test_x2_malformed_row_table(gpu):
    """Decreasing offsets count as empty experts and rows stay clipped to R: no write past row R."""
    E, K, N = 5, 256, 64
    row_off = np.array([0, 30, 10, 40, 40, 60], np.int32)      # expert 1 "negative", as the single call
    R = int(row_off[-1])
    x = synth.normal(1630, R * K)
    ta, tb = synth.q4_tensor(1631, E * N, K), synth.q4_tensor(1632, E * N, K)
    pa, pb = gpu.planes("q4", ta), gpu.planes("q4", tb)
    xb, rb = gpu.up(x), gpu.up(row_off)
    guard = 64 * N
    ya = gpu.up(np.full(R * N + guard, 7.0, np.float32))
    yb = gpu.up(np.full(R * N + guard, 7.0, np.float32))
    gpu.ctx.moe_matmul_t_q4_x2(xb, rb, pa, ya, pb, yb, E, R, K, N)
    for b in (ya, yb):
        assert np.all(gpu.ctx.download(b, np.float32, R * N + guard)[R * N:] == 7.0)


def test_x2_k0_and_errors(gpu):
    E, N = 3, 32
    row_off = np.array([0, 2, 2, 5], np.int32)
    t = synth.q4_tensor(1640, E * N, 64)
    p = gpu.planes("q4", t)
    xb, rb = gpu.up(synth.normal(1641, 5 * 64)), gpu.up(row_off)
    ya = gpu.up(np.full(5 * N, 3.0, np.float32))
    yb = gpu.up(np.full(5 * N, 3.0, np.float32))
    gpu.ctx.moe_matmul_t_q4_x2(xb, rb, p, ya, p, yb, E, 5, 0, N)        # K == 0: both zero
    assert np.all(gpu.ctx.download(ya, np.float32, 5 * N) == 0) and np.all(gpu.ctx.download(yb, np.float32, 5 * N) == 0)
    with pytest.raises(BrikError):                                      # K not a multiple of 32
        gpu.ctx.moe_matmul_t_q4_x2(xb, rb, p, ya, p, yb, E, 5, 48, N)
    with pytest.raises(BrikError):                                      # second output missing
        gpu.ctx.moe_matmul_t_q4_x2(xb, rb, p, ya, p, None, E, 5, 64, N)
