"""GPU parity: the HIP kernels through the C ABI against the CPU oracle on identical seeded inputs.

Bars (from the task): dequantized weights bit-exact; outputs within max relative error 1e-3 with
f32 accumulation, measured normwise (max|y - r| / max|r|) and componentwise
(|y - r| <= 1e-3 * sum_k |x_k w_k|). The M == 1 GEMV keeps f32 arithmetic end to end and is held
to a tighter 1e-5; the MFMA GEMM rounds operands to f16 and is held to the 1e-3 bar.
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth, layout
from brimkern_amd.capi import (BrikError, BRIK_EINVAL, BRIK_EALIGN, BRIK_OPT_PATH, BRIK_OPT_GEMV_VARIANT,
                               BRIK_GEMV_VARIANTS, BRIK_OPT_GEMM_TILE, BRIK_GEMM_TILES)
from helpers import Gpu, load_golden, normwise_rel, componentwise_ok, moe_oracle_abs, PLANES, REL_TOL

pytestmark = pytest.mark.gpu
GEMV_TOL = 1e-5
CASES, MOE = load_golden()


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    ctx.set_option(BRIK_OPT_PATH, 0)
    ctx.set_option(BRIK_OPT_GEMV_VARIANT, 0)
    ctx.set_option(BRIK_OPT_GEMM_TILE, 0)
    g.free()


def oracle_mm(fmt, x, t, M, K, N, absden=True):
    args = [t[k] for k in PLANES[fmt]]
    return {"q8": O.matmul_t_q8, "q4": O.matmul_t_q4, "q3": O.matmul_t_q3}[fmt](x, *args, M, K, N, absden=absden)


def oracle_deq(fmt, t):
    args = [t[k] for k in PLANES[fmt]]
    return {"q8": O.dequant_q8, "q4": O.dequant_q4, "q3": O.dequant_q3}[fmt](*args)


def check(y, r, den, tol):
    rel = normwise_rel(y, r)
    assert rel <= tol, f"normwise rel {rel:.3e} > {tol}"
    assert componentwise_ok(y, r, den, tol), "componentwise bound violated"
    return rel


# ---- golden fixtures (reference selfValidate shapes) -----------------------------------

@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_golden_fixture(gpu, case):
    fmt, M, K, N = case["fmt"], case["M"], case["K"], case["N"]
    planes = gpu.planes(fmt, case)
    assert np.array_equal(gpu.dequant(fmt, planes, N * K), case["deq"])
    y = gpu.matmul(fmt, case["x"], planes, M, K, N)
    r = case["y"].reshape(M, N)
    assert normwise_rel(y, r) <= (GEMV_TOL if M == 1 else REL_TOL)
    if M == 1:
        # the reference's own gate, |got - ref| < 1e-3 absolute (kernels.ts:2263-2264), holds for the
        # f32 GEMV; the f16-operand MFMA path (M >= 2) is held to the 1e-3 relative bar instead
        assert np.abs(y - r).max() < 1e-3


def test_golden_moe(gpu):
    m = MOE
    E, K, N, R = m["E"], m["K"], m["N"], m["R"]
    planes = gpu.planes("q4", dict(m, N=E * N))
    xb, rb = gpu.up(m["x"]), gpu.up(m["row_off"])
    yb = gpu.up(np.zeros(R * N, np.float32))
    gpu.ctx.moe_matmul_t_q4(xb, rb, *planes, yb, E, R, K, N)
    y = gpu.ctx.download(yb, np.float32, R * N)
    assert normwise_rel(y, m["y"]) <= REL_TOL


# ---- dequant bit-exactness at the full benchmark sizes ----------------------------------------

@pytest.mark.parametrize("fmt,N,K,seed", [
    ("q8", 4864, 896, 1),        # Qwen2.5-0.5B FFN
    ("q4", 9728, 2560, 2),       # Qwen3-4B gate/up (also the prefill GEMM weight)
    ("q4", 2560, 9728, 3),       # Qwen3-4B down
    ("q3", 151936, 2560, 4),     # Qwen3-4B q3 LM head
])
def test_dequant_bit_exact(gpu, fmt, N, K, seed):
    t = synth.tensor(fmt, seed, N, K)
    planes = gpu.planes(fmt, t)
    got = gpu.dequant(fmt, planes, N * K)
    assert np.array_equal(got.view(np.uint32), oracle_deq(fmt, t).view(np.uint32))


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_one_hot_gemv_is_dequant_column(gpu, fmt):
    """x = e_k makes the GEMV output column k of deq(W) exactly: pins the in-register dequant."""
    N, K = 300, 2560
    t = synth.tensor(fmt, 9, N, K)
    planes = gpu.planes(fmt, t)
    deq = oracle_deq(fmt, t).reshape(N, K)
    for k in (0, 1, 7, 31, 32, 1000, 2559):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        y = gpu.matmul(fmt, x, planes, 1, K, N)
        assert np.array_equal(y.ravel().view(np.uint32), deq[:, k].copy().view(np.uint32)), f"k={k}"


# ---- decode GEMV at the benchmark shapes -------------------------------------------------

GEMV_SHAPES = [
    ("q8", 896, 4864),                                     # Qwen2.5-0.5B FFN
    ("q4", 2560, 4096), ("q4", 2560, 1024), ("q4", 2560, 9728), ("q4", 9728, 2560),   # Qwen3-4B layer set
    ("q3", 2560, 151936),                                  # Qwen3-4B LM head
]


@pytest.mark.parametrize("fmt,K,N", GEMV_SHAPES)
def test_gemv_baseline_shapes(gpu, fmt, K, N):
    t = synth.tensor(fmt, 17 + N, N, K)
    x = synth.normal(5 + K, K)
    planes = gpu.planes(fmt, t)
    y = gpu.matmul(fmt, x, planes, 1, K, N)
    r, den = oracle_mm(fmt, x, t, 1, K, N)
    check(y, r, den, GEMV_TOL)


@pytest.mark.parametrize("variant", range(1, BRIK_GEMV_VARIANTS + 1))
@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_gemv_variants(gpu, fmt, variant):
    """Every GEMV tiling variant (team width, rows per team, pipeline depth), single and grouped,
    at a ragged shape (N odd, K/32 not a multiple of the team width)."""
    K, N = 1056, 777
    t = synth.tensor(fmt, 23, N, K)
    x = synth.normal(24, K)
    planes = gpu.planes(fmt, t)
    gpu.ctx.set_option(BRIK_OPT_GEMV_VARIANT, variant)
    y = gpu.matmul(fmt, x, planes, 1, K, N)
    r, den = oracle_mm(fmt, x, t, 1, K, N)
    check(y, r, den, GEMV_TOL)
    xb = gpu.up(x)
    yb = gpu.up(np.zeros(N, np.float32))
    names = PLANES[fmt]
    job = {"x": xb, "p0": planes[0], "p1": planes[1] if fmt == "q3" else None, "sc": planes[names.index("sc")],
           "mn": planes[names.index("mn")] if "mn" in names else None, "y": yb, "K": K, "N": N}
    plan = gpu.ctx.gemv_plan(fmt, [job])
    plan.run()
    yg = gpu.ctx.download(yb, np.float32, N)
    plan.destroy()
    check(yg, r, den, GEMV_TOL)


# ---- prefill GEMM and small-M -----------------------------------------------------------

@pytest.mark.parametrize("fmt,M,K,N", [
    ("q4", 512, 2560, 9728),     # Qwen3-4B prefill, M = 512
    ("q8", 64, 896, 4864),
    ("q3", 48, 2560, 4096),
    ("q4", 2, 2560, 1024), ("q4", 5, 128, 6), ("q4", 17, 96, 65), ("q8", 3, 64, 130), ("q3", 65, 160, 33),
])
def test_gemm_parity(gpu, fmt, M, K, N):
    """The automatic choice (small M may take the GEMV, see test_small_m_routing) and the forced MFMA
    GEMM, each against the oracle."""
    t = synth.tensor(fmt, 31 + M, N, K)
    x = synth.normal(32 + M, M * K)
    planes = gpu.planes(fmt, t)
    r, den = oracle_mm(fmt, x, t, M, K, N)
    check(gpu.matmul(fmt, x, planes, M, K, N), r, den, REL_TOL)
    gpu.ctx.set_option(BRIK_OPT_PATH, 2)
    check(gpu.matmul(fmt, x, planes, M, K, N), r, den, REL_TOL)


@pytest.mark.parametrize("K", [256, 1024, 1056, 2048, 2080, 2560])
def test_gemm_staged_row_scales(gpu, K):
    """Rows of very different magnitudes through the MFMA path's x staging: one wave per row for
    staged rows of at most 2048 halves (two or four 8-element chunks per lane), one block per row
    above. Each row's power-of-two scale brings its maximum into f16 range, so rows near 1e-30, 1e30
    and past f16's maximum meet the componentwise bound, and a zero row gives exact zeros."""
    M, N = 9, 160
    t = synth.tensor("q4", 40 + K, N, K)
    x = synth.normal(41 + K, M * K).reshape(M, K)
    x[1] *= 1e-30
    x[2] *= 1e30
    x[3] = 0.0
    x[4] *= 3e4
    x[5, ::7] = 0.0
    planes = gpu.planes("q4", t)
    r, den = oracle_mm("q4", x.ravel(), t, M, K, N)
    gpu.ctx.set_option(BRIK_OPT_PATH, 2)
    y = gpu.matmul("q4", x.ravel(), planes, M, K, N)
    check(y, r, den, REL_TOL)
    assert not np.any(y[3])


@pytest.mark.parametrize("M,K", [(262150, 64), (65541, 2560)])
def test_gemm_staging_grid_loops(gpu, M, K):
    """More rows than the x staging grid's 65536 blocks cover: one wave per row (K <= 2048, four rows
    per block: past 262144 rows) and one block per row (past 65536 rows), so its blocks loop over the
    rest; the MFMA path's result against the oracle on every row."""
    N = 8
    t = synth.tensor("q4", 50 + K, N, K)
    x = synth.normal(51 + K, M * K)
    planes = gpu.planes("q4", t)
    r, den = oracle_mm("q4", x, t, M, K, N)
    gpu.ctx.set_option(BRIK_OPT_PATH, 2)
    check(gpu.matmul("q4", x, planes, M, K, N), r, den, REL_TOL)


@pytest.mark.parametrize("M", [2, 3, 4, 8, 15, 16, 32])
@pytest.mark.parametrize("K,N", [(2560, 4096), (2560, 9728), (9728, 2560), (2560, 1024)])
def test_small_m_routing(gpu, M, K, N):
    """Small M at the Qwen3-4B shapes, on whichever path the runtime picks (the GEMV re-streaming W per
    row, or the MFMA GEMM): held to the GEMM's 1e-3 bar, and to the GEMV's 1e-5 when the result is
    that accurate (the GEMV path)."""
    t = synth.q4_tensor(700 + M, N, K)
    x = synth.normal(701 + M, M * K)
    planes = gpu.planes("q4", t)
    y = gpu.matmul("q4", x, planes, M, K, N)
    r, den = oracle_mm("q4", x, t, M, K, N)
    check(y, r, den, REL_TOL)
    gpu.ctx.set_option(BRIK_OPT_PATH, 1)
    check(gpu.matmul("q4", x, planes, M, K, N), r, den, GEMV_TOL)


@pytest.mark.parametrize("K", [96, 1056])
@pytest.mark.parametrize("tile", range(1, BRIK_GEMM_TILES + 1))
@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_gemm_every_tile(gpu, fmt, tile, K):
    # ragged in M and N (partial row and column tiles), 9 column tiles of 128: one full XCD-ordered
    # group of 8 plus the row-major remainder; K = 96 is the shortest pipeline (2 steps), K = 1056 runs
    # 10 steps, which is not a multiple of the W register ring of the prefetching tiles (3 to 5 slots)
    M, N = 130, 1100
    t = synth.tensor(fmt, 35, N, K)
    x = synth.normal(36, M * K)
    planes = gpu.planes(fmt, t)
    gpu.ctx.set_option(BRIK_OPT_GEMM_TILE, tile)
    y = gpu.matmul(fmt, x, planes, M, K, N)
    r, den = oracle_mm(fmt, x, t, M, K, N)
    check(y, r, den, REL_TOL)


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_forced_paths_agree(gpu, fmt):
    M, K, N = 6, 512, 200
    t = synth.tensor(fmt, 41, N, K)
    x = synth.normal(42, M * K)
    planes = gpu.planes(fmt, t)
    r, den = oracle_mm(fmt, x, t, M, K, N)
    gpu.ctx.set_option(BRIK_OPT_PATH, 1)
    check(gpu.matmul(fmt, x, planes, M, K, N), r, den, GEMV_TOL)
    gpu.ctx.set_option(BRIK_OPT_PATH, 2)
    check(gpu.matmul(fmt, x[:K], planes, 1, K, N), r[:1], den[:1], REL_TOL)


# ---- MoE expert-grouped q4 (64 experts) ------------------------------------------------------

@pytest.mark.parametrize("which", ["gate", "down"])
def test_moe_e64(gpu, which):
    T, H, E, F, TOPK = 256, 2048, 64, 768, 8
    K, N = (H, F) if which == "gate" else (F, H)
    rows, row_off = synth.moe_routing(77, T, E, TOPK)
    R = rows.size
    assert R == T * TOPK and np.diff(row_off).min() >= 0
    t = synth.q4_tensor(78 if which == "gate" else 79, E * N, K)
    if which == "gate":
        x = synth.normal(80, T * H).reshape(T, H)[rows]        # gathered token rows
    else:
        x = synth.normal(81, R * K).reshape(R, K)
    planes = gpu.planes("q4", t)
    xb, rb = gpu.up(np.ascontiguousarray(x)), gpu.up(row_off)
    yb = gpu.up(np.zeros(R * N, np.float32))
    gpu.ctx.moe_matmul_t_q4(xb, rb, *planes, yb, E, R, K, N)
    y = gpu.ctx.download(yb, np.float32, R * N)
    r = O.moe_matmul_t_q4(x, row_off, t["nib"], t["sc"], t["mn"], E, K, N)
    ra, den = moe_oracle_abs(x, row_off, t, E, K, N)
    assert np.array_equal(ra, r)
    check(y, r, den, REL_TOL)


@pytest.mark.parametrize("tile", range(0, BRIK_GEMM_TILES + 1))
def test_moe_every_tile(gpu, tile):
    """Every tile on an expert-grouped launch with uneven experts (one of 0 rows, some above 64) and a
    K of 24 steps (the prefetching tiles' rings wrap several times)."""
    E, K, N = 12, 1536 * 2, 160
    row_off = np.array([0, 3, 3, 40, 110, 111, 150, 230, 250, 251, 300, 330, 332], np.int32)
    R = int(row_off[-1])
    t = synth.q4_tensor(92, E * N, K)
    x = synth.normal(93, R * K)
    planes = gpu.planes("q4", t)
    gpu.ctx.set_option(BRIK_OPT_GEMM_TILE, tile)
    xb, rb = gpu.up(x), gpu.up(row_off)
    yb = gpu.up(np.full(R * N, np.nan, np.float32))
    gpu.ctx.moe_matmul_t_q4(xb, rb, *planes, yb, E, R, K, N)
    y = gpu.ctx.download(yb, np.float32, R * N)
    r, den = moe_oracle_abs(x, row_off, t, E, K, N)
    check(y, r, den, REL_TOL)


@pytest.mark.parametrize("tile", range(0, BRIK_GEMM_TILES + 1))
def test_moe_empty_experts(gpu, tile):
    gpu.ctx.set_option(BRIK_OPT_GEMM_TILE, tile)
    E, K, N = 6, 64, 40
    row_off = np.array([0, 0, 5, 5, 5, 9, 9], np.int32)
    t = synth.q4_tensor(90, E * N, K)
    x = synth.normal(91, 9 * K)
    planes = gpu.planes("q4", t)
    xb, rb = gpu.up(x), gpu.up(row_off)
    yb = gpu.up(np.full(9 * N, np.nan, np.float32))
    gpu.ctx.moe_matmul_t_q4(xb, rb, *planes, yb, E, 9, K, N)
    y = gpu.ctx.download(yb, np.float32, 9 * N)
    r, den = moe_oracle_abs(x, row_off, t, E, K, N)
    check(y, r, den, REL_TOL)


# ---- edge cases and error behaviour --------------------------------------------------------

@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_empty_and_degenerate_shapes(gpu, fmt):
    K, N = 64, 10
    t = synth.tensor(fmt, 50, N, K)
    planes = gpu.planes(fmt, t)
    x = synth.normal(51, 3 * K)
    # M == 0 and N == 0 are no-ops: y untouched
    yb = gpu.up(np.full(30, 7.0, np.float32))
    fn = {"q8": gpu.ctx.matmul_t_q8, "q4": gpu.ctx.matmul_t_q4, "q3": gpu.ctx.matmul_t_q3}[fmt]
    xb = gpu.up(x)
    fn(xb, *planes, yb, 0, K, N)
    fn(xb, *planes, yb, 3, K, 0)
    assert np.all(gpu.ctx.download(yb, np.float32, 30) == 7.0)
    # K == 0 writes zeros
    fn(xb, *planes, yb, 3, 0, N)
    assert np.all(gpu.ctx.download(yb, np.float32, 30) == 0.0)
    # ragged N and M around the tile sizes
    for M, N2 in ((1, 1), (1, 17), (2, 1), (3, 65), (64, 64), (65, 63)):
        t2 = synth.tensor(fmt, 52 + M + N2, N2, 96)
        x2 = synth.normal(53, M * 96)
        y = gpu.matmul(fmt, x2, gpu.planes(fmt, t2), M, 96, N2)
        r, den = oracle_mm(fmt, x2, t2, M, 96, N2)
        check(y, r, den, REL_TOL)


def test_invalid_arguments(gpu):
    K, N = 64, 8
    t = synth.q4_tensor(60, N, K)
    planes = gpu.planes("q4", t)
    xb = gpu.up(synth.normal(61, 2 * K))
    yb = gpu.up(np.zeros(2 * N, np.float32))
    with pytest.raises(BrikError) as e:
        gpu.ctx.matmul_t_q4(xb, *planes, yb, 2, 48, N)          # K % 32 != 0
    assert e.value.code == BRIK_EINVAL
    with pytest.raises(BrikError) as e:
        gpu.ctx.matmul_t_q4(xb, *planes, yb, -1, K, N)
    assert e.value.code == BRIK_EINVAL
    with pytest.raises(BrikError) as e:
        gpu.ctx.matmul_t_q4(None, *planes, yb, 2, K, N)
    assert e.value.code == BRIK_EINVAL
    with pytest.raises(BrikError) as e:
        gpu.ctx.matmul_t_q4(xb.ptr + 4, *planes, yb, 1, K, N)     # misaligned activation
    assert e.value.code == BRIK_EALIGN
    with pytest.raises(BrikError) as e:
        gpu.ctx.matmul_t_q4(xb, planes[0] + 8, planes[1], planes[2], yb, 1, K, N)   # misaligned nibbles
    assert e.value.code == BRIK_EALIGN
    with pytest.raises(BrikError):
        gpu.ctx.set_option(BRIK_OPT_GEMV_VARIANT, BRIK_GEMV_VARIANTS + 1)


def test_bit_flip_is_detected(gpu):
    """Negative control: corrupting one nibble byte must break parity (the check is not vacuous)."""
    K, N = 256, 64
    t = synth.q4_tensor(70, N, K)
    x = synth.normal(71, K)
    bad = dict(t, nib=t["nib"].copy())
    bad["nib"][5 * K // 2 + 3] ^= 0x11
    y = gpu.matmul("q4", x, gpu.planes("q4", bad), 1, K, N)
    r, _ = oracle_mm("q4", x, t, 1, K, N)
    assert np.abs(y.ravel() - r.ravel()).max() > 0
    assert np.argmax(np.abs(y.ravel() - r.ravel())) == 5


# ---- grouped plans and non-finite activations -----------------------------------------------

def test_grouped_plan_layer_set(gpu):
    """A plan over a small 'layer set': jobs of different K and N sharing x buffers, like the
    q/k/v + gate/up + down projections of one decoder layer."""
    shapes = [(256, 384), (256, 96), (256, 96), (256, 700), (704, 256)]
    xs = {256: synth.normal(301, 256), 704: synth.normal(302, 704)}
    xb = {k: gpu.up(v) for k, v in xs.items()}
    jobs, refs = [], []
    for i, (K, N) in enumerate(shapes):
        t = synth.q4_tensor(310 + i, N, K)
        nib, sc, mn = gpu.planes("q4", t)
        yb = gpu.up(np.zeros(N, np.float32))
        jobs.append({"x": xb[K], "p0": nib, "sc": sc, "mn": mn, "y": yb, "K": K, "N": N})
        refs.append(oracle_mm("q4", xs[K], t, 1, K, N))
    plan = gpu.ctx.gemv_plan("q4", jobs)
    for _ in range(2):                      # plans are reusable
        plan.run()
    for j, (r, den) in zip(jobs, refs):
        y = gpu.ctx.download(j["y"], np.float32, j["N"])
        check(y, r, den, GEMV_TOL)
    plan.destroy()


def test_grouped_plan_rejects_bad_jobs(gpu):
    t = synth.q4_tensor(320, 8, 64)
    nib, sc, mn = gpu.planes("q4", t)
    xb, yb = gpu.up(synth.normal(321, 64)), gpu.up(np.zeros(8, np.float32))
    good = {"x": xb, "p0": nib, "sc": sc, "mn": mn, "y": yb, "K": 64, "N": 8}
    for bad in (dict(good, K=48), dict(good, N=0), dict(good, K=0), dict(good, mn=None), dict(good, x=xb.ptr + 4)):
        with pytest.raises(BrikError):
            gpu.ctx.gemv_plan("q4", [good, bad])


@pytest.mark.parametrize("fmt", ["q4", "q3"])
def test_staged_single_row(gpu, fmt):
    """A single M = 1 matrix of at least 24576 rows stages x once per call (one staging block) and its
    blocks copy the image: a finite row matches the oracle, and a row holding Inf takes the exact path
    through the staged flag."""
    K, N = 256, 24583
    t = synth.tensor(fmt, 340, N, K)
    planes = gpu.planes(fmt, t)
    for bad in (False, True):
        x = synth.normal(341, K)
        if bad:
            x[100] = -np.inf
        y2 = gpu.matmul(fmt, x, planes, 1, K, N)
        r, den = oracle_mm(fmt, x, t, 1, K, N)
        if bad:
            y, r0 = y2[0], r.reshape(-1)
            inf = np.isinf(y)
            assert np.array_equal(np.isnan(y), np.isnan(r0)) and np.array_equal(inf, np.isinf(r0))
            assert np.array_equal(np.sign(y[inf]), np.sign(r0[inf]))
        else:
            check(y2, r, den, GEMV_TOL)


@pytest.mark.parametrize("variant", range(0, BRIK_GEMV_VARIANTS + 1))
@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_non_finite_activation_follows_f32_semantics(gpu, fmt, variant):
    """Inf/NaN in x cannot be held in the integer limbs; such a row takes the exact f32 path and
    yields the same Inf/NaN pattern as the f64 reference sum, under every tiling variant (including
    those with fewer than 16 rows per block iteration); N = 40 is not a multiple of any row set."""
    K, N = 256, 40
    t = synth.tensor(fmt, 330, N, K)
    planes = gpu.planes(fmt, t)
    x = synth.normal(331, 3 * K).reshape(3, K)
    x[0, 17] = np.inf
    x[1, 200] = np.nan
    gpu.ctx.set_option(BRIK_OPT_PATH, 1)        # GEMV for every row
    gpu.ctx.set_option(BRIK_OPT_GEMV_VARIANT, variant)
    y = gpu.matmul(fmt, x, planes, 3, K, N)
    r, den = oracle_mm(fmt, x, t, 3, K, N)
    for row in (0, 1):
        assert np.array_equal(np.isnan(y[row]), np.isnan(r[row]))
        assert np.array_equal(np.isposinf(y[row]), np.isposinf(r[row]))
        assert np.array_equal(np.isneginf(y[row]), np.isneginf(r[row]))
    check(y[2], r[2], den[2], GEMV_TOL)          # the finite row is unaffected
