"""GPU parity of the exact kernels behind the decode headline and of every GEMV variant at the
Qwen3-4B row lengths, through the C ABI, against the oracle (the reference's own q4 gate compares the
kernel with the CPU matmul on the same inputs, kernels.ts:2325-2340).

The headline step is a grouped plan over whole Qwen3-4B layer sets: at least 24576 rows, so the plan
stages every distinct input row once (brik_gemv_stage_q4) and its blocks copy the staged image; the
automatic variant for that many rows streams whole K = 2560 rows per step (16 lanes x 5 groups = 80
groups = one row), so K = 2560 runs the EVEN branch (every group of every step exists) and K = 9728
(304 groups) the clamped one. The variant tests run every tiling variant at K = 2560 and K = 9728,
single-matrix and grouped, with x staged in-block and pre-staged, so both branches of every variant
meet both staging forms.

Bar: the GEMV's 1e-5, normwise (max|y - r| / max|r|) and componentwise (|y - r| <= 1e-5 sum|x w|).
"""
import functools

import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth
from brimkern_amd.capi import BRIK_OPT_GEMV_VARIANT, BRIK_GEMV_VARIANTS
from helpers import Gpu, PLANES, normwise_rel, componentwise_ok

pytestmark = pytest.mark.gpu
TOL = 1e-5
QWEN3_4B = [("q", 2560, 4096), ("k", 2560, 1024), ("v", 2560, 1024),
            ("gate", 2560, 9728), ("up", 2560, 9728), ("down", 9728, 2560)]
PRESTAGE_ROWS = 24576           # plans (and single M = 1 q4 / q3 matrices) of this many rows pre-stage x
WHOLE_ROW_VARIANT = 8           # 1 + index of the 16-lane, 2-row, 5-group variant


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    ctx.set_option(BRIK_OPT_GEMV_VARIANT, 0)
    g.free()


def check(y, r, den):
    rel = normwise_rel(y, r)
    assert rel <= TOL, f"normwise rel {rel:.3e}"
    assert componentwise_ok(y, r, den, TOL), "componentwise bound violated"


def oracle_mm(fmt, x, t):
    fn = getattr(O, f"matmul_t_{fmt}")
    r, den = fn(x, *[t[k] for k in PLANES[fmt]], 1, t["K"], t["N"], absden=True)
    return r.ravel(), den.ravel()


@functools.lru_cache(maxsize=None)
def case(fmt, K, N, seed):
    """A seeded tensor, an input row and the oracle's result (cached: each variant reuses them)."""
    t = synth.tensor(fmt, seed, N, K)
    x = synth.normal(seed + 1, K)
    r, den = oracle_mm(fmt, x, t)
    return t, x, r, den


def job_of(fmt, planes, xb, yb, K, N):
    names = PLANES[fmt]
    return {"x": xb, "p0": planes[0], "p1": planes[1] if fmt == "q3" else None, "sc": planes[names.index("sc")],
            "mn": planes[names.index("mn")] if "mn" in names else None, "y": yb, "K": K, "N": N}


@pytest.mark.parametrize("variant", [0, WHOLE_ROW_VARIANT], ids=["auto", "whole_row"])
def test_headline_plan_qwen3_4b_layers(gpu, variant):
    """The bench's step at two layers: 12 matrices (K = 2560 and 9728, N from 1024 to 9728) sharing two
    input rows, one plan, pre-staged; every job against the oracle, on two runs of the plan."""
    layers = 2
    xs = {2560: synth.normal(101, 2560), 9728: synth.normal(102, 9728)}
    xb = {k: gpu.up(v) for k, v in xs.items()}
    jobs, expect = [], []
    for layer in range(layers):
        for si, (name, K, N) in enumerate(QWEN3_4B):
            t = synth.q4_tensor(200 + 10 * layer + si, N, K)
            yb = gpu.up(np.full(N, np.nan, np.float32))
            jobs.append(job_of("q4", gpu.planes("q4", t), xb[K], yb, K, N))
            expect.append(oracle_mm("q4", xs[K], t))
    assert sum(j["N"] for j in jobs) >= PRESTAGE_ROWS
    gpu.ctx.set_option(BRIK_OPT_GEMV_VARIANT, variant)
    plan = gpu.ctx.gemv_plan("q4", jobs)
    try:
        for _ in range(2):
            plan.run()
            for j, (r, den) in zip(jobs, expect):
                check(gpu.ctx.download(j["y"], np.float32, j["N"]), r, den)
                gpu.ctx.h2d(j["y"], np.full(j["N"], np.nan, np.float32))
    finally:
        plan.destroy()


@pytest.mark.parametrize("K", [2560, 9728])
@pytest.mark.parametrize("variant", range(1, BRIK_GEMV_VARIANTS + 1))
@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_variant_in_block_staging(gpu, fmt, variant, K):
    """Every variant at K = 2560 and 9728 with x staged inside each block: one matrix (M = 1) and a
    one-job plan, N = 777 (ragged against every row set)."""
    N = 777
    t, x, r, den = case(fmt, K, N, 500 + K)
    planes = gpu.planes(fmt, t)
    gpu.ctx.set_option(BRIK_OPT_GEMV_VARIANT, variant)
    check(gpu.matmul(fmt, x, planes, 1, K, N), r, den)
    xb, yb = gpu.up(x), gpu.up(np.full(N, np.nan, np.float32))
    plan = gpu.ctx.gemv_plan(fmt, [job_of(fmt, planes, xb, yb, K, N)])
    plan.run()
    y = gpu.ctx.download(yb, np.float32, N)
    plan.destroy()
    check(y, r, den)


@pytest.mark.parametrize("K", [2560, 9728])
@pytest.mark.parametrize("variant", range(1, BRIK_GEMV_VARIANTS + 1))
@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_variant_prestaged(gpu, fmt, variant, K):
    """Every variant at K = 2560 and 9728 with x pre-staged: a one-job plan of 24583 rows (the plan's
    staging launch) and, for q4 / q3, the same matrix as one M = 1 call (the single-row staging
    launch; q8 stages in-block at every size)."""
    N = PRESTAGE_ROWS + 7
    t, x, r, den = case(fmt, K, N, 600 + K)
    planes = gpu.planes(fmt, t)
    gpu.ctx.set_option(BRIK_OPT_GEMV_VARIANT, variant)
    xb, yb = gpu.up(x), gpu.up(np.full(N, np.nan, np.float32))
    plan = gpu.ctx.gemv_plan(fmt, [job_of(fmt, planes, xb, yb, K, N)])
    plan.run()
    y = gpu.ctx.download(yb, np.float32, N)
    plan.destroy()
    check(y, r, den)
    if fmt != "q8":
        check(gpu.matmul(fmt, x, planes, 1, K, N), r, den)


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_prestaged_norm_degenerate_factor(gpu, fmt):
    """A zero row with eps = 0 gives the RMSNorm factor 1 / sqrt(0) = inf and every output NaN, as the
    reference's x * inv * g does (rmsnormCpu, kernels.ts:3395-3404); in a pre-staged plan the staging
    launch (16 waves) computes that factor and must send the job to the per-element path, while a
    second input of the same plan with a finite factor stays on the fast path."""
    K, N = 512, PRESTAGE_ROWS // 2 + 5
    t = synth.tensor(fmt, 660, N, K)
    w = synth.normal(661, K) * 0.5 + 1
    x2 = synth.normal(662, K)
    zero = np.zeros(K, np.float32)
    zb, xb2, wb = gpu.up(zero), gpu.up(x2), gpu.up(w)
    y1, y2 = gpu.up(np.zeros(N, np.float32)), gpu.up(np.zeros(N, np.float32))
    planes = gpu.planes(fmt, t)
    jobs = [dict(job_of(fmt, planes, zb, y1, K, N), norm_w=wb, eps=0.0),
            dict(job_of(fmt, planes, xb2, y2, K, N), norm_w=wb, eps=0.0)]
    assert 2 * N >= PRESTAGE_ROWS
    plan = gpu.ctx.gemv_plan(fmt, jobs)
    plan.run()
    a, b = gpu.ctx.download(y1, np.float32, N), gpu.ctx.download(y2, np.float32, N)
    plan.destroy()
    with np.errstate(all="ignore"):
        r2, den2 = oracle_mm(fmt, O.rmsnorm(x2, w, 1, K, 0.0, False), t)
    assert np.isnan(a).all()
    check(b, r2, den2)
