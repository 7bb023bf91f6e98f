"""GPU parity of the fused GEMV plan jobs (brik_gemv_job_ex): RMSNorm / SwiGLU / GeGLU input
transforms and residual adds, through the C ABI, against the oracle (the reference's CPU layer ops,
kernels.ts:3395-3404, 3498-3530, followed by the oracle matmul).

The chain test runs the matmul side of one Qwen3-4B decoder layer as four plans, the way
recordLayerKV records it (kernels.ts:1701-1741): q/k/v on rmsnorm(x), wo + residual, gate/up on
rmsnorm(h), down on swiglu(gate, up) + residual. Attention is outside this library; its output is
a seeded vector here.
"""
import numpy as np
import pytest

import oracle as O
from brimkern_amd import synth
from brimkern_amd.capi import BrikError, BRIK_EINVAL, BRIK_EALIGN
from helpers import Gpu, PLANES, normwise_rel

pytestmark = pytest.mark.gpu

TOL = 1e-5   # the GEMV bar (24-bit staged x, f32 accumulation); the transforms run in f32 on the GPU


@pytest.fixture()
def gpu(ctx):
    g = Gpu(ctx)
    yield g
    g.free()


def oracle_mm(fmt, x, t, K, N):
    return getattr(O, f"matmul_t_{fmt}")(np.asarray(x, np.float32), *[t[p] for p in PLANES[fmt]], 1, K, N).ravel()


def job(gpu, fmt, t, xb, yb, K, N, **fuse):
    planes = gpu.planes(fmt, t)
    names = {"q8": ("p0", "sc"), "q4": ("p0", "sc", "mn"), "q3": ("p0", "p1", "sc", "mn")}[fmt]
    j = dict(zip(names, planes), x=xb, y=yb, K=K, N=N)
    j.update(fuse)
    return j


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
@pytest.mark.parametrize("case", ["norm", "norm_one_plus", "swiglu", "geglu", "res", "all"])
def test_fused_job(gpu, fmt, case):
    K, N = 1024, 700
    t = synth.tensor(fmt, 50, N, K)
    x = synth.normal(51, K) * 3
    gate = synth.normal(52, K) * 2
    w = synth.normal(53, K) * 0.5 + 1
    res = synth.normal(54, N)
    xb, gb, wb, rb = gpu.up(x), gpu.up(gate), gpu.up(w), gpu.up(res)
    yb = gpu.up(np.zeros(N, np.float32))
    fuse, xin, radd = {}, x, np.zeros(N, np.float32)
    if case in ("swiglu", "geglu", "all"):
        fuse.update(gate=gb, gelu=case == "geglu")
        xin = (O.geglu if case == "geglu" else O.swiglu)(gate, xin)
    if case in ("norm", "norm_one_plus", "all"):
        one_plus = case == "norm_one_plus"
        fuse.update(norm_w=wb, eps=1e-6, one_plus=one_plus)
        xin = O.rmsnorm(xin, w, 1, K, 1e-6, one_plus)
    if case in ("res", "all"):
        fuse.update(res=rb)
        radd = res
    plan = gpu.ctx.gemv_plan(fmt, [job(gpu, fmt, t, xb, yb, K, N, **fuse)])
    plan.run()
    y = gpu.ctx.download(yb, np.float32, N)
    plan.destroy()
    r = oracle_mm(fmt, xin, t, K, N) + radd
    assert normwise_rel(y, r) <= TOL


def test_residual_in_place(gpu):
    # y = y + x . W^T (res aliasing y), as the layer's h += down
    K, N = 512, 300
    t = synth.tensor("q4", 60, N, K)
    x = synth.normal(61, K)
    y0 = synth.normal(62, N)
    xb, yb = gpu.up(x), gpu.up(y0)
    plan = gpu.ctx.gemv_plan("q4", [job(gpu, "q4", t, xb, yb, K, N, res=yb)])
    plan.run()
    plan.run()                                   # twice: y0 + 2 x . W^T
    y = gpu.ctx.download(yb, np.float32, N)
    plan.destroy()
    assert normwise_rel(y, y0 + 2 * oracle_mm("q4", x, t, K, N)) <= TOL


def test_fused_rejects_bad_flags_and_alignment(gpu):
    K, N = 256, 64
    t = synth.tensor("q4", 70, N, K)
    xb, yb = gpu.up(synth.normal(71, K)), gpu.up(np.zeros(N, np.float32))
    wb = gpu.up(np.ones(K + 4, np.float32))
    j = job(gpu, "q4", t, xb, yb, K, N, norm_w=wb.offset(4))
    with pytest.raises(BrikError) as e:
        gpu.ctx.gemv_plan("q4", [j])
    assert e.value.code == BRIK_EALIGN


def test_decode_layer_chain_qwen3_4b(gpu):
    d, qd, kvd, ffn = 2560, 4096, 1024, 9728
    eps = 1e-6
    W = {n: synth.tensor("q4", 80 + i, N, K) for i, (n, K, N) in enumerate(
        [("q", d, qd), ("k", d, kvd), ("v", d, kvd), ("o", qd, d), ("gate", d, ffn), ("up", d, ffn),
         ("down", ffn, d)])}
    x = synth.normal(90, d) * 2
    attn = synth.normal(91, qd)                  # stands in for the attention output
    an, fn = synth.normal(92, d) * 0.2 + 1, synth.normal(93, d) * 0.2 + 1
    xb, attnb, anb, fnb = gpu.up(x), gpu.up(attn), gpu.up(an), gpu.up(fn)
    out = {n: gpu.up(np.zeros(N, np.float32)) for n, N in
           [("q", qd), ("k", kvd), ("v", kvd), ("h", d), ("gate", ffn), ("up", ffn), ("y", d)]}
    K_of = {"q": d, "k": d, "v": d, "o": qd, "gate": d, "up": d, "down": ffn}
    N_of = {"q": qd, "k": kvd, "v": kvd, "o": d, "gate": ffn, "up": ffn, "down": d}
    plans = [
        gpu.ctx.gemv_plan("q4", [job(gpu, "q4", W[n], xb, out[n], d, N_of[n], norm_w=anb, eps=eps)
                                 for n in ("q", "k", "v")]),
        gpu.ctx.gemv_plan("q4", [job(gpu, "q4", W["o"], attnb, out["h"], qd, d, res=xb)]),
        gpu.ctx.gemv_plan("q4", [job(gpu, "q4", W[n], out["h"], out[n], d, ffn, norm_w=fnb, eps=eps)
                                 for n in ("gate", "up")]),
        gpu.ctx.gemv_plan("q4", [job(gpu, "q4", W["down"], out["up"], out["y"], ffn, d, gate=out["gate"],
                                     res=out["h"])]),
    ]
    for p in plans:
        p.run()
    got = {n: gpu.ctx.download(out[n], np.float32, out[n].nbytes // 4) for n in out}
    for p in plans:
        p.destroy()
    # oracle chain (kernels.ts:3508-3530 without attention)
    n1 = O.rmsnorm(x, an, 1, d, eps)
    for n in ("q", "k", "v"):
        assert normwise_rel(got[n], oracle_mm("q4", n1, W[n], d, N_of[n])) <= TOL
    h = (x + oracle_mm("q4", attn, W["o"], qd, d)).astype(np.float32)
    assert normwise_rel(got["h"], h) <= TOL
    n2 = O.rmsnorm(got["h"], fn, 1, d, eps)     # from the GPU's h, so each stage is checked on its own
    gate = oracle_mm("q4", n2, W["gate"], d, ffn)
    up = oracle_mm("q4", n2, W["up"], d, ffn)
    assert normwise_rel(got["gate"], gate) <= TOL and normwise_rel(got["up"], up) <= TOL
    g = O.swiglu(got["gate"], got["up"])
    y = (got["h"] + oracle_mm("q4", g, W["down"], ffn, d)).astype(np.float32)
    assert normwise_rel(got["y"], y) <= TOL


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_prestaged_large_plan(gpu, fmt):
    """A plan of at least 24576 rows stages every distinct input row once per run (a staging launch)
    and its blocks copy the staged image instead of staging it themselves. Jobs here share one input
    (same x, same RMSNorm: staged once), use another with SwiGLU + residual, and a third input holds
    Inf, so its job must take the exact path through the staged flag."""
    cases = [  # (K, N, input id, fuse)
        (1024, 12000, "a", "norm"), (1024, 8000, "a", "norm"), (512, 6000, "b", "swiglu_res"), (256, 1000, "c", "plain"),
    ]
    xs = {"a": synth.normal(71, 1024) * 2, "b": synth.normal(72, 512), "c": synth.normal(73, 256)}
    xs["c"][37] = np.inf
    gate = synth.normal(74, 512)
    w = synth.normal(75, 1024) * 0.3 + 1
    xb = {k: gpu.up(v) for k, v in xs.items()}
    gb, wb = gpu.up(gate), gpu.up(w)
    jobs, expect, outs = [], [], []
    for i, (K, N, xi, fuse) in enumerate(cases):
        t = synth.tensor(fmt, 80 + i, N, K)
        yb = gpu.up(np.zeros(N, np.float32))
        f, xin, radd = {}, xs[xi], np.zeros(N, np.float32)
        if fuse == "norm":
            f.update(norm_w=wb, eps=1e-6)
            xin = O.rmsnorm(xin, w, 1, K, 1e-6, False)
        elif fuse == "swiglu_res":
            res = synth.normal(76, N)
            f.update(gate=gb, res=gpu.up(res))
            xin, radd = O.swiglu(gate, xin), res
        jobs.append(job(gpu, fmt, t, xb[xi], yb, K, N, **f))
        expect.append(oracle_mm(fmt, xin, t, K, N) + radd)
        outs.append((yb, N))
    assert sum(N for _, N, _, _ in cases) >= 24576
    plan = gpu.ctx.gemv_plan(fmt, jobs)
    for rep in range(2):
        plan.run()
        for (yb, N), r, (_, _, xi, _) in zip(outs, expect, cases):
            y = gpu.ctx.download(yb, np.float32, N)
            if xi == "c":
                assert np.array_equal(np.isnan(y), np.isnan(r))
                assert np.array_equal(np.isposinf(y), np.isposinf(r)) and np.array_equal(np.isneginf(y), np.isneginf(r))
                fin = np.isfinite(r)
                assert np.array_equal(y[fin], y[fin]) and np.allclose(y[fin], r[fin], rtol=1e-5, atol=0)
            else:
                assert normwise_rel(y, r) <= TOL
    plan.destroy()


@pytest.mark.parametrize("fmt", ["q8", "q4", "q3"])
def test_norm_degenerate_factor(gpu, fmt):
    """A zero row with eps = 0 has the RMSNorm factor 1 / sqrt(0) = inf, and the reference's
    x * inv * g is 0 * inf = NaN in every element (rmsnormCpu, kernels.ts:3395-3404): every output
    is NaN. The staged image leaves the factor out and scales each row's result by it, so such a
    factor has to take the per-element path instead. A second job of the same plan, with a finite
    factor, stays on the fast path."""
    K, N = 512, 300
    t = synth.tensor(fmt, 60, N, K)
    w = synth.normal(61, K) * 0.5 + 1
    x2 = synth.normal(62, K)
    zero = np.zeros(K, np.float32)
    zb, xb2, wb = gpu.up(zero), gpu.up(x2), gpu.up(w)
    y1, y2 = gpu.up(np.zeros(N, np.float32)), gpu.up(np.zeros(N, np.float32))
    plan = gpu.ctx.gemv_plan(fmt, [job(gpu, fmt, t, zb, y1, K, N, norm_w=wb, eps=0.0),
                                   job(gpu, fmt, t, xb2, y2, K, N, norm_w=wb, eps=0.0)])
    plan.run()
    a, b = gpu.ctx.download(y1, np.float32, N), gpu.ctx.download(y2, np.float32, N)
    plan.destroy()
    with np.errstate(all="ignore"):
        r1 = oracle_mm(fmt, O.rmsnorm(zero, w, 1, K, 0.0, False), t, K, N)
        r2 = oracle_mm(fmt, O.rmsnorm(x2, w, 1, K, 0.0, False), t, K, N)
    assert np.isnan(r1).all() and np.isnan(a).all()
    assert normwise_rel(b, r2) <= TOL
